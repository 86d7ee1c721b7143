"""The C ABI library loads and exports every entry point declared in
include/flashtrie_amd.h; argument errors are reported without a GPU."""

import ctypes
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashtrie_amd.h")
LIB = os.path.join(ROOT, "flash-trie_amd", "libflashtrie_amd.so")


def declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"\b(ft_[a-z_]+)\s*\(", src)))


def test_exports_every_declared_symbol(ft):
    lib = ctypes.CDLL(LIB)
    names = declared()
    assert "ft_search" in names and "ft_create" in names
    for n in names:
        assert hasattr(lib, n), n


def test_argument_errors_without_device(ft):
    lib = ctypes.CDLL(LIB)
    lib.ft_create.restype = ctypes.c_int
    lib.ft_create.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                              ctypes.c_void_p]
    lib.ft_strerror.restype = ctypes.c_char_p
    lib.ft_last_error.restype = ctypes.c_char_p
    out = ctypes.c_void_p()
    assert lib.ft_create(None, 0, 0, ctypes.byref(out)) == -1       # FT_E_ARG
    bad = np.zeros(256, dtype=np.uint8)
    assert lib.ft_create(bad.ctypes.data, bad.size, 0, ctypes.byref(out)) == -7
    assert b"magic" in lib.ft_last_error()
    assert lib.ft_strerror(-4) == b"request exceeds the reserved workspace"
    lib.ft_reserve.restype = ctypes.c_int
    assert lib.ft_reserve(None, 1, 1, 1, 1, 1, 1) == -1
    lib.ft_stage.restype = ctypes.c_int
    assert lib.ft_stage(None, None, 0) == -1
