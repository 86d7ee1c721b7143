"""The C ABI library loads and exports every entry point declared in
include/flashtrie_amd.h; argument errors are reported without a GPU."""

import ctypes
import os
import re

import numpy as np
import pytest

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


def _create(lib, img):
    lib.ft_create.restype = ctypes.c_int
    lib.ft_create.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                              ctypes.c_void_p]
    lib.ft_last_error.restype = ctypes.c_char_p
    lib.ft_destroy.argtypes = [ctypes.c_void_p]
    out = ctypes.c_void_p()
    rc = lib.ft_create(img.ctypes.data, img.size, 0, ctypes.byref(out))
    if rc == 0:  # a GPU host: the valid image made a context
        lib.ft_destroy(out)
    return rc, lib.ft_last_error().decode()


def test_create_rejects_corrupt_images_before_any_device_call(ft):
    # ft_create validates the whole blob on the host: a corrupt node record,
    # parent link or tail offset is FT_E_IMAGE (-7), never a device read out
    # of bounds.  Here (no GPU) a valid image gets as far as the device
    # lookup (FT_E_DEVICE, -8); on a GPU host it makes a context.
    lib = ctypes.CDLL(LIB)
    t = ft.Trie()
    t.build([[1, 2, 3, 4], [1, 2, 3, 5], [7], [8, 9], [8, 10, 11]])
    img = np.array(t.image(), dtype=np.uint8)
    hdr = np.frombuffer(img[:64].tobytes(), dtype="<u8", count=8)
    n, ro, po_, to = int(hdr[1]), int(hdr[4]), int(hdr[5]), int(hdr[6])
    rc, msg = _create(lib, img)
    assert rc in (0, -8), (rc, msg)

    def rec_word(node, field):  # u32 view index of a record field
        return (ro + 16 * node) // 4 + field

    def corrupt(word_index, value):
        bad = img.copy()
        bad.view(np.uint32)[word_index] = value
        return bad

    recs = img[ro:ro + (n + 1) * 16].view(np.uint32).reshape(-1, 4)
    link = next(v for v in range(n) if recs[v, 3] & 0x40000000)
    cases = [
        (corrupt(rec_word(1, 0), n + 5), "breadth first"),       # child_begin past N
        (corrupt(rec_word(0, 0), 0), "start at id 1"),          # root's children
        (corrupt(rec_word(n, 0), n - 1), "sentinel"),
        (corrupt(po_ // 4 + 2, 0xFFFF), "inconsistent"),         # parent link
        (corrupt(rec_word(link, 2), 1 << 30), "tail"),           # tail offset
        (corrupt(rec_word(2, 1), 0x7FFFFFFF), "inconsistent"),   # token id
        (corrupt(rec_word(2, 3), int(recs[2, 3]) ^ 0x80000000), "num_keys"),
    ]
    for bad, what in cases:
        rc, msg = _create(lib, bad)
        assert rc == -7, (what, rc, msg)
        assert what in msg, (what, msg)


# ---- the C ABI driven from ctypes, as the integration guide shows ---------

from cabi import Request, Result  # noqa: E402


def test_struct_layouts_match_the_header(tmp_path):
    # the ctypes mirrors against what a C compiler makes of the header
    # (sizeof and every field offset of ft_request and ft_result)
    import subprocess
    fields = {"ft_request": [f for f, _ in Request._fields_],
              "ft_result": [f for f, _ in Result._fields_]}
    src = ['#include <stddef.h>', '#include <stdio.h>', '#include "flashtrie_amd.h"',
           "int main(void) {"]
    for st, fs in fields.items():
        src.append(f'  printf("{st} %zu\\n", sizeof({st}));')
        for f in fs:
            src.append(f'  printf("{st}.{f} %zu\\n", offsetof({st}, {f}));')
    src.append("  return 0; }")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src) + "\n")
    exe = tmp_path / "layout"
    subprocess.check_call(["gcc", "-I" + os.path.join(ROOT, "include"), str(c), "-o", str(exe)])
    out = dict(l.split() for l in subprocess.check_output([str(exe)], text=True).splitlines())
    for st, cls in (("ft_request", Request), ("ft_result", Result)):
        assert int(out[st]) == ctypes.sizeof(cls), st
        for f in fields[st]:
            assert int(out[f"{st}.{f}"]) == getattr(cls, f).offset, (st, f)
