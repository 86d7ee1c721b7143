"""ctypes mirrors of include/flashtrie_amd.h (ft_request, ft_result) and
helpers that drive the C ABI library the way another host language would."""

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "flash-trie_amd", "libflashtrie_amd.so")

U32P = ctypes.POINTER(ctypes.c_uint32)
F32P = ctypes.POINTER(ctypes.c_float)
F64P = ctypes.POINTER(ctypes.c_double)


class Request(ctypes.Structure):
    _fields_ = [("beams", U32P), ("num_beams", ctypes.c_uint32),
                ("num_steps", ctypes.c_uint32), ("topk", ctypes.c_uint32),
                ("topk_id", U32P), ("topk_logp", F32P),
                ("topk_id_rows", ctypes.c_void_p), ("topk_logp_rows", ctypes.c_void_p),
                ("token_logp_threshold", ctypes.c_float),
                ("sent_logp_threshold", ctypes.c_double),
                ("length_norm", ctypes.c_double), ("early_exit", ctypes.c_int)]


class Result(ctypes.Structure):
    _fields_ = [("capacity", ctypes.c_uint32), ("token_stride", ctypes.c_uint32),
                ("count", ctypes.c_uint32), ("status", ctypes.c_int32),
                ("logp_norm", F64P), ("length", U32P), ("tokens", U32P),
                ("device_ms", ctypes.c_double * 4),
                ("step_stats", ctypes.POINTER(ctypes.c_uint64))]


# ft_result_fn: void (*)(void* user, size_t r)
RESULT_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_size_t)


def load():
    lib = ctypes.CDLL(LIB)
    lib.ft_create.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                              ctypes.POINTER(ctypes.c_void_p)]
    lib.ft_reserve.argtypes = [ctypes.c_void_p] + [ctypes.c_size_t] * 6
    for name in ("ft_search", "ft_search_noalloc"):
        if hasattr(lib, name):
            getattr(lib, name).argtypes = [ctypes.c_void_p, ctypes.POINTER(Request),
                                           ctypes.c_size_t, ctypes.POINTER(Result),
                                           ctypes.c_void_p]
    if hasattr(lib, "ft_search_each"):
        lib.ft_search_each.argtypes = [ctypes.c_void_p, ctypes.POINTER(Request),
                                       ctypes.c_size_t, ctypes.POINTER(Result),
                                       ctypes.c_void_p, RESULT_FN, ctypes.c_void_p]
    lib.ft_stage.argtypes = [ctypes.c_void_p, ctypes.POINTER(Request), ctypes.c_size_t]
    lib.ft_launch_range.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t]
    lib.ft_fetch.argtypes = [ctypes.c_void_p, ctypes.POINTER(Result), ctypes.c_size_t,
                             ctypes.c_void_p]
    lib.ft_destroy.argtypes = [ctypes.c_void_p]
    lib.ft_last_error.restype = ctypes.c_char_p
    return lib


def check(lib, rc):
    if rc != 0:
        raise RuntimeError(f"{rc}: {lib.ft_last_error().decode()}")


class Batch:
    """Requests over numpy arrays (kept alive here): beams [n][T], ids and
    logp [n][T][K]; results with room for F beams of T tokens."""

    def __init__(self, beams, ids, lp, tok_thr, sent_thr, alpha, early, F):
        self.beams = np.ascontiguousarray(beams, dtype=np.uint32)
        self.ids = np.ascontiguousarray(ids, dtype=np.uint32)
        self.lp = np.ascontiguousarray(lp, dtype=np.float32)
        n, T, K = self.ids.shape
        self.n = n
        self.reqs = (Request * n)()
        for i in range(n):
            r = self.reqs[i]
            r.beams = self.beams[i].ctypes.data_as(U32P)
            r.num_beams = self.beams.shape[1]
            r.num_steps = T
            r.topk = K
            r.topk_id = self.ids[i].ctypes.data_as(U32P)
            r.topk_logp = self.lp[i].ctypes.data_as(F32P)
            r.token_logp_threshold = tok_thr
            r.sent_logp_threshold = sent_thr
            r.length_norm = alpha
            r.early_exit = int(early[i] if np.ndim(early) else early)
        self.norms = np.zeros((n, F), dtype=np.float64)
        self.lens = np.zeros((n, F), dtype=np.uint32)
        self.toks = np.zeros((n, F, T), dtype=np.uint32)
        self.res = (Result * n)()
        for i in range(n):
            self.res[i].capacity = F
            self.res[i].token_stride = T
            self.res[i].logp_norm = self.norms[i].ctypes.data_as(F64P)
            self.res[i].length = self.lens[i].ctypes.data_as(U32P)
            self.res[i].tokens = self.toks[i].ctypes.data_as(U32P)

    def results(self, i):
        """(sequences, norms) of request i."""
        c = self.res[i].count
        seqs = [self.toks[i, j, :self.lens[i, j]].tolist() for j in range(c)]
        return seqs, self.norms[i, :c].copy()
