"""ctypes wrapper of the CPU parity oracle (test infrastructure only).

Imported only by tests/, ``__graft_entry__.smoke()`` and bench.py's
cpu_baseline leg.  The oracle restates the reference CPU path
``LoudsTrie::tbs`` (lib/marisa/grimoire/trie/louds-trie.cc:75-177) and the
MARISA BFS trie build (louds-trie.cc:477-588); see oracle.cc for the map.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

AS_WRITTEN = 0
FAST = 1

_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, u64, u32p = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p
        L.ot_build.restype = vp
        L.ot_build.argtypes = [vp, vp, u64]
        L.ot_wrap_image.restype = vp
        L.ot_wrap_image.argtypes = [vp, vp, u64]
        L.ot_free.argtypes = [vp]
        L.ot_num_nodes.restype = u64
        L.ot_num_nodes.argtypes = [vp]
        L.ot_num_keys.restype = u64
        L.ot_num_keys.argtypes = [vp]
        L.ot_num_edge_tokens.restype = u64
        L.ot_num_edge_tokens.argtypes = [vp]
        L.ot_export.restype = ctypes.c_int
        L.ot_export.argtypes = [vp, vp, vp, vp, vp]
        L.ot_tbs.restype = ctypes.c_int
        L.ot_tbs.argtypes = [vp, vp, u64, vp, vp, u64, u64, ctypes.c_float,
                             ctypes.c_double, ctypes.c_double, ctypes.c_int,
                             ctypes.c_int, u64, vp, vp, vp, vp, vp, vp]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def pack_keys(keys):
    """List of token lists -> (flat uint32 tokens, uint64 offsets)."""
    lens = np.fromiter((len(k) for k in keys), dtype=np.uint64,
                       count=len(keys))
    offs = np.zeros(len(keys) + 1, dtype=np.uint64)
    np.cumsum(lens, out=offs[1:])
    toks = np.fromiter((t for k in keys for t in k), dtype=np.uint32,
                       count=int(offs[-1]))
    return toks, offs


class OracleTrie:
    """A trie built by the restated MARISA builder, or a view over a device
    image held in host memory."""

    def __init__(self, handle, keep=()):
        self.h = handle
        self._keep = keep

    @classmethod
    def from_keys(cls, keys=None, toks=None, offs=None):
        if keys is not None:
            toks, offs = pack_keys(keys)
        toks = np.ascontiguousarray(toks, dtype=np.uint32)
        offs = np.ascontiguousarray(offs, dtype=np.uint64)
        if toks.size == 0:
            toks = np.zeros(1, dtype=np.uint32)
        h = lib().ot_build(_ptr(toks), _ptr(offs), len(offs) - 1)
        if not h:
            raise RuntimeError("oracle build failed")
        return cls(h)

    @classmethod
    def from_image(cls, recs, tail, num_nodes):
        recs = np.ascontiguousarray(recs)
        tail = np.ascontiguousarray(tail, dtype=np.uint32)
        if tail.size == 0:
            tail = np.zeros(1, dtype=np.uint32)
        h = lib().ot_wrap_image(_ptr(recs), _ptr(tail), num_nodes)
        return cls(h, keep=(recs, tail))

    @classmethod
    def from_trie(cls, t):
        """The oracle over a flashtrie.Trie's own image (no copy: it keeps
        views of the image's record and tail arrays)."""
        img = t.image_view()
        hdr = np.frombuffer(img[:64].tobytes(), dtype="<u8", count=8)
        nn, tl, ro, to = int(hdr[1]), int(hdr[3]), int(hdr[4]), int(hdr[6])
        recs = img[ro:ro + (nn + 1) * 16]
        tail = img[to:to + max(tl, 1) * 4].view(np.uint32)
        return cls.from_image(recs, tail, nn)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.ot_free(self.h)
            self.h = None

    def num_nodes(self):
        return int(lib().ot_num_nodes(self.h))

    def num_keys(self):
        return int(lib().ot_num_keys(self.h))

    def export(self):
        """(child_begin[N+1], edge_begin[N+1], edge_tok[], terminal[N])."""
        n = self.num_nodes()
        ne = int(lib().ot_num_edge_tokens(self.h))
        cb = np.zeros(n + 1, dtype=np.uint32)
        eb = np.zeros(n + 1, dtype=np.uint64)
        et = np.zeros(max(ne, 1), dtype=np.uint32)
        term = np.zeros(n, dtype=np.uint8)
        rc = lib().ot_export(self.h, _ptr(cb), _ptr(eb), _ptr(et), _ptr(term))
        if rc != 0:
            raise RuntimeError("export needs a trie built from keys")
        return cb, eb, et[:ne], term

    def tbs(self, beams, topk_id, topk_logp, token_logp_threshold=-10.0,
            sents_logp_threshold=-40.0, length_norm=5.0, early_exit=False,
            variant=FAST, with_nodes=False, with_work=False):
        """Returns (sents, logp_norm) like ``flashtrie.tbs``; sents is a list
        of token lists in the reference's output order."""
        beams = np.ascontiguousarray(beams, dtype=np.uint32)
        ids = np.ascontiguousarray(topk_id, dtype=np.uint32)
        lp = np.ascontiguousarray(topk_logp, dtype=np.float32)
        if ids.ndim != 2 or ids.shape != lp.shape:
            raise ValueError("topk_id / topk_logp must be 2-D of one shape")
        T, K = ids.shape
        cap = int(beams[-1]) if beams.size else 0
        cap = max(cap, 1)
        count = np.zeros(1, dtype=np.uint64)
        norm = np.zeros(cap, dtype=np.float64)
        ln = np.zeros(cap, dtype=np.uint32)
        tok = np.zeros(cap * max(T, 1), dtype=np.uint32)
        nodes = np.zeros(cap, dtype=np.uint64)
        work = np.zeros(7, dtype=np.uint64)
        if ids.size == 0:
            ids = np.zeros((1, 1), dtype=np.uint32)
            lp = np.zeros((1, 1), dtype=np.float32)
        rc = lib().ot_tbs(self.h, _ptr(beams), beams.size, _ptr(ids), _ptr(lp),
                          T, K, float(token_logp_threshold),
                          float(sents_logp_threshold), float(length_norm),
                          int(bool(early_exit)), int(variant), cap,
                          _ptr(count), _ptr(norm), _ptr(ln), _ptr(tok),
                          _ptr(nodes), _ptr(work))
        if rc < 0:
            raise ValueError(f"oracle tbs: undefined-behaviour input ({rc})")
        n = int(count[0])
        sents = [tok[i * T:i * T + int(ln[i])].tolist() for i in range(n)]
        res = (sents, norm[:n].copy())
        if with_nodes:
            res = res + (nodes[:n].copy(),)
        if with_work:
            res = res + (work.copy(),)
        return res
