"""ft_search_noalloc (the entry point that allocates nothing: its batch
lives in one static device array per device) against ft_search, the entry
point it is a variant of: identical results, bit for bit, on two calls in a
row (the second smaller, so stale contents of the shared array would show),
with and without steps shared between workgroups, and at beam = topk =
1000; sizes beyond the array are an FT_E_LIMIT before any device work."""

import ctypes

import numpy as np
import pytest

from cabi import Batch, check, load

pytestmark = pytest.mark.gpu


def _ctx(lib, image):
    ctx = ctypes.c_void_p()
    check(lib, lib.ft_create(image.ctypes.data, image.nbytes, 0, ctypes.byref(ctx)))
    return ctx


def _same(lib, ctx, b_ref, b_na, what, po_trie=None, args=None):
    n = b_ref.n
    print("no-alloc case", what, flush=True)
    check(lib, lib.ft_search(ctx, b_ref.reqs, n, b_ref.res, None))
    check(lib, lib.ft_search_noalloc(ctx, b_na.reqs, n, b_na.res, None))
    for i in range(n):
        assert b_na.res[i].status == b_ref.res[i].status == 0, (what, i)
        assert b_na.res[i].count == b_ref.res[i].count, (what, i)
        s_ref, n_ref = b_ref.results(i)
        s_na, n_na = b_na.results(i)
        assert s_na == s_ref, (what, i)
        assert np.array_equal(n_na, n_ref), (what, i)
        if po_trie is not None:
            beams, ids, lp, early = args
            want = po_trie.tbs(beams[i], ids[i], lp[i], -10.0, -40.0, 5.0, bool(early[i]))
            assert s_na == want[0] and np.array_equal(n_na, want[1]), (what, i)


def _batch(ft, t, first, n, T, K, B, seed, vocab=4096):
    ids, lp = ft.synth_requests(t, first, n, vocab, T, K, B, 0.3, 2.0, True, seed, model=1)
    beams = np.full((n, T), B, dtype=np.uint32)
    early = [(first + i) % 2 for i in range(n)]
    mk = lambda: Batch(beams, ids, lp, -10.0, -40.0, 5.0, early, B)  # noqa: E731
    return mk(), mk(), (beams, ids, lp, early)


@pytest.fixture(scope="module")
def trie(ft, po):
    toks, offs = ft.synth_keys(50000, 4096, 3, 8, 1.1, 31)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    return t, np.array(t.image(), dtype=np.uint8), po.OracleTrie.from_keys(toks=toks, offs=offs)


def test_noalloc_matches_search_twice(ft, trie):
    t, image, o = trie
    lib = load()
    ctx = _ctx(lib, image)
    try:
        check(lib, lib.ft_reserve(ctx, 4, 64, 8, 32, 32 * 8, 4096))
        r1, n1, a1 = _batch(ft, t, 0, 4, 8, 64, 32, 31)
        _same(lib, ctx, r1, n1, "first call: batch 4, beam 32, K 64, 8 steps", o, a1)
        # second, smaller call: a batch of 2, narrower beams, fewer steps
        r2, n2, a2 = _batch(ft, t, 10, 2, 6, 32, 16, 32)
        _same(lib, ctx, r2, n2, "second call: batch 2, beam 16, K 32, 6 steps", o, a2)
    finally:
        lib.ft_destroy(ctx)


def test_noalloc_shared_steps(ft, trie, monkeypatch):
    # every step spread over 8 workgroups: helpers read the step from the
    # control block in the array, which each call clears
    monkeypatch.setenv("FT_WGS", "8")
    monkeypatch.setenv("FT_SHARE_MIN", "0")
    t, image, o = trie
    lib = load()
    ctx = _ctx(lib, image)
    try:
        check(lib, lib.ft_reserve(ctx, 3, 64, 8, 32, 32 * 8, 4096))
        r1, n1, a1 = _batch(ft, t, 20, 3, 8, 64, 32, 33)
        _same(lib, ctx, r1, n1, "shared steps, batch 3", o, a1)
        r2, n2, a2 = _batch(ft, t, 30, 1, 5, 48, 24, 34)
        _same(lib, ctx, r2, n2, "shared steps, batch 1 after batch 3", o, a2)
    finally:
        lib.ft_destroy(ctx)


def test_noalloc_beam_1000_and_limits(ft, trie):
    t, image, o = trie
    lib = load()
    ctx = _ctx(lib, image)
    try:
        check(lib, lib.ft_reserve(ctx, 2, 1000, 8, 1000, 8000, 8000))
        r1, n1, a1 = _batch(ft, t, 40, 1, 8, 1000, 1000, 35)
        _same(lib, ctx, r1, n1, "batch 1, beam = topk = 1000", o, a1)
        # batch 8 at beam = topk = 1000 needs ~640 MB: refused before any
        # device work
        big = _batch(ft, t, 50, 8, 8, 1000, 1000, 36)[1]
        rc = lib.ft_search_noalloc(ctx, big.reqs, 8, big.res, None)
        assert rc == -4, rc
        assert b"scratch" in lib.ft_last_error()
        # the array still works after the refusal
        r2, n2, a2 = _batch(ft, t, 60, 2, 8, 64, 32, 37)
        _same(lib, ctx, r2, n2, "batch 2 after a refused batch", o, a2)
    finally:
        lib.ft_destroy(ctx)
