"""Seeded synthetic generators: determinism, and the paper-scale trie
generator produces exactly the trie the builder makes from the keys it
encodes (same BFS ids, edges and terminals)."""

import numpy as np
import pytest

from helpers import decode_image, image_logical


def _keys_of(img):
    """All keys of an image, by walking it (edges expanded)."""
    cb, edges, term = image_logical(img)
    keys = []
    stack = [(0, [])]
    while stack:
        n, pre = stack.pop()
        if term[n]:
            keys.append(pre)
        for c in range(cb[n], cb[n + 1]):
            stack.append((c, pre + edges[c]))
    return keys


@pytest.mark.parametrize("n", [2000, 30000])
def test_paper_trie_equals_builder(ft, n):
    t = ft.Trie()
    ft.synth_paper_trie(t, n, 5000, 1.05, 7)
    ft.validate_image(t)
    keys = _keys_of(t.image())
    assert len(keys) == t.num_keys()
    u = ft.Trie()
    u.build(keys)
    assert np.array_equal(t.image(), u.image())


def test_paper_trie_thread_independent(ft):
    imgs = []
    for threads in (1, 3, 8):
        t = ft.Trie()
        ft.synth_paper_trie(t, 200000, 2200000, 1.05, 3, threads=threads)
        imgs.append(t.image())
    assert np.array_equal(imgs[0], imgs[1]) and np.array_equal(imgs[0], imgs[2])


def test_paper_trie_shape(ft):
    t = ft.Trie()
    ft.synth_paper_trie(t, 300000, 2200000, 1.05, 0)
    n, recs, _, _ = decode_image(t.image_view())
    meta = recs["meta"][:n]
    depth = meta & 0xFFFF
    term = (meta >> 31).astype(bool)
    lengths = depth[term]
    assert lengths.min() >= 3 and lengths.max() <= 16
    assert 5.5 < lengths.mean() < 6.5
    assert t.num_keys() > 0.97 * 300000


def test_synth_keys_deterministic(ft):
    a = ft.synth_keys(5000, 4096, 3, 8, 1.1, 9)
    b = ft.synth_keys(5000, 4096, 3, 8, 1.1, 9)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    lens = np.diff(a[1])
    assert lens.min() >= 3 and lens.max() <= 8
    keys = {tuple(a[0][a[1][i]:a[1][i + 1]]) for i in range(5000)}
    assert len(keys) == 5000


def test_synth_requests_rows_sorted_and_valid(ft):
    toks, offs = ft.synth_keys(20000, 4096, 3, 8, 1.1, 1)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    for model in (0, 1):
        ids, lp = ft.synth_requests(t, 0, 8, 4096, 8, 64, 16, 0.3, 2.0, True, 5,
                                    model=model)
        assert (np.diff(ids.astype(np.int64), axis=2) > 0).all()
        assert not np.isnan(lp).any() and (lp < 0).all()
        ids2, lp2 = ft.synth_requests(t, 0, 8, 4096, 8, 64, 16, 0.3, 2.0, True,
                                      5, threads=1, model=model)
        assert np.array_equal(ids, ids2) and np.array_equal(lp, lp2)


def test_paper_trie_topped_up_to_exact_unique_keys(ft):
    # draws give some number of unique keys; unique_keys tops the trie up to
    # exactly that many by making internal nodes (>= 2 children, string depth
    # >= lmin) terminal -- prefix keys -- without changing the structure
    base = ft.Trie()
    ft.synth_paper_trie(base, 30000, 5000, 1.05, 7)
    t = ft.Trie()
    want = base.num_keys() + 123
    ft.synth_paper_trie(t, 30000, 5000, 1.05, 7, unique_keys=want)
    ft.validate_image(t)
    assert t.num_keys() == want
    n, r0, p0, tl0 = decode_image(base.image())
    n1, r1, p1, tl1 = decode_image(t.image())
    assert n == n1 and np.array_equal(p0, p1) and np.array_equal(tl0, tl1)
    for f in ("child_begin", "first_tok", "tail_off"):
        assert np.array_equal(r0[f], r1[f])
    m0, m1 = r0["meta"][:n], r1["meta"][:n]
    added = np.nonzero((m1 >> 31) & ~(m0 >> 31) & 1)[0]
    assert len(added) == 123
    assert np.array_equal(m0 & 0x7FFFFFFF, m1 & 0x7FFFFFFF)
    deg = np.diff(r0["child_begin"].astype(np.int64))[:n]
    assert (deg[added] >= 2).all() and ((m0[added] & 0xFFFF) >= 3).all()
    # the keys really are the old ones plus the added prefixes, all distinct,
    # and the builder makes the same image from them
    keys = _keys_of(t.image())
    assert len(keys) == len({tuple(k) for k in keys}) == want
    u = ft.Trie()
    u.build(keys)
    assert np.array_equal(t.image(), u.image())
    # seeded: the same call gives the same trie; a target below the count is
    # an error
    t2 = ft.Trie()
    ft.synth_paper_trie(t2, 30000, 5000, 1.05, 7, unique_keys=want)
    assert np.array_equal(t.image(), t2.image())
    with pytest.raises(RuntimeError, match="more than the target"):
        ft.synth_paper_trie(ft.Trie(), 30000, 5000, 1.05, 7,
                            unique_keys=base.num_keys() - 1)


def test_keys_of_round_trip(ft):
    # keys_of lists every key in lexicographic order; building from them
    # gives the same image
    t = ft.Trie()
    ft.synth_paper_trie(t, 20000, 3000, 1.05, 5)
    toks, offs = ft.keys_of(t)
    keys = [tuple(toks[offs[i]:offs[i + 1]]) for i in range(offs.size - 1)]
    assert len(keys) == t.num_keys()
    assert keys == sorted(set(tuple(k) for k in _keys_of(t.image())))
    u = ft.Trie()
    u.build_arrays(toks, offs)
    assert np.array_equal(t.image(), u.image())
    # a seeded random order of the same keys builds the same image
    st, so = ft.keys_of(t, 7)
    shuffled = [tuple(st[so[i]:so[i + 1]]) for i in range(so.size - 1)]
    assert shuffled != keys and sorted(shuffled) == keys
    w = ft.Trie()
    w.build_arrays(st, so)
    assert np.array_equal(t.image(), w.image())
