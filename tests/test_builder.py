"""The product's image builder against the oracle's restated MARISA build:
same node ids, edges, terminals; image invariants; save / load."""

import os

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from helpers import decode_image, image_logical, oracle_logical


def _same_trie(ft, po, keys=None, toks=None, offs=None):
    t = ft.Trie()
    if keys is not None:
        t.build(keys)
        o = po.OracleTrie.from_keys(keys)
    else:
        t.build_arrays(toks, offs)
        o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    a = image_logical(t.image())
    b = oracle_logical(o)
    assert np.array_equal(a[0], b[0])
    assert a[1] == b[1]
    assert np.array_equal(a[2], b[2])
    assert t.num_keys() == o.num_keys()
    assert t.num_nodes() == o.num_nodes()
    return t


@settings(max_examples=80, deadline=None)
@given(st.lists(st.lists(st.integers(0, 7), min_size=0, max_size=7),
                min_size=1, max_size=50))
def test_matches_oracle_small(ft, po, keys):
    _same_trie(ft, po, keys=keys)


def test_matches_oracle_synthetic(ft, po):
    toks, offs = ft.synth_keys(30000, 4096, 3, 8, 1.1, 11)
    assert len(offs) - 1 == 30000
    _same_trie(ft, po, toks=toks, offs=offs)


def test_empty_key_and_duplicates(ft, po):
    _same_trie(ft, po, keys=[[], [1], [1], [1, 2], []])


def test_image_fields(ft):
    t = ft.Trie()
    t.build([[1, 2, 3, 4], [1, 2, 3, 5], [7]])
    n, recs, parent, tail = decode_image(t.image())
    assert n == 5
    meta = recs["meta"]
    depth = meta & 0xFFFF
    elen = (meta >> 16) & 0x3FFF
    assert depth[:5].tolist() == [0, 3, 1, 4, 4]
    assert elen[:5].tolist() == [0, 3, 1, 1, 1]
    assert parent.tolist() == [0, 0, 0, 1, 1]
    assert tail[recs["tail_off"][1]:recs["tail_off"][1] + 3].tolist() == [1, 2, 3]
    assert recs["child_begin"][5] == 5   # sentinel


def test_rejects_large_token(ft):
    t = ft.Trie()
    with pytest.raises(RuntimeError, match="2\\^31"):
        t.build([[1, 2 ** 31]])


def test_save_load_roundtrip(ft, tmp_path):
    t = ft.Trie()
    t.build([[3, 1], [3, 2, 9], [4]])
    p = str(tmp_path / "trie.ftimg")
    t.save(p)
    u = ft.Trie()
    u.load(p)
    assert np.array_equal(t.image(), u.image())
    assert u.num_keys() == 3 and u.num_tries() == 1
    m = ft.Trie()
    m.mmap(p)
    assert np.array_equal(t.image(), m.image())


def test_mmap_maps_images_and_converts_marisa_files(ft, tmp_path):
    # an image file is mapped and used in place; a MARISA trie file is
    # converted from the mapping; both search like the built trie, and the
    # mapping stays valid after the file is unlinked (the mapping holds it)
    toks, offs = ft.synth_keys(3000, 512, 2, 6, 1.1, 5)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    p_img, p_bin = str(tmp_path / "trie.ftimg"), str(tmp_path / "trie.bin")
    t.save(p_img)
    t.save_marisa(p_bin)
    ids, lp = ft.synth_requests(t, 0, 3, 512, 6, 16, 8, 0.3, 2.0, True, 5, model=1)
    want = [ft.tbs(t, [8] * 6, ids[r].tolist(), lp[r].tolist(), -10.0, -40.0, 5.0, False)
            for r in range(3)]
    for path in (p_img, p_bin):
        m = ft.Trie()
        m.mmap(path)
        if path == p_img:
            import os
            os.unlink(path)
        if path == p_img:  # (a converted MARISA file keeps its shared tail)
            assert np.array_equal(t.image(), m.image()), path
        assert m.num_keys() == t.num_keys() and m.num_nodes() == t.num_nodes()
        for r in range(3):
            got = ft.tbs(m, [8] * 6, ids[r].tolist(), lp[r].tolist(), -10.0, -40.0, 5.0,
                         False)
            assert got[0] == want[r][0] and list(got[1]) == list(want[r][1])
    with pytest.raises(RuntimeError):
        ft.Trie().mmap(str(tmp_path / "missing.ftimg"))
    empty = tmp_path / "empty.ftimg"
    empty.write_bytes(b"")
    with pytest.raises(RuntimeError):
        ft.Trie().mmap(str(empty))
    short = tmp_path / "short.ftimg"
    short.write_bytes(t.image().tobytes()[:1000])
    with pytest.raises(RuntimeError):
        ft.Trie().mmap(str(short))


def test_load_rejects_truncated_marisa_file(ft, tmp_path):
    # a MARISA header followed by too few bytes for its sections
    p = tmp_path / "trie.bin"
    p.write_bytes(b"We love Marisa." + b"\0" * 64)
    with pytest.raises(RuntimeError, match="truncated"):
        ft.Trie().load(str(p))


def test_load_rejects_corrupt_image(ft, tmp_path):
    t = ft.Trie()
    t.build([[3, 1], [3, 2, 9], [4]])
    img = t.image().copy()
    _, recs, _, _ = decode_image(img)
    ro = 256
    img[ro + 16 + 0] = 0   # node 1's child_begin -> 0 (not BFS)
    p = tmp_path / "bad.ftimg"
    p.write_bytes(img.tobytes())
    with pytest.raises(RuntimeError):
        ft.Trie().load(str(p))


def test_uninitialised_trie_errors(ft):
    t = ft.Trie()
    with pytest.raises(RuntimeError):
        t.num_keys()
    t.build([[1]])
    with pytest.raises(RuntimeError, match="init_tbs_gpu"):
        ft.bs_tbs_gpu(t, 1, [[1]], [[[1]]], [[[-1.0]]], -10, -40, 5, False)
