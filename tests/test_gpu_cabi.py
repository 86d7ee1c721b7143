"""The C ABI driven from ctypes, as another host language would: ft_create,
ft_reserve, ft_search, and ft_stage / ft_launch_range / ft_fetch, against the
oracle; and a second process searching on the GPU while this one lives."""

import ctypes

import numpy as np
import pytest

from cabi import Batch, check, load


@pytest.mark.gpu
def test_c_abi_search_through_ctypes(ft, po):
    lib = load()
    toks, offs = ft.synth_keys(30000, 4096, 3, 8, 1.1, 21)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    image = np.array(t.image(), dtype=np.uint8)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    B, T, K, F, n = 16, 8, 32, 16, 4
    ids, lp = ft.synth_requests(t, 0, n, 4096, T, K, B, 0.3, 2.0, True, 21, model=1)
    beams = np.full((n, T), B, dtype=np.uint32)
    early = [i % 2 for i in range(n)]
    b = Batch(beams, ids, lp, -10.0, -40.0, 5.0, early, F)
    ctx = ctypes.c_void_p()
    check(lib, lib.ft_create(image.ctypes.data, image.nbytes, 0, ctypes.byref(ctx)))
    try:
        check(lib, lib.ft_reserve(ctx, n, K, T, B, B * T, 4096))
        print("ctypes ft_search batch", n, flush=True)
        check(lib, lib.ft_search(ctx, b.reqs, n, b.res, None))
        for i in range(n):
            want = o.tbs(beams[i], ids[i], lp[i], -10.0, -40.0, 5.0, bool(early[i]))
            got = b.results(i)
            assert b.res[i].status == 0
            assert got[0] == want[0], i
            assert np.array_equal(got[1], want[1]), i
        # a staged request that no launch covered comes back FT_E_STATE
        check(lib, lib.ft_stage(ctx, b.reqs, n))
        check(lib, lib.ft_launch_range(ctx, 0, 2))
        rc = lib.ft_fetch(ctx, b.res, n, None)
        assert rc == -5, rc
        assert [b.res[i].status for i in range(n)] == [0, 0, -5, -5]
        want = o.tbs(beams[1], ids[1], lp[1], -10.0, -40.0, 5.0, True)
        assert b.results(1)[0] == want[0]
    finally:
        lib.ft_destroy(ctx)


@pytest.mark.gpu
def test_search_each_hands_over_every_request(ft, po):
    """ft_search_each calls back once for every request whose results are
    complete -- the results are already the oracle's when the callback
    runs -- and not for a request that fails to pack (whose error the call
    returns); a request with final beam 0 is handed over with no results."""
    lib = load()
    from cabi import RESULT_FN
    toks, offs = ft.synth_keys(30000, 4096, 3, 8, 1.1, 22)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    image = np.array(t.image(), dtype=np.uint8)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    B, T, K, F, n = 16, 8, 32, 16, 8
    ids, lp = ft.synth_requests(t, 0, n, 4096, T, K, B, 0.3, 2.0, True, 22, model=1)
    beams = np.full((n, T), B, dtype=np.uint32)
    beams[3, T - 1] = 0  # final beam 0: outputs untouched (louds-trie.cc:114-117)
    lp = lp.copy()
    ctx = ctypes.c_void_p()
    check(lib, lib.ft_create(image.ctypes.data, image.nbytes, 0, ctypes.byref(ctx)))
    try:
        check(lib, lib.ft_reserve(ctx, n, K, T, B, B * T, 4096))
        for bad in (None, 5):
            lpx = lp.copy()
            if bad is not None:
                lpx[bad, 2, 7] = np.nan
            b = Batch(beams, ids, lpx, -10.0, -40.0, 5.0, False, F)
            seen, at_call = [], {}

            def on_result(user, r):
                seen.append(r)
                at_call[r] = (b.res[r].status, b.results(r))

            cb = RESULT_FN(on_result)
            print("ctypes ft_search_each batch", n, "bad", bad, flush=True)
            rc = lib.ft_search_each(ctx, b.reqs, n, b.res, None, cb, None)
            want_seen = [r for r in range(n) if r != bad]
            assert sorted(seen) == want_seen, seen
            if bad is None:
                assert rc == 0, lib.ft_last_error()
            else:
                assert rc == -6, rc  # FT_E_INPUT, naming the request
                assert f"request {bad}" in lib.ft_last_error().decode()
            for r in want_seen:
                status, (seqs, norms) = at_call[r]
                assert status == 0
                if r == 3:
                    assert seqs == [], seqs
                    continue
                want = o.tbs(beams[r], ids[r], lpx[r], -10.0, -40.0, 5.0, False)
                assert seqs == want[0], r
                assert np.array_equal(norms, want[1]), r
    finally:
        lib.ft_destroy(ctx)


@pytest.mark.gpu
def test_second_process_searches_after_this_one(ft, tmp_path):
    # launches are ordinary (no cooperative launch), so a second process can
    # search on the GPU while this one, which has searched already, lives
    import subprocess

    from test_cli import CLI, write_dataset
    t = ft.Trie()
    t.build([[1, 2, 3, 4], [1, 2, 3, 5], [7]])
    t.init_tbs_gpu(1, max_num_topk=8, max_num_outpos=4, max_num_out_beams=8,
                   max_num_out_tokens=32, max_num_inter_beams=64)
    got = ft.bs_tbs_gpu(t, 1, [[8] * 4], [[[1, 2, 3, 4, 5, 7]] * 4],
                        [[[-0.5, -3, -3, -3, -3, -1.0]] * 4], -10.0, -40.0, 0.0, False)
    assert got[0][0]
    write_dataset(ft, str(tmp_path))
    p = subprocess.run([CLI, "-g", "-a", str(tmp_path), "8", "4"], capture_output=True,
                       text=True, timeout=300)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    assert "12/12 requests identical on CPU and GPU" in p.stdout
