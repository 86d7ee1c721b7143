"""GPU parity: the HIP search (through flashtrie -> the C ABI) against the CPU
oracle on identical seeded inputs.  Sequences and lengths bit-exact; scores
within 1e-5 relative (they are in fact bit-identical: the length-norm
factor comes from a host pow table and the f64 additions are the same)."""

import math

import numpy as np
import pytest

from helpers import assert_same_results, load_golden

pytestmark = pytest.mark.gpu

KA = load_golden("known_answers.json")


def _gpu_trie(ft, keys=None, toks=None, offs=None, batch=8, topk=64, steps=16,
              beams=64, inter=1 << 16):
    t = ft.Trie()
    if keys is not None:
        t.build(keys)
    else:
        t.build_arrays(toks, offs)
    t.init_tbs_gpu(batch, max_num_topk=topk, max_num_outpos=steps,
                   max_num_out_beams=beams, max_num_out_tokens=beams * steps,
                   max_num_inter_beams=inter)
    return t


@pytest.mark.parametrize("case", KA, ids=[c["name"] for c in KA])
def test_known_answers(ft, case):
    print("KA case", case["name"], flush=True)
    t = _gpu_trie(ft, keys=case["keys"])
    sents, norms, _, phases = ft.bs_tbs_gpu(
        t, 1, [case["beams"]], [case["topk_id"]], [case["topk_logp"]],
        case["token_logp_threshold"], case["sents_logp_threshold"],
        case["length_norm"], case["early_exit"])
    assert sents[0] == case["expect_sents"]
    assert np.allclose(norms[0], case["expect_scores_approx"], rtol=1e-6, atol=0)
    assert len(phases[0]) == 5
    s2, n2, _ = ft.tbs(t, case["beams"], case["topk_id"], case["topk_logp"],
                       case["token_logp_threshold"], case["sents_logp_threshold"],
                       case["length_norm"], case["early_exit"], True)
    assert s2 == sents[0] and list(n2) == list(norms[0])


def test_known_answers_batched(ft):
    # KA-5, KA-6, KA-7 share a trie and parameters: one launch
    cases = [c for c in KA if c["name"].startswith(("KA-5", "KA-6", "KA-7"))]
    t = _gpu_trie(ft, keys=cases[0]["keys"])
    sents, norms, _, _ = ft.bs_tbs_gpu(
        t, len(cases), [c["beams"] for c in cases], [c["topk_id"] for c in cases],
        [c["topk_logp"] for c in cases], -10.0, -40.0, 0.0, False)
    for c, s, n in zip(cases, sents, norms):
        assert s == c["expect_sents"], c["name"]
        assert np.allclose(n, c["expect_scores_approx"], rtol=1e-6, atol=0)


def test_random_tiny_tries(ft, po):
    rng = np.random.default_rng(7)
    for case in range(120):
        vocab = int(rng.integers(2, 10))
        keys = sorted({tuple(rng.integers(0, vocab, int(rng.integers(1, 7))))
                       for _ in range(int(rng.integers(1, 40)))})
        keys = [list(map(int, k)) for k in keys]
        T = int(rng.integers(1, 8))
        K = int(rng.integers(1, vocab + 1))
        B = int(rng.integers(1, 6))
        ids = np.stack([np.sort(rng.choice(vocab, K, replace=False))
                        for _ in range(T)]).astype(np.uint32)
        # quantised logps make exact norm ties common
        lp = (-rng.integers(0, 8, (T, K)) * 0.5).astype(np.float32)
        beams = [int(rng.integers(1, B + 1)) for _ in range(T)]
        early = bool(rng.integers(0, 2))
        alpha = float(rng.choice([0.0, 1.0, 5.0]))
        print("tiny case", case, flush=True)
        t = _gpu_trie(ft, keys=keys, batch=1, topk=16, steps=8, beams=8)
        got = ft.bs_tbs_gpu(t, 1, [beams], [ids.tolist()], [lp.tolist()],
                            -3.0, -9.0, alpha, early)
        o = po.OracleTrie.from_keys(keys)
        want = o.tbs(beams, ids, lp, -3.0, -9.0, alpha, early)
        assert_same_results((got[0][0], got[1][0]), want, f"tiny case {case}")


C1 = dict(n=100000, vocab=32768, lmin=3, lmax=8, s=1.1, seed=0)


@pytest.fixture(scope="module")
def c1(ft, po):
    toks, offs = ft.synth_keys(C1["n"], C1["vocab"], C1["lmin"], C1["lmax"],
                               C1["s"], C1["seed"])
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=8, topk=32, steps=8, beams=10,
                  inter=1024)
    ids, lp = ft.synth_requests(t, 0, 200, C1["vocab"], 8, 32, 8, 0.3, 2.0,
                                True, 0)
    return t, po.OracleTrie.from_keys(toks=toks, offs=offs), ids, lp


@pytest.mark.parametrize("early", [False, True])
def test_c1_batch1(ft, c1, early):
    t, o, ids, lp = c1
    beams = [10] * 8
    nonempty = 0
    for r in range(200):
        got = ft.bs_tbs_gpu(t, 1, [beams], [ids[r].tolist()], [lp[r].tolist()],
                            -10.0, -40.0, 5.0, early)
        want = o.tbs(beams, ids[r], lp[r], -10.0, -40.0, 5.0, early)
        assert_same_results((got[0][0], got[1][0]), want, f"C1 request {r}")
        nonempty += len(want[0]) > 0
    assert nonempty > 150


def test_c1_batched_numpy(ft, c1):
    t, o, ids, lp = c1
    beams = np.full((8, 8), 10, dtype=np.uint32)
    for b0 in range(0, 64, 8):
        ft.stage(t, beams, ids[b0:b0 + 8], lp[b0:b0 + 8], -10.0, -40.0, 5.0, False)
        ft.launch(t)
        count, norms, lens, toks, timing = ft.fetch(t)
        assert timing["kernel_ms"] > 0
        for i in range(8):
            want = o.tbs(beams[i], ids[b0 + i], lp[b0 + i], -10.0, -40.0, 5.0, False)
            n = int(count[i])
            sents = [toks[i, j, :lens[i, j]].tolist() for j in range(n)]
            assert_same_results((sents, norms[i, :n]), want, f"batch {b0}+{i}")


def test_bs_tbs_gpu_argument_forms(ft, c1):
    """bs_tbs_gpu reads lists, tuples and numpy arrays (a [B][T][K] batch,
    per-request [T][K] arrays, float64 logps, int64 ids) in place: every
    form gives the same results as the reference's nested lists, and those
    equal the oracle's."""
    t, o, ids, lp = c1
    B = 8
    beams = [[10] * 8] * B
    for b0 in range(0, 32, B):
        bi, bl = ids[b0:b0 + B], lp[b0:b0 + B]
        print("argument forms, requests", b0, flush=True)
        forms = {
            "lists": (beams, bi.tolist(), bl.tolist()),
            "np3d": (np.full((B, 8), 10, np.uint32), bi, bl),
            "np2d_each": (beams, list(bi), list(bl)),
            "f64_i64": (beams, bi.astype(np.int64), bl.astype(np.float64)),
            "tuples": (tuple(map(tuple, beams)), tuple(r.tolist() for r in bi),
                       tuple(r.tolist() for r in bl)),
        }
        ref = None
        for name, (bb, ii, ll) in forms.items():
            sents, norms, ms, phase = ft.bs_tbs_gpu(t, B, bb, ii, ll, -10.0, -40.0, 5.0,
                                                    False)
            assert isinstance(sents, list) and isinstance(norms[0], list), name
            assert ms >= 0 and len(phase) == B and len(phase[0]) == 5, name
            if ref is None:
                ref = (sents, norms)
                for i in range(B):
                    want = o.tbs([10] * 8, bi[i], bl[i], -10.0, -40.0, 5.0, False)
                    assert_same_results((sents[i], norms[i]), want, f"{b0}+{i}")
            else:
                assert sents == ref[0], name
                assert [np.asarray(n).view(np.uint64).tolist() for n in norms] == \
                    [np.asarray(n).view(np.uint64).tolist() for n in ref[1]], name
    # tbs(use_gpu=True) with numpy arrays
    for r in range(4):
        got = ft.tbs(t, np.full(8, 10), ids[r], lp[r], -10.0, -40.0, 5.0, False, True)
        want = o.tbs([10] * 8, ids[r], lp[r], -10.0, -40.0, 5.0, False)
        assert_same_results(got[:2], want, f"tbs request {r}")


def test_c1_as_written_oracle(ft, c1, po):
    t, o, ids, lp = c1
    for r in range(10):
        got = ft.tbs(t, [10] * 8, ids[r].tolist(), lp[r].tolist(), -10.0, -40.0,
                     5.0, False, True)
        want = o.tbs([10] * 8, ids[r], lp[r], -10.0, -40.0, 5.0, False,
                     variant=po.AS_WRITTEN)
        assert_same_results(got[:2], want, f"C1 request {r} (as written)")


def test_ties_everywhere(ft, c1):
    # alpha = 1e6 underflows every length factor beyond depth 1 to 0, so all
    # norms tie and the arrival-order rule decides every cut
    t, o, ids, lp = c1
    for r in range(40):
        for early in (False, True):
            got = ft.bs_tbs_gpu(t, 1, [[10] * 8], [ids[r].tolist()],
                                [lp[r].tolist()], -10.0, -40.0, 1e6, early)
            want = o.tbs([10] * 8, ids[r], lp[r], -10.0, -40.0, 1e6, early)
            assert_same_results((got[0][0], got[1][0]), want, f"tie request {r}")


def test_unsorted_rows(ft, c1):
    t, o, ids, lp = c1
    rng = np.random.default_rng(3)
    for r in range(30):
        perm = np.stack([rng.permutation(32) for _ in range(8)])
        i2 = np.take_along_axis(ids[r], perm, 1)
        l2 = np.take_along_axis(lp[r], perm, 1)
        got = ft.bs_tbs_gpu(t, 1, [[6] * 8], [i2.tolist()], [l2.tolist()],
                            -10.0, -40.0, 5.0, r % 2 == 1)
        want = o.tbs([6] * 8, i2, l2, -10.0, -40.0, 5.0, r % 2 == 1)
        assert_same_results((got[0][0], got[1][0]), want, f"unsorted {r}")


def test_streamed_rows_arrive_during_the_search(ft, c1):
    # Batches of 4: the host publishes every request's first rows before it
    # packs the rest of any, and a leader copies the later rows -- and, once
    # a row after those comes out of order, the proposal indices of every
    # row -- when a step first needs them.  Logps rounded to halves make ties,
    # so the staged indices decide arrival order.
    t, o, ids, lp = c1
    rng = np.random.default_rng(11)
    for b0 in range(0, 32, 4):
        I, L, want = [], [], []
        early = (b0 // 4) % 2 == 1
        for r in range(b0, b0 + 4):
            i2 = ids[r].copy()
            l2 = np.round(lp[r] * 2.0) / 2.0
            if r % 2 == 0:
                tt = 3 + r % 5
                perm = rng.permutation(i2.shape[1])
                i2[tt] = i2[tt][perm]
                l2[tt] = l2[tt][perm]
            I.append(i2.tolist())
            L.append(l2.tolist())
            want.append(o.tbs([6] * 8, i2, l2, -10.0, -40.0, 5.0, early))
        got = ft.bs_tbs_gpu(t, 4, [[6] * 8] * 4, I, L, -10.0, -40.0, 5.0, early)
        for k in range(4):
            assert_same_results((got[0][k], got[1][k]), want[k], f"streamed rows {b0 + k}")
    # a NaN in a late row withdraws the batch's call; the next call is sound
    bad = lp[1].copy()
    bad[6, 2] = np.nan
    with pytest.raises(RuntimeError, match="NaN"):
        ft.bs_tbs_gpu(t, 4, [[6] * 8] * 4, [ids[r].tolist() for r in range(4)],
                      [lp[0].tolist(), bad.tolist(), lp[2].tolist(), lp[3].tolist()],
                      -10.0, -40.0, 5.0, False)
    got = ft.bs_tbs_gpu(t, 4, [[6] * 8] * 4, [ids[r].tolist() for r in range(4)],
                        [lp[r].tolist() for r in range(4)], -10.0, -40.0, 5.0, False)
    for k in range(4):
        want = o.tbs([6] * 8, ids[k], lp[k], -10.0, -40.0, 5.0, False)
        assert_same_results((got[0][k], got[1][k]), want, f"after withdrawal {k}")


@pytest.mark.parametrize("K,T", [(10, 8), (7, 8), (32, 2)])
def test_streamed_split_rows(ft, c1, K, T):
    # The split of a streamed request is the first row h >= 3 with h * K a
    # multiple of 8 (row arrays split on 16 bytes): K = 10 moves it to 4,
    # K = 7 leaves none before T = 8 (whole requests), T = 2 has none.  Rows
    # after the split come out of order in half the requests.
    t, o, ids, lp = c1
    rng = np.random.default_rng(17 + K + T)
    for b0 in range(0, 16, 4):
        I, L, want = [], [], []
        for r in range(b0, b0 + 4):
            i2 = ids[r][:T, :K].copy()
            l2 = lp[r][:T, :K].copy()
            if r % 2 == 1 and T > 4:
                tt = 4 + r % (T - 4)
                perm = rng.permutation(K)
                i2[tt] = i2[tt][perm]
                l2[tt] = l2[tt][perm]
            I.append(i2.tolist())
            L.append(l2.tolist())
            want.append(o.tbs([6] * T, i2, l2, -10.0, -40.0, 5.0, False))
        got = ft.bs_tbs_gpu(t, 4, [[6] * T] * 4, I, L, -10.0, -40.0, 5.0, False)
        for k in range(4):
            assert_same_results((got[0][k], got[1][k]), want[k],
                                f"split K={K} T={T} request {b0 + k}")


def test_mixed_beam_widths(ft, c1):
    t, o, ids, lp = c1
    rng = np.random.default_rng(5)
    for r in range(30):
        beams = [int(x) for x in rng.integers(1, 11, 8)]
        got = ft.bs_tbs_gpu(t, 1, [beams], [ids[r].tolist()], [lp[r].tolist()],
                            -10.0, -40.0, 5.0, False)
        want = o.tbs(beams, ids[r], lp[r], -10.0, -40.0, 5.0, False)
        assert_same_results((got[0][0], got[1][0]), want, f"mixed {r}")


def test_request_errors(ft, c1):
    t, o, ids, lp = c1
    row = ids[0].tolist()
    bad = [list(r) for r in row]
    bad[2][1] = bad[2][0]  # duplicate token id
    with pytest.raises(RuntimeError, match="duplicate"):
        ft.bs_tbs_gpu(t, 1, [[10] * 8], [bad], [lp[0].tolist()], -10, -40, 5, False)
    nan = lp[0].copy()
    nan[1, 3] = np.nan
    with pytest.raises(RuntimeError, match="NaN"):
        ft.bs_tbs_gpu(t, 1, [[10] * 8], [row], [nan.tolist()], -10, -40, 5, False)
    with pytest.raises(RuntimeError, match="max_num_out_beams"):
        ft.bs_tbs_gpu(t, 1, [[11] * 8], [row], [lp[0].tolist()], -10, -40, 5, False)
    with pytest.raises(RuntimeError):
        ft.bs_tbs_gpu(t, 9, [[10] * 8] * 9, [row] * 9, [lp[0].tolist()] * 9,
                      -10, -40, 5, False)
    # final beam 0 leaves the outputs untouched (empty)
    s, n, _, _ = ft.bs_tbs_gpu(t, 2, [[10] * 7 + [0], [10] * 8], [row, row],
                               [lp[0].tolist()] * 2, -10, -40, 5, False)
    assert s[0] == [] and list(n[0]) == []
    want = o.tbs([10] * 8, ids[0], lp[0], -10, -40, 5, False)
    assert_same_results((s[1], n[1]), want)
    # the context still works after errors
    got = ft.bs_tbs_gpu(t, 1, [[10] * 8], [row], [lp[0].tolist()], -10, -40, 5, False)
    assert_same_results((got[0][0], got[1][0]), want)


def test_conversion_errors_come_first(ft, c1):
    """An element that cannot be converted raises the conversion's error
    (TypeError, as pybind11's caster does), before any search error of the
    batch: a plan error of a later request, or a packing error of an
    earlier one; a ragged row raises marisa::Trie's shape error; the next
    call is unaffected."""
    t, o, ids, lp = c1
    rows = [ids[r].tolist() for r in range(8)]
    lps = [lp[r].tolist() for r in range(8)]
    beams = [[10] * 8 for _ in range(8)]

    def with_text(r):
        bad = [list(x) for x in rows[r]]
        bad[3][4] = "7"
        return bad

    print("conversion error alone", flush=True)
    bi = list(rows)
    bi[3] = with_text(3)
    with pytest.raises(TypeError, match="incompatible arguments"):
        ft.bs_tbs_gpu(t, 8, beams, bi, lps, -10.0, -40.0, 5.0, False)
    print("conversion error before a later request's plan error", flush=True)
    bi = list(rows)
    bi[2] = with_text(2)
    bb = [list(b) for b in beams]
    bb[5] = [11] * 8  # above max_num_out_beams
    with pytest.raises(TypeError, match="incompatible arguments"):
        ft.bs_tbs_gpu(t, 8, bb, bi, lps, -10.0, -40.0, 5.0, False)
    print("conversion error after an earlier request's packing error", flush=True)
    bi = list(rows)
    bi[6] = with_text(6)
    bl = list(lps)
    nan = lp[1].copy()
    nan[2, 7] = np.nan
    bl[1] = nan.tolist()
    with pytest.raises(TypeError, match="incompatible arguments"):
        ft.bs_tbs_gpu(t, 8, beams, bi, bl, -10.0, -40.0, 5.0, False)
    print("ragged row in a converted request", flush=True)
    bi = list(rows)
    bi[4] = [list(x) for x in rows[4]]
    bi[4][5] = bi[4][5][:-1]
    with pytest.raises(RuntimeError, match="ragged"):
        ft.bs_tbs_gpu(t, 8, beams, bi, lps, -10.0, -40.0, 5.0, False)
    print("after the errors", flush=True)
    s, n, _, _ = ft.bs_tbs_gpu(t, 8, beams, rows, lps, -10.0, -40.0, 5.0, False)
    for i in range(8):
        want = o.tbs([10] * 8, ids[i], lp[i], -10.0, -40.0, 5.0, False)
        assert_same_results((s[i], n[i]), want, f"after the errors, {i}")


@pytest.mark.parametrize("early", [False, True])
def test_streamed_batches(ft, c1, early):
    # bs_tbs_gpu packs each request after the launch and the kernel picks it
    # up from host memory: batches of 8 mixing token-sorted rows with
    # shuffled ones (whose caller indices are staged), a final beam of 0, and
    # a request that fails to pack (withdrawn with the ones after it: the
    # call fails naming it, and the next call on the context works)
    t, o, ids, lp = c1
    rng = np.random.default_rng(11)
    for b0 in range(0, 64, 8):
        beams, bi, bl = [], [], []
        for i in range(8):
            r = b0 + i
            i2, l2 = ids[r], lp[r]
            if rng.integers(2):
                perm = np.stack([rng.permutation(32) for _ in range(8)])
                i2 = np.take_along_axis(i2, perm, 1)
                l2 = np.take_along_axis(l2, perm, 1)
            bw = [int(x) for x in rng.integers(1, 11, 8)]
            if i == 3 and b0 == 8:
                bw[-1] = 0
            beams.append(bw)
            bi.append(i2)
            bl.append(l2)
        print("streamed batch", b0, "early", early, flush=True)
        s, n, _, _ = ft.bs_tbs_gpu(t, 8, beams, [x.tolist() for x in bi],
                                   [x.tolist() for x in bl], -10.0, -40.0, 5.0, early)
        for i in range(8):
            if beams[i][-1] == 0:
                assert s[i] == [] and list(n[i]) == []
                continue
            want = o.tbs(beams[i], bi[i], bl[i], -10.0, -40.0, 5.0, early)
            assert_same_results((s[i], n[i]), want, f"streamed {b0}+{i}")
    rows = [ids[r].tolist() for r in range(8)]
    lps = [lp[r].tolist() for r in range(8)]
    lps[5] = lp[5].copy()
    lps[5][2, 7] = np.nan
    lps[5] = lps[5].tolist()
    with pytest.raises(RuntimeError, match="request 5: topk_logp holds NaN"):
        ft.bs_tbs_gpu(t, 8, [[10] * 8] * 8, rows, lps, -10.0, -40.0, 5.0, early)
    s, n, _, _ = ft.bs_tbs_gpu(t, 8, [[10] * 8] * 8, rows,
                               [lp[r].tolist() for r in range(8)], -10.0, -40.0, 5.0, early)
    for i in range(8):
        want = o.tbs([10] * 8, ids[i], lp[i], -10.0, -40.0, 5.0, early)
        assert_same_results((s[i], n[i]), want, f"after the withdrawn batch, {i}")


@pytest.mark.parametrize("head_rows", ["0", "3"])
def test_not_ready_requests_are_searched_again(ft, po, monkeypatch, head_rows):
    # The host packs 3 ms late and the kernel waits 1 us for a request's
    # rows: every leader (and helper 1, which copies the later rows) gives
    # up after its bounded wait and reports the request not ready, and the
    # host searches those requests again from the staged path.  The results
    # are the oracle's; the next call on the same context is sound.
    monkeypatch.setenv("FT_READY_TICKS", "100")
    monkeypatch.setenv("FT_PACK_DELAY_US", "3000")
    monkeypatch.setenv("FT_HEAD_ROWS", head_rows)
    toks, offs = ft.synth_keys(C1["n"], C1["vocab"], C1["lmin"], C1["lmax"],
                               C1["s"], C1["seed"])
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=8, topk=32, steps=8, beams=10,
                  inter=1024)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 16, C1["vocab"], 8, 32, 8, 0.3, 2.0, True, 0)
    for b0 in (0, 8):
        print("not-ready batch", b0, "head_rows", head_rows, flush=True)
        s, n, _, _ = ft.bs_tbs_gpu(t, 8, [[10] * 8] * 8, ids[b0:b0 + 8], lp[b0:b0 + 8],
                                   -10.0, -40.0, 5.0, b0 == 8)
        for i in range(8):
            want = o.tbs([10] * 8, ids[b0 + i], lp[b0 + i], -10.0, -40.0, 5.0, b0 == 8)
            assert_same_results((s[i], n[i]), want, f"not ready {b0}+{i}")
    got = ft.tbs(t, [10] * 8, ids[0], lp[0], -10.0, -40.0, 5.0, False, True)
    assert_same_results(got[:2], o.tbs([10] * 8, ids[0], lp[0], -10.0, -40.0, 5.0, False))


def test_history_limit_is_an_error(ft):
    toks, offs = ft.synth_keys(5000, 256, 3, 6, 1.1, 1)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    t.init_tbs_gpu(1, max_num_topk=32, max_num_outpos=6, max_num_out_beams=10,
                   max_num_out_tokens=60, max_num_inter_beams=12)
    ids, lp = ft.synth_requests(t, 0, 1, 256, 6, 32, 8, 0.3, 2.0, True, 0)
    with pytest.raises(RuntimeError, match="max_num_inter_beams"):
        ft.bs_tbs_gpu(t, 1, [[10] * 6], [ids[0].tolist()], [lp[0].tolist()],
                      -10, -40, 5, False)


def test_c2_scale_b100(ft, po):
    # 1M keys over a 256k vocabulary, beam 100, K 100, 12 steps
    toks, offs = ft.synth_keys(1000000, 262144, 4, 12, 1.1, 1)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=4, topk=100, steps=12,
                  beams=100, inter=4096)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 24, 262144, 12, 100, 50, 0.3, 2.0, True, 1)
    for b0 in range(0, 24, 4):
        got = ft.bs_tbs_gpu(t, 4, [[100] * 12] * 4,
                            [ids[b0 + i].tolist() for i in range(4)],
                            [lp[b0 + i].tolist() for i in range(4)],
                            -10.0, -40.0, 5.0, False)
        for i in range(4):
            want = o.tbs([100] * 12, ids[b0 + i], lp[b0 + i], -10.0, -40.0, 5.0,
                         False)
            assert_same_results((got[0][i], got[1][i]), want, f"C2 {b0 + i}")


def test_beam_1000(ft, po):
    toks, offs = ft.synth_keys(1000000, 262144, 3, 10, 1.05, 2)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=2, topk=1000, steps=10,
                  beams=1000, inter=16384)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 4, 262144, 10, 1000, 1000, 0.3, 2.5, True, 2)
    for r in range(4):
        got = ft.bs_tbs_gpu(t, 1, [[1000] * 10], [ids[r].tolist()],
                            [lp[r].tolist()], -10.0, -40.0, 5.0, False)
        want = o.tbs([1000] * 10, ids[r], lp[r], -10.0, -40.0, 5.0, False)
        assert_same_results((got[0][0], got[1][0]), want, f"B1000 {r}")


@pytest.mark.parametrize("scan_mult,wide_min,fp_max", [
    ("0", "0", "16"), ("0", "2", "16"), ("0", "2", "0"), ("999999", "512", "16"),
    ("1", "64", "16"), ("1", "64", "0")])
def test_lookup_modes(ft, po, monkeypatch, scan_mult, wide_min, fp_max):
    # scan_mult 0 sends every parent with children to the binary search
    # (wide_min 0) or the hash tables (wide_min 2); 999999 scans all.
    # fp_max 0 reads every hashed lookup's bucket (no fingerprint filter).
    monkeypatch.setenv("FT_SCAN_MULT", scan_mult)
    monkeypatch.setenv("FT_WIDE_MIN", wide_min)
    monkeypatch.setenv("FT_FP_MAX_LOG2", fp_max)
    toks, offs = ft.synth_keys(50000, 4096, 3, 8, 1.1, 4)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=4, topk=32, steps=8,
                  beams=16, inter=2048)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 24, 4096, 8, 32, 16, 0.3, 2.0, True, 4,
                                model=1)
    for b0 in range(0, 24, 4):
        got = ft.bs_tbs_gpu(t, 4, [[16] * 8] * 4,
                            [ids[b0 + i].tolist() for i in range(4)],
                            [lp[b0 + i].tolist() for i in range(4)],
                            -10.0, -40.0, 5.0, b0 % 8 == 4)
        for i in range(4):
            want = o.tbs([16] * 8, ids[b0 + i], lp[b0 + i], -10.0, -40.0, 5.0,
                         b0 % 8 == 4)
            assert_same_results((got[0][i], got[1][i]), want,
                                f"modes {scan_mult}/{wide_min}/{fp_max} req {b0 + i}")


@pytest.mark.parametrize("wgs,share_min", [("2", "0"), ("7", "0"), ("64", "0"),
                                           ("32", "100")])
def test_shared_steps(ft, po, monkeypatch, wgs, share_min):
    # steps expanded by a leader plus helper workgroups (share_min 0: every
    # step is shared), with ties and early exit
    monkeypatch.setenv("FT_WGS", wgs)
    monkeypatch.setenv("FT_SHARE_MIN", share_min)
    toks, offs = ft.synth_keys(80000, 8192, 3, 8, 1.1, 6)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=4, topk=64, steps=8,
                  beams=32, inter=4096)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 16, 8192, 8, 64, 32, 0.3, 2.0, True, 8,
                                model=1)
    for b0 in range(0, 16, 4):
        for alpha, early in ((5.0, False), (1e6, False), (5.0, True)):
            got = ft.bs_tbs_gpu(t, 4, [[32] * 8] * 4,
                                [ids[b0 + i].tolist() for i in range(4)],
                                [lp[b0 + i].tolist() for i in range(4)],
                                -10.0, -40.0, alpha, early)
            for i in range(4):
                want = o.tbs([32] * 8, ids[b0 + i], lp[b0 + i], -10.0, -40.0,
                             alpha, early)
                assert_same_results((got[0][i], got[1][i]), want,
                                    f"wgs {wgs} req {b0 + i} {alpha} {early}")


@pytest.mark.parametrize("wgs", ["2", "16"])
def test_leader_takes_over_unclaimed_slices(ft, po, monkeypatch, wgs):
    # helpers that never claim their slices of a shared step (a test knob):
    # after its grace period the leader takes every slice over and expands
    # it itself -- the step never waits for a workgroup that is not running
    monkeypatch.setenv("FT_WGS", wgs)
    monkeypatch.setenv("FT_SHARE_MIN", "0")
    monkeypatch.setenv("FT_TEST_NO_CLAIMS", "1")
    toks, offs = ft.synth_keys(40000, 4096, 3, 8, 1.1, 13)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=2, topk=64, steps=8,
                  beams=32, inter=4096)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 6, 4096, 8, 64, 32, 0.3, 2.0, True, 13,
                                model=1)
    for b0 in range(0, 6, 2):
        for early in (False, True):
            got = ft.bs_tbs_gpu(t, 2, [[32] * 8] * 2,
                                [ids[b0 + i].tolist() for i in range(2)],
                                [lp[b0 + i].tolist() for i in range(2)],
                                -10.0, -40.0, 5.0, early)
            for i in range(2):
                want = o.tbs([32] * 8, ids[b0 + i], lp[b0 + i], -10.0, -40.0,
                             5.0, early)
                assert_same_results((got[0][i], got[1][i]), want,
                                    f"no claims, wgs {wgs} req {b0 + i} {early}")


def test_fresh_contexts_shared_steps(ft, po, monkeypatch):
    # contexts created and destroyed one after another, every step shared: a
    # new workspace may sit on memory an earlier context used, so its control
    # words start cleared and launch epochs never repeat across contexts --
    # helpers act only on steps their own leader posts
    monkeypatch.setenv("FT_WGS", "16")
    monkeypatch.setenv("FT_SHARE_MIN", "0")
    toks, offs = ft.synth_keys(30000, 4096, 3, 8, 1.1, 9)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    shapes = [(4, 32, 16), (2, 64, 32), (4, 32, 16), (1, 16, 8), (3, 48, 24)]
    for rnd, (batch, topk, beams) in enumerate(shapes):
        print("fresh context", rnd, batch, topk, beams, flush=True)
        t = _gpu_trie(ft, toks=toks, offs=offs, batch=batch, topk=topk,
                      steps=8, beams=beams, inter=4096)
        ids, lp = ft.synth_requests(t, rnd, batch, 4096, 8, topk, beams, 0.3,
                                    2.0, True, 3, model=1)
        for early in (False, True):
            got = ft.bs_tbs_gpu(t, batch, [[beams] * 8] * batch,
                                [ids[i].tolist() for i in range(batch)],
                                [lp[i].tolist() for i in range(batch)],
                                -10.0, -40.0, 5.0, early)
            for i in range(batch):
                want = o.tbs([beams] * 8, ids[i], lp[i], -10.0, -40.0, 5.0, early)
                assert_same_results((got[0][i], got[1][i]), want,
                                    f"context {rnd} req {i} early {early}")
        del t


def test_trie_loaded_from_marisa_file(ft, po, tmp_path):
    # a MARISA trie.bin (num_tries 1, label order) loaded and searched on the
    # GPU: same node ids, so the same results as the oracle on the keys
    toks, offs = ft.synth_keys(60000, 300000, 2, 9, 1.1, 12)
    src = ft.Trie()
    src.build_arrays(toks, offs)
    p = str(tmp_path / "trie.bin")
    src.save_marisa(p)
    t = ft.Trie()
    t.load(p)
    t.init_tbs_gpu(4, max_num_topk=64, max_num_outpos=9, max_num_out_beams=32,
                   max_num_out_tokens=32 * 9, max_num_inter_beams=4096)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 8, 300000, 9, 64, 32, 0.3, 2.0, True, 6, model=1)
    for b0 in (0, 4):
        got = ft.bs_tbs_gpu(t, 4, [[32] * 9] * 4, [ids[b0 + i].tolist() for i in range(4)],
                            [lp[b0 + i].tolist() for i in range(4)], -10.0, -40.0, 5.0,
                            b0 == 4)
        for i in range(4):
            want = o.tbs([32] * 9, ids[b0 + i], lp[b0 + i], -10.0, -40.0, 5.0, b0 == 4)
            assert_same_results((got[0][i], got[1][i]), want, f"marisa file req {b0 + i}")


@pytest.mark.parametrize("alpha,early", [(0.0, False), (0.0, True), (5.0, False)])
def test_wide_tied_selection(ft, po, alpha, early):
    # 4096 proposals into a 6000-way root with three logp values: thousands
    # of equal norms share one histogram bin (more than the selection keeps
    # in LDS), so the boundary is narrowed bit by bit and the arrival-order
    # rule cuts the tie
    keys = []
    for t in range(6000):
        keys += [[t], [t, t % 3], [t, 1000 + t % 5, t % 7]]
    rng = np.random.default_rng(11)
    T, K = 3, 4096
    ids = np.stack([np.sort(rng.choice(6000, K, replace=False)),
                    np.arange(K), np.arange(K)]).astype(np.uint32)
    vals = np.array([-0.5, -1.0, -2.0], dtype=np.float32)
    lp = vals[rng.choice(3, (T, K), p=[0.01, 0.95, 0.04])]
    t = _gpu_trie(ft, keys=keys, batch=2, topk=K, steps=T, beams=3000,
                  inter=16384)
    o = po.OracleTrie.from_keys(keys)
    for beams in ([7, 7, 7], [2500, 3000, 40], [3000, 5, 3000]):
        print("wide tie", alpha, early, beams, flush=True)
        got = ft.bs_tbs_gpu(t, 1, [beams], [ids.tolist()], [lp.tolist()],
                            -10.0, -40.0, alpha, early)
        want = o.tbs(beams, ids, lp, -10.0, -40.0, alpha, early)
        assert_same_results((got[0][0], got[1][0]), want,
                            f"wide tie {alpha} {early} {beams}")


@pytest.mark.parametrize("early", [True, False])
def test_stress_long_keys_tight_thresholds(ft, po, early):
    # the stress shape at small scale: long keys (16-32 tokens), 32 steps,
    # tight thresholds (token -4, sentence -20) that reject most candidates,
    # early exit on and off, a batch of 8 in one launch
    toks, offs = ft.synth_keys(60000, 8192, 16, 32, 1.1, 12)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=8, topk=64, steps=32,
                  beams=48, inter=1 << 16)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 16, 8192, 32, 64, 48, 0.3, 2.0, True, 12,
                                model=1)
    # a final beam of 3: early exit cuts `selected` at its third push
    beams = [48] * 31 + [3]
    for b0 in range(0, 16, 8):
        print("stress batch", b0, early, flush=True)
        got = ft.bs_tbs_gpu(t, 8, [beams] * 8,
                            [ids[b0 + i].tolist() for i in range(8)],
                            [lp[b0 + i].tolist() for i in range(8)],
                            -4.0, -20.0, 5.0, early)
        for i in range(8):
            want = o.tbs(beams, ids[b0 + i], lp[b0 + i], -4.0, -20.0, 5.0,
                         early)
            assert_same_results((got[0][i], got[1][i]), want,
                                f"stress req {b0 + i} early={early}")
        assert any(len(s) for s in got[0]), "every stress request came back empty"


@pytest.mark.parametrize("K,mode", [(8192, "default"), (4097, "default"),
                                    (20000, "default"), (8192, "search"),
                                    (8192, "scan"), (8192, "shared")])
def test_rows_longer_than_lds(ft, po, monkeypatch, K, mode):
    # K above the 4096 proposals the LDS row holds: the row is searched where
    # it is staged.  A 32k-token vocabulary, so the wide root takes K hashed
    # lookups; "search" sends every parent to the binary search, "scan" scans
    # every child, "shared" spreads every step over 7 workgroups.  Streamed
    # batches with shuffled rows (staged caller indices), logps rounded to
    # halves (ties cut by arrival order) and early exit; then the staged path.
    if mode == "search":
        monkeypatch.setenv("FT_SCAN_MULT", "0")
        monkeypatch.setenv("FT_WIDE_MIN", "0")
    elif mode == "scan":
        monkeypatch.setenv("FT_SCAN_MULT", "999999")
    elif mode == "shared":
        monkeypatch.setenv("FT_WGS", "7")
        monkeypatch.setenv("FT_SHARE_MIN", "0")
    V, T, B = 32768, 5, 48
    toks, offs = ft.synth_keys(150000, V, 3, 7, 1.1, 21)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=4, topk=K, steps=T, beams=B,
                  inter=4096)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 8, V, T, K, B, 0.3, 2.0, True, 21, model=1)
    lp = np.round(lp * 2.0) / 2.0
    rng = np.random.default_rng(K)
    for r in range(0, 8, 3):
        perm = np.stack([rng.permutation(K) for _ in range(T)])
        ids[r] = np.take_along_axis(ids[r], perm, 1)
        lp[r] = np.take_along_axis(lp[r], perm, 1)
    beams = [B] * (T - 1) + [12]
    for b0 in (0, 4):
        early = b0 == 4
        print("long rows", K, mode, "batch", b0, flush=True)
        got = ft.bs_tbs_gpu(t, 4, [beams] * 4, ids[b0:b0 + 4], lp[b0:b0 + 4],
                            -10.0, -40.0, 5.0, early)
        for i in range(4):
            want = o.tbs(beams, ids[b0 + i], lp[b0 + i], -10.0, -40.0, 5.0, early)
            assert_same_results((got[0][i], got[1][i]), want,
                                f"K {K} {mode} req {b0 + i} early={early}")
        assert any(len(x) for x in got[0])
    ft.stage(t, np.full((4, T), B, np.uint32), ids[:4], lp[:4], -10.0, -40.0, 5.0, False)
    ft.launch(t)
    count, norms, lens, tk, _ = ft.fetch(t)
    for i in range(4):
        want = o.tbs([B] * T, ids[i], lp[i], -10.0, -40.0, 5.0, False)
        n = int(count[i])
        assert_same_results(([tk[i, j, :lens[i, j]].tolist() for j in range(n)],
                             norms[i, :n]), want, f"K {K} {mode} staged {i}")


def test_louds_child_index_is_switched_off(ft, monkeypatch):
    monkeypatch.setenv("FT_CHILD_INDEX", "louds")
    t = ft.Trie()
    t.build([[1, 2], [3]])
    with pytest.raises(RuntimeError, match="switched off"):
        t.init_tbs_gpu(1, max_num_topk=4, max_num_outpos=2, max_num_out_beams=2,
                       max_num_out_tokens=4, max_num_inter_beams=8)


@pytest.mark.parametrize("root_dir,scan_mult,wide_min", [
    ("force", "2", "64"), ("force", "0", "2"), ("force", "999999", "512"),
    ("0", "2", "64"), ("0", "0", "2")])
def test_root_directory(ft, po, monkeypatch, root_dir, scan_mult, wide_min):
    # Step 0 looks the root's children up in the token-indexed root
    # directory (forced here for a scanned root too) and builds step 1's
    # parent table from it -- for children that are scanned, searched,
    # hashed and link parents alike -- or, with FT_ROOT_DIR=0, from the
    # node records and tables as every later step does.  Both equal the
    # oracle, on tiny tries with ties and on a wider one.
    monkeypatch.setenv("FT_ROOT_DIR", root_dir)
    monkeypatch.setenv("FT_SCAN_MULT", scan_mult)
    monkeypatch.setenv("FT_WIDE_MIN", wide_min)
    rng = np.random.default_rng(11)
    for case in range(30):
        vocab = int(rng.integers(2, 10))
        keys = sorted({tuple(rng.integers(0, vocab, int(rng.integers(1, 7))))
                       for _ in range(int(rng.integers(1, 40)))})
        keys = [list(map(int, k)) for k in keys]
        T = int(rng.integers(1, 8))
        K = int(rng.integers(1, vocab + 1))
        ids = np.stack([np.sort(rng.choice(vocab, K, replace=False))
                        for _ in range(T)]).astype(np.uint32)
        lp = (-rng.integers(0, 8, (T, K)) * 0.5).astype(np.float32)
        beams = [int(rng.integers(1, 6)) for _ in range(T)]
        early = bool(rng.integers(0, 2))
        print("root directory", root_dir, scan_mult, wide_min, "tiny case", case, flush=True)
        t = _gpu_trie(ft, keys=keys, batch=1, topk=16, steps=8, beams=8)
        got = ft.bs_tbs_gpu(t, 1, [beams], [ids.tolist()], [lp.tolist()],
                            -3.0, -9.0, 1.0, early)
        want = po.OracleTrie.from_keys(keys).tbs(beams, ids, lp, -3.0, -9.0, 1.0, early)
        assert_same_results((got[0][0], got[1][0]), want, f"tiny case {case}")
    toks, offs = ft.synth_keys(50000, 4096, 3, 8, 1.1, 5)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=4, topk=32, steps=8,
                  beams=16, inter=2048)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 16, 4096, 8, 32, 16, 0.3, 2.0, True, 5, model=1)
    for b0 in range(0, 16, 4):
        print("root directory", root_dir, scan_mult, wide_min, "requests", b0, flush=True)
        got = ft.bs_tbs_gpu(t, 4, [[16] * 8] * 4,
                            [ids[b0 + i].tolist() for i in range(4)],
                            [lp[b0 + i].tolist() for i in range(4)],
                            -10.0, -40.0, 5.0, b0 == 8)
        for i in range(4):
            want = o.tbs([16] * 8, ids[b0 + i], lp[b0 + i], -10.0, -40.0, 5.0, b0 == 8)
            assert_same_results((got[0][i], got[1][i]), want, f"request {b0 + i}")


def test_root_tokens_beyond_the_directory(ft, po):
    # a root child token of 2^25 or more: no root directory, the root's
    # table or search as before
    keys = [[1, 2], [1, 3], [5], [(1 << 25) + 7, 2], [(1 << 30), 4, 4]]
    t = _gpu_trie(ft, keys=keys, batch=1, topk=4, steps=3, beams=4)
    ids = np.array([[1, 5, (1 << 25) + 7, 1 << 30], [2, 3, 4, 9], [4, 5, 6, 7]], np.uint32)
    lp = np.array([[-0.5, -1.0, -0.25, -2.0], [-0.1, -0.2, -0.3, -0.4],
                   [-1.0, -1.5, -2.0, -2.5]], np.float32)
    for early in (False, True):
        print("large root tokens, early", early, flush=True)
        got = ft.bs_tbs_gpu(t, 1, [[4, 4, 4]], [ids.tolist()], [lp.tolist()],
                            -10.0, -40.0, 1.0, early)
        want = po.OracleTrie.from_keys(keys).tbs([4, 4, 4], ids, lp, -10.0, -40.0, 1.0, early)
        assert_same_results((got[0][0], got[1][0]), want, f"early {early}")


def test_topk_limit(ft):
    t = ft.Trie()
    t.build([[1], [2]])
    t.init_tbs_gpu(1, max_num_topk=65535, max_num_outpos=2, max_num_out_beams=2,
                   max_num_out_tokens=4, max_num_inter_beams=8)
    with pytest.raises(RuntimeError, match="65535"):
        t.init_tbs_gpu(1, max_num_topk=65536, max_num_outpos=2, max_num_out_beams=2,
                       max_num_out_tokens=4, max_num_inter_beams=8)


@pytest.mark.skip(reason="the LOUDS child-index kernel faulted the GPU once (tiny tries, "
                         "after the long-row tests) and the cause is not found; "
                         "FT_CHILD_INDEX=louds is switched off until it is")
def test_louds_child_index(ft, po, monkeypatch):
    # child ranges from the LOUDS rank/select directory (FT_CHILD_INDEX=louds)
    # instead of the node records: tiny random tries, a 50k-key trie in
    # batches, and a 6000-way root (zeros far apart around its run of ones)
    monkeypatch.setenv("FT_CHILD_INDEX", "louds")
    rng = np.random.default_rng(17)
    for case in range(40):
        vocab = int(rng.integers(2, 10))
        keys = sorted({tuple(rng.integers(0, vocab, int(rng.integers(1, 7))))
                       for _ in range(int(rng.integers(1, 40)))})
        keys = [list(map(int, k)) for k in keys]
        T, K = int(rng.integers(1, 8)), int(rng.integers(1, vocab + 1))
        ids = np.stack([np.sort(rng.choice(vocab, K, replace=False))
                        for _ in range(T)]).astype(np.uint32)
        lp = (-rng.integers(0, 8, (T, K)) * 0.5).astype(np.float32)
        beams = [int(rng.integers(1, 6)) for _ in range(T)]
        t = _gpu_trie(ft, keys=keys, batch=1, topk=16, steps=8, beams=8)
        got = ft.bs_tbs_gpu(t, 1, [beams], [ids.tolist()], [lp.tolist()],
                            -3.0, -9.0, 5.0, False)
        want = po.OracleTrie.from_keys(keys).tbs(beams, ids, lp, -3.0, -9.0, 5.0, False)
        assert_same_results((got[0][0], got[1][0]), want, f"louds tiny {case}")
    toks, offs = ft.synth_keys(50000, 4096, 3, 8, 1.1, 4)
    t = _gpu_trie(ft, toks=toks, offs=offs, batch=4, topk=32, steps=8, beams=16,
                  inter=2048)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 16, 4096, 8, 32, 16, 0.3, 2.0, True, 4, model=1)
    for b0 in range(0, 16, 4):
        got = ft.bs_tbs_gpu(t, 4, [[16] * 8] * 4, [ids[b0 + i].tolist() for i in range(4)],
                            [lp[b0 + i].tolist() for i in range(4)], -10.0, -40.0, 5.0, False)
        for i in range(4):
            want = o.tbs([16] * 8, ids[b0 + i], lp[b0 + i], -10.0, -40.0, 5.0, False)
            assert_same_results((got[0][i], got[1][i]), want, f"louds 50k {b0 + i}")
    keys = []
    for k in range(6000):
        keys += [[k], [k, k % 3], [k, 1000 + k % 5, k % 7]]
    t = _gpu_trie(ft, keys=keys, batch=1, topk=4096, steps=3, beams=3000, inter=16384)
    o = po.OracleTrie.from_keys(keys)
    ids = np.stack([np.sort(rng.choice(6000, 4096, replace=False)),
                    np.arange(4096), np.arange(4096)]).astype(np.uint32)
    lp = np.array([-0.5, -1.0, -2.0], dtype=np.float32)[rng.choice(3, (3, 4096))]
    got = ft.bs_tbs_gpu(t, 1, [[2500, 3000, 40]], [ids.tolist()], [lp.tolist()],
                        -10.0, -40.0, 5.0, False)
    want = o.tbs([2500, 3000, 40], ids, lp, -10.0, -40.0, 5.0, False)
    assert_same_results((got[0][0], got[1][0]), want, "louds wide root")
