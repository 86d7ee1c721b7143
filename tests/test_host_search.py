"""flashtrie.tbs(use_gpu=False) -- the library's host implementation of the
search -- against the oracle on seeded workloads, edge cases and errors."""

import numpy as np
import pytest

from helpers import assert_same_results, load_golden

KA = load_golden("known_answers.json")


@pytest.mark.parametrize("case", KA, ids=[c["name"] for c in KA])
def test_known_answers(ft, case):
    t = ft.Trie()
    t.build(case["keys"])
    sents, norms, _ = ft.tbs(t, case["beams"], case["topk_id"],
                             case["topk_logp"], case["token_logp_threshold"],
                             case["sents_logp_threshold"], case["length_norm"],
                             case["early_exit"], False)
    assert sents == case["expect_sents"]
    assert np.allclose(norms, case["expect_scores_approx"], rtol=1e-6, atol=0)


@pytest.fixture(scope="module")
def c1_like(ft, po):
    toks, offs = ft.synth_keys(20000, 2048, 3, 8, 1.1, 5)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    return t, po.OracleTrie.from_keys(toks=toks, offs=offs)


@pytest.mark.parametrize("early", [False, True])
@pytest.mark.parametrize("alpha", [0.0, 5.0, 1e6])
def test_matches_oracle(ft, c1_like, early, alpha):
    t, o = c1_like
    T, K = 8, 32
    ids, lp = ft.synth_requests(t, 0, 30, 2048, T, K, 8, 0.3, 2.0, True, 3)
    for r in range(30):
        beams = [10] * T
        got = ft.tbs(t, beams, ids[r].tolist(), lp[r].tolist(), -10.0, -40.0,
                     alpha, early, False)
        want = o.tbs(beams, ids[r], lp[r], -10.0, -40.0, alpha, early)
        assert_same_results(got[:2], want, f"request {r}")


def test_unsorted_rows(ft, c1_like):
    t, o = c1_like
    ids, lp = ft.synth_requests(t, 100, 10, 2048, 6, 32, 8, 0.3, 2.0, True, 3)
    rng = np.random.default_rng(0)
    for r in range(10):
        perm = np.stack([rng.permutation(32) for _ in range(6)])
        i2 = np.take_along_axis(ids[r], perm, 1)
        l2 = np.take_along_axis(lp[r], perm, 1)
        got = ft.tbs(t, [7] * 6, i2.tolist(), l2.tolist(), -10, -40, 5, False, False)
        want = o.tbs([7] * 6, i2, l2, -10, -40, 5, False)
        assert_same_results(got[:2], want)


def test_errors(ft):
    t = ft.Trie()
    t.build([[1], [2]])
    with pytest.raises(RuntimeError, match="empty"):
        ft.tbs(t, [], [[1]], [[-1.0]], -10, -40, 5, False, False)
    with pytest.raises(RuntimeError, match="ragged"):
        ft.tbs(t, [2, 2], [[1, 2], [1]], [[-1.0, -1.0], [-1.0]], -10, -40, 5,
               False, False)
    with pytest.raises(RuntimeError, match="beam width 0"):
        ft.tbs(t, [0, 2], [[1], [2]], [[-1.0], [-1.0]], -10, -40, 5, False, False)
    # final beam 0: outputs untouched (empty here)
    assert ft.tbs(t, [2, 0], [[1], [2]], [[-1.0], [-1.0]], -10, -40, 5, False,
                  False)[:2] == ([], [])
