"""C3 and C4 at full size: the paper trie (800,000,000 unique keys over a
2.2M-token vocabulary, key length 3-16, Zipf(1.05)), 16 steps, K = beam,
thresholds -10 / -40, alpha 5.  64 seeded requests per beam width (100, 500,
1000) and proposal model (the reference example's shape, and the stated
softmax model with 30% of the mass on one key path), searched at batch 1
through bs_tbs_gpu (C3) and at batch 8 in numpy batches (C4), each compared
bit for bit with the CPU oracle on the same image (louds-trie.cc:75-177)."""

import pytest

import workloads as wl
from scale_common import check_bs_tbs_gpu, check_numpy_batches, oracle_all, result_stats

pytestmark = pytest.mark.gpu

CASES = [(model, beam) for model in ("example", "literal") for beam in (100, 500, 1000)]
N = 64


@pytest.fixture(scope="module")
def paper(ft, po):
    print("building the paper trie (800M unique keys)", flush=True)
    t = wl.trie(ft, "paper")
    assert t.num_keys() == wl.PAPER_KEYS
    t.init_tbs_gpu(8, max_num_topk=1000, max_num_outpos=16, max_num_out_beams=1000,
                   max_num_out_tokens=16000, max_num_inter_beams=16000)
    ot = po.OracleTrie.from_trie(t)
    cases = {}
    for model, beam in CASES:
        beams, ids, lp = wl.requests(ft, t, "paper", model, 7000 * beam, N, beam)
        want = oracle_all(ot, beams, ids, lp, wl.RULES["paper"])
        print(f"paper {model} beam {beam} oracle:", result_stats(want), flush=True)
        cases[(model, beam)] = (beams, ids, lp, want)
    yield t, cases
    t.clear()


@pytest.mark.parametrize("model,beam", CASES)
def test_c3_paper_batch1(ft, paper, model, beam):
    t, cases = paper
    beams, ids, lp, want = cases[(model, beam)]
    print("C3", model, beam, flush=True)
    check_bs_tbs_gpu(ft, t, beams, ids, lp, wl.RULES["paper"], want, 1,
                     f"C3 {model} beam {beam}")


@pytest.mark.parametrize("model,beam", CASES)
def test_c4_paper_batch8(ft, paper, model, beam):
    t, cases = paper
    beams, ids, lp, want = cases[(model, beam)]
    print("C4", model, beam, flush=True)
    check_numpy_batches(ft, t, beams, ids, lp, wl.RULES["paper"], want, 8,
                        f"C4 {model} beam {beam}")
