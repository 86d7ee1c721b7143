"""C2 at its full size: 10M keys over a 256k vocabulary (key length 4-12,
Zipf(1.1)), beam = K = 100, 12 steps, 1,000 seeded requests, searched at
batch 1 (bs_tbs_gpu) and at batch 8 (numpy batches) and compared bit for bit
with the CPU oracle on the same image (louds-trie.cc:75-177).

Proposal rows: the softmax model of the configuration (log-softmax of
N(0, 2^2) logits) with 30% of the mass on 100 seeded key paths -- with no
forced mass, K = 100 random tokens of 256k almost never continue a key and
every search would stop at step 0."""

import pytest

import workloads as wl
from scale_common import check_bs_tbs_gpu, check_numpy_batches, oracle_all, result_stats

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def c2(ft, po):
    print("building the C2 trie (10M keys)", flush=True)
    t = wl.trie(ft, "c2")
    t.init_tbs_gpu(8, max_num_topk=100, max_num_outpos=12, max_num_out_beams=100,
                   max_num_out_tokens=1200, max_num_inter_beams=1200)
    ids, lp = ft.synth_requests(t, 0, 1000, wl.VOCAB["c2"], 12, 100, 100, 0.3, 2.0,
                                True, 0, model=0)
    import numpy as np
    beams = np.full((1000, 12), 100, dtype=np.uint32)
    want = oracle_all(po.OracleTrie.from_trie(t), beams, ids, lp, wl.RULES["c2"])
    print("C2 oracle:", result_stats(want), flush=True)
    yield t, beams, ids, lp, want
    t.clear()


def test_c2_batch1_1000_requests(ft, c2):
    t, beams, ids, lp, want = c2
    nonempty = check_bs_tbs_gpu(ft, t, beams, ids, lp, wl.RULES["c2"], want, 1, "C2 b1")
    assert nonempty > 900


def test_c2_batch8_1000_requests(ft, c2):
    t, beams, ids, lp, want = c2
    check_numpy_batches(ft, t, beams, ids, lp, wl.RULES["c2"], want, 8, "C2 b8")
