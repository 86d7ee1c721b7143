"""C5 at full size: the stress trie (200M keys over a 2.2M-token vocabulary,
every token a child of the root, keys of 16-32 tokens), beam = K = 1000, 32
steps, thresholds -4 / -20 so that most candidates fail, early exit on,
batch 8 -- plus the same requests without early exit -- compared bit for
bit with the CPU oracle on the same image (louds-trie.cc:75-177, early exit
at :81-83)."""

import numpy as np
import pytest

import workloads as wl
from scale_common import check_numpy_batches, oracle_all, result_stats

pytestmark = pytest.mark.gpu
N = 64


@pytest.fixture(scope="module")
def stress(ft, po):
    print("building the stress trie (200M keys)", flush=True)
    t = wl.trie(ft, "stress")
    t.init_tbs_gpu(8, max_num_topk=1000, max_num_outpos=32, max_num_out_beams=1000,
                   max_num_out_tokens=32000, max_num_inter_beams=32000)
    beams, ids, lp = wl.requests(ft, t, "stress", "example", 0, N, 1000)
    yield t, po.OracleTrie.from_trie(t), beams, ids, lp
    t.clear()


@pytest.mark.parametrize("early", [True, False])
def test_c5_stress_batch8(ft, stress, early):
    t, ot, beams, ids, lp = stress
    tok, sent, alpha, _ = wl.RULES["stress"]
    rules = (tok, sent, alpha, early)
    want = oracle_all(ot, beams, ids, lp, rules)
    print("C5 early", early, "oracle:", result_stats(want), flush=True)
    assert sum(len(w[0]) > 0 for w in want) > N // 2
    check_numpy_batches(ft, t, beams, ids, lp, rules, want, 8, f"C5 early={early}")


def test_c5_final_beam_cut_by_early_exit(ft, stress):
    # a final beam of 5: early exit stops at the fifth selected push
    t, ot, beams, ids, lp = stress
    b5 = beams.copy()
    b5[:, -1] = 5
    want = oracle_all(ot, b5[:16], ids[:16], lp[:16], wl.RULES["stress"])
    assert all(len(w[0]) <= 5 for w in want)
    check_numpy_batches(ft, t, b5[:16], ids[:16], lp[:16], wl.RULES["stress"], want, 8,
                        "C5 final beam 5")
    assert np.array_equal(b5[:, :-1], beams[:, :-1])
