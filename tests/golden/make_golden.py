"""Writes the golden fixtures under tests/golden/.

known_answers.json -- hand-derived cases.  Every expected output below was
worked out by reading the reference CPU path (not by running any code):
LoudsTrie::tbs / tbs_lookup_ (lib/marisa/grimoire/trie/louds-trie.cc:75-177),
the bounded heap Candidates::push / pop (lib/marisa/grimoire/trie/
candidates.h:16-80) and Agent::logp_norm (include/marisa/agent.h:69-72).

oracle_regression.json -- small random cases with the oracle's outputs, kept
to catch regressions in the oracle itself (they pin nothing on their own).

Run: python tests/golden/make_golden.py
"""

import json
import math
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def ka_cases():
    cases = []
    # KA-1, the link quirk.  node1 is a non-terminal link [1,2,3] with
    # children 4 and 5.  Entering node1 consumes only token 1; the next step
    # looks up a child of node1 (skipping 2,3), and the terminal child then
    # replays KB = [1,2,3,4] from position |Q| = 2, i.e. tokens 3 then 4.
    lp = [[-3.0] * 6 for _ in range(4)]
    col = {1: 0, 2: 1, 3: 2, 4: 3, 5: 4, 7: 5}
    for t, d in enumerate([{1: -0.5, 7: -1.0}, {2: -0.5, 4: -0.6, 5: -0.9},
                           {3: -0.5, 4: -0.7}, {4: -0.5, 5: -0.8}]):
        for tok, v in d.items():
            lp[t][col[tok]] = v
    cases.append({
        "name": "KA-1 link quirk",
        "keys": [[1, 2, 3, 4], [1, 2, 3, 5], [7]],
        "beams": [10, 10, 10, 10],
        "topk_id": [[1, 2, 3, 4, 5, 7]] * 4,
        "topk_logp": lp,
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 0.0, "early_exit": False,
        # f32 logps summed in f64
        "expect_sents": [[1, 5, 3, 5], [1, 4, 3, 4], [7]],
        "expect_scores_approx": [-2.7, -2.1, -1.0],
        "expect_trie": {
            "child_begin": [1, 3, 5, 5, 5, 5],
            "edges": [[], [1, 2, 3], [7], [4], [5]],
            "terminal": [0, 0, 1, 1, 1],
        },
    })
    # KA-2, early exit fires inside the step at the push that fills
    # `selected` (louds-trie.cc:81-83): [1] and [2] are pushed, [3] never is.
    cases.append({
        "name": "KA-2 early exit",
        "keys": [[1], [2], [3]],
        "beams": [2], "topk_id": [[1, 2, 3]], "topk_logp": [[-3.0, -1.0, -2.0]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 0.0, "early_exit": True,
        "expect_sents": [[1], [2]], "expect_scores_approx": [-3.0, -1.0],
    })
    # KA-2b, same without early exit: the bounded heap keeps the best two.
    cases.append({
        "name": "KA-2b no early exit",
        "keys": [[1], [2], [3]],
        "beams": [2], "topk_id": [[1, 2, 3]], "topk_logp": [[-3.0, -1.0, -2.0]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 0.0, "early_exit": False,
        "expect_sents": [[3], [2]], "expect_scores_approx": [-2.0, -1.0],
    })
    # KA-3, no proposal matches: empty output.
    cases.append({
        "name": "KA-3 no match",
        "keys": [[1], [2]],
        "beams": [4], "topk_id": [[5, 6]], "topk_logp": [[-1.0, -1.0]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 5.0, "early_exit": False,
        "expect_sents": [], "expect_scores_approx": [],
    })
    # KA-4, length norm: d = 1 gives factor 1 for any alpha; d = 2 gives
    # (6/7)^alpha.  [5] -> -1.0 ; [5,6] -> -1.5 * (6/7)^5.
    cases.append({
        "name": "KA-4 length norm",
        "keys": [[5], [5, 6]],
        "beams": [10, 10], "topk_id": [[5], [6]], "topk_logp": [[-1.0], [-0.5]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 5.0, "early_exit": False,
        "expect_sents": [[5], [5, 6]],
        "expect_scores_approx": [-1.0, -1.5 * math.pow(6.0 / 7.0, 5.0)],
    })
    # KA-5, tie at capacity 1: [1] is pushed first; [2] and [3] have the
    # same norm, which is not > top, so they are rejected (candidates.h:50-55).
    cases.append({
        "name": "KA-5 tie rejected",
        "keys": [[1], [2], [3]],
        "beams": [1], "topk_id": [[1, 2, 3]], "topk_logp": [[-1.0, -1.0, -1.0]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 0.0, "early_exit": False,
        "expect_sents": [[1]], "expect_scores_approx": [-1.0],
    })
    # KA-6, tie with eviction at capacity 2: heap {[1],[2]} (both -1), then
    # [3] (-0.5) enters and the worst -- equal norm, smaller node id -- is
    # evicted: [1] (node 1) goes, [2] (node 2) stays.
    cases.append({
        "name": "KA-6 tie evicts smaller node id",
        "keys": [[1], [2], [3]],
        "beams": [2], "topk_id": [[1, 2, 3]], "topk_logp": [[-1.0, -1.0, -0.5]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 0.0, "early_exit": False,
        "expect_sents": [[2], [3]], "expect_scores_approx": [-1.0, -0.5],
    })
    # KA-7, arrival order decides: unsorted row [1,3,2].  Heap {[1], [3]}
    # is full when [2] (-1, equal to the worst) arrives and is rejected.
    cases.append({
        "name": "KA-7 late tie rejected",
        "keys": [[1], [2], [3]],
        "beams": [2], "topk_id": [[1, 3, 2]], "topk_logp": [[-1.0, -0.5, -1.0]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 0.0, "early_exit": False,
        "expect_sents": [[1], [3]], "expect_scores_approx": [-1.0, -0.5],
    })
    # KA-8, output order among equal norms is ascending node id
    # (louds-trie.cc:168-176 pops the worst first).
    cases.append({
        "name": "KA-8 output tie order",
        "keys": [[1], [2]],
        "beams": [2], "topk_id": [[2, 1]], "topk_logp": [[-1.0, -1.0]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 0.0, "early_exit": False,
        "expect_sents": [[1], [2]], "expect_scores_approx": [-1.0, -1.0],
    })
    # KA-9, thresholds: token threshold is `<=` (a logp equal to it is
    # dropped) and the sentence threshold applies to the running sum.
    cases.append({
        "name": "KA-9 thresholds",
        "keys": [[1, 2], [3, 4], [5]],
        "beams": [10, 10], "topk_id": [[1, 3, 5], [2, 4, 6]],
        "topk_logp": [[-2.0, -1.0, -4.0], [-3.5, -2.0, -1.0]],
        "token_logp_threshold": -4.0, "sents_logp_threshold": -5.0,
        "length_norm": 0.0, "early_exit": False,
        # [5]: -4 <= -4 dropped.  [1,2]: -2 + -3.5 = -5.5 <= -5 dropped.
        # [3,4]: -1 + -2 = -3 kept.
        "expect_sents": [[3, 4]], "expect_scores_approx": [-3.0],
    })
    # KA-10, a terminal link leaf consumes its tail one token per step and
    # is selected only when the whole tail is consumed.
    cases.append({
        "name": "KA-10 terminal link",
        "keys": [[8, 9, 10], [11]],
        "beams": [5, 5, 5], "topk_id": [[8, 11], [9, 12], [10, 13]],
        "topk_logp": [[-1.0, -2.0], [-1.0, -1.0], [-1.0, -1.0]],
        "token_logp_threshold": -10.0, "sents_logp_threshold": -40.0,
        "length_norm": 0.0, "early_exit": False,
        "expect_sents": [[8, 9, 10], [11]], "expect_scores_approx": [-3.0, -2.0],
    })
    return cases


def regression_cases():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)),
                                    "oracle"))
    import numpy as np
    import pyoracle
    rng = np.random.default_rng(2024)
    out = []
    for i in range(12):
        vocab = int(rng.integers(3, 12))
        nkeys = int(rng.integers(2, 30))
        keys = sorted({tuple(rng.integers(0, vocab, int(rng.integers(1, 6))))
                       for _ in range(nkeys)})
        keys = [list(map(int, k)) for k in keys]
        T = int(rng.integers(1, 7))
        K = int(rng.integers(1, vocab + 1))
        ids = np.stack([np.sort(rng.choice(vocab, K, replace=False))
                        for _ in range(T)]).astype(np.uint32)
        lp = (-rng.random((T, K)) * 4).astype(np.float32)
        beams = [int(rng.integers(1, 6)) for _ in range(T)]
        ee = bool(rng.integers(0, 2))
        alpha = float(rng.choice([0.0, 1.0, 5.0]))
        tr = pyoracle.OracleTrie.from_keys(keys)
        sents, norms = tr.tbs(beams, ids, lp, -3.5, -9.0, alpha, ee)
        out.append({"keys": keys, "beams": beams, "topk_id": ids.tolist(),
                    "topk_logp": lp.tolist(), "token_logp_threshold": -3.5,
                    "sents_logp_threshold": -9.0, "length_norm": alpha,
                    "early_exit": ee, "expect_sents": sents,
                    "expect_norms_hex": [float(x).hex() for x in norms]})
    return out


def main():
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(ka_cases(), f, indent=1)
    with open(os.path.join(HERE, "oracle_regression.json"), "w") as f:
        json.dump(regression_cases(), f)
    print("wrote known_answers.json, oracle_regression.json")


if __name__ == "__main__":
    main()
