"""The synthetic workloads the benchmark and the full-size parity tests run:
tries and seeded proposal rows, with their sizes in one place.

* c1     100k keys over a 32k vocabulary, length 3-8, Zipf(1.1); beam 10,
         K = 32, 8 steps (the CPU plumbing configuration)
* c2     10M keys over a 256k vocabulary, length 4-12, Zipf(1.1); beam =
         K = 100, 12 steps
* paper  800,000,000 unique keys over a 2.2M vocabulary, length 3-16 (mean
         ~6), Zipf(1.05) prefix sharing; beams 100 / 500 / 1000 with K =
         beam, 16 steps
* stress 200M keys over a 2.2M vocabulary (every token is a root child),
         length 16-32; beam = K = 1000, 32 steps, early exit, thresholds
         -4 / -20

Proposal models: "example" is the shape of the reference's example
generator (examples/make_example_data.py:119-145): as many seeded key paths
as the beam is wide, forced tokens U(-2.2, -0.2), distractors U(-12, -4);
"literal" is the configuration as stated: log-softmax of N(0, sigma^2)
logits over the whole vocabulary (its log-partition taken analytically)
with 30% of the mass on one seeded key path.
"""

import numpy as np

# The paper trie: this many independent key draws give 799,489,109 unique
# keys (the rest are duplicates); the trie is topped up to exactly
# PAPER_KEYS with prefix keys (internal nodes of depth >= 3 made terminal,
# 0.064% of the keys).
PAPER_KEYS = 800_000_000
PAPER_DRAWS = 845_450_000
PAPER_VOCAB = 2_200_000
STRESS_KEYS = 200_000_000

# token / sentence log-prob thresholds, length-norm alpha, early exit
RULES = {"c1": (-10.0, -40.0, 5.0, False), "c2": (-10.0, -40.0, 5.0, False),
         "paper": (-10.0, -40.0, 5.0, False), "stress": (-4.0, -20.0, 5.0, True)}
STEPS = {"c1": 8, "c2": 12, "paper": 16, "stress": 32}
VOCAB = {"c1": 32768, "c2": 262144, "paper": PAPER_VOCAB, "stress": PAPER_VOCAB}
SIGMA = {"c1": 2.0, "c2": 2.0, "paper": 2.5, "stress": 2.5}


def trie(ft, name):
    """A new flashtrie.Trie holding the workload's trie."""
    t = ft.Trie()
    if name == "c1":
        toks, offs = ft.synth_keys(100_000, 32768, 3, 8, 1.1, 0)
        t.build_arrays(toks, offs)
    elif name == "c2":
        toks, offs = ft.synth_keys(10_000_000, 262144, 4, 12, 1.1, 0)
        t.build_arrays(toks, offs)
    elif name == "paper":
        ft.synth_paper_trie(t, PAPER_DRAWS, PAPER_VOCAB, 1.05, 0,
                            unique_keys=PAPER_KEYS)
    elif name == "stress":
        ft.synth_paper_trie(t, STRESS_KEYS, PAPER_VOCAB, 1.05, 1, lmin=16,
                            lmax=32, p_end=0.25)
    else:
        raise ValueError(name)
    return t


def requests(ft, t, name, model, first, n, beam, topk=None):
    """Seeded requests [first, first + n) of the workload: beams [n][T] (all
    `beam`), ids and logp [n][T][K] (K = topk, default the beam), rows in
    ascending token order."""
    T, V, K = STEPS[name], VOCAB[name], topk or beam
    if model == "literal":
        ids, lp = ft.synth_requests(t, first, n, V, T, K, 1, 0.3, SIGMA[name],
                                    True, 0, model=0)
    elif model == "example":
        ids, lp = ft.synth_requests(t, first, n, V, T, K, beam, 0.3, SIGMA[name],
                                    True, 0, model=1)
    else:
        raise ValueError(model)
    return np.full((n, T), beam, dtype=np.uint32), ids, lp
