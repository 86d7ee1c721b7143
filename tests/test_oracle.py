"""Pins the CPU oracle (oracle/oracle.cc) before anything is compared to it.

* hand-derived known answers (tests/golden/known_answers.json);
* brute-force enumeration of the admissible keys on tiny tries where no
  pruning happens and no link node has children;
* structural invariants of the restated MARISA build;
* the two oracle variants (as-written cost model / fast) agree.
"""

import itertools
import math

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st, HealthCheck

from helpers import load_golden, oracle_logical

KA = load_golden("known_answers.json")


@pytest.mark.parametrize("case", KA, ids=[c["name"] for c in KA])
@pytest.mark.parametrize("variant", [0, 1])
def test_known_answers(po, case, variant):
    tr = po.OracleTrie.from_keys(case["keys"])
    sents, norms = tr.tbs(case["beams"], np.array(case["topk_id"]),
                          np.array(case["topk_logp"], dtype=np.float32),
                          case["token_logp_threshold"],
                          case["sents_logp_threshold"], case["length_norm"],
                          case["early_exit"], variant=variant)
    assert sents == case["expect_sents"]
    assert np.allclose(norms, case["expect_scores_approx"], rtol=1e-6, atol=0)


def test_ka1_structure(po):
    case = KA[0]
    cb, edges, term = oracle_logical(po.OracleTrie.from_keys(case["keys"]))
    assert cb.tolist() == case["expect_trie"]["child_begin"]
    assert edges == case["expect_trie"]["edges"]
    assert term.tolist() == case["expect_trie"]["terminal"]


def test_final_beam_zero_leaves_outputs_untouched(po):
    tr = po.OracleTrie.from_keys([[1], [2]])
    sents, norms = tr.tbs([3, 0], np.array([[1, 2], [1, 2]]),
                          np.full((2, 2), -1.0, dtype=np.float32))
    assert sents == [] and norms.size == 0


def test_length_norm_closed_form(po):
    # s * (6 / (5 + d))^alpha with the host pow (agent.h:69-72)
    tr = po.OracleTrie.from_keys([[1, 2, 3]])
    ids = np.array([[1], [2], [3]], dtype=np.uint32)
    lp = np.array([[-0.25], [-0.5], [-0.75]], dtype=np.float32)
    for alpha in (0.0, 1.0, 2.5, 5.0):
        sents, norms = tr.tbs([4, 4, 4], ids, lp, -10, -40, alpha, False)
        assert sents == [[1, 2, 3]]
        assert norms[0] == -1.5 * math.pow(6.0 / 8.0, alpha)


def _walk(cb, edges, key):
    """Terminal node of `key` in a logical trie (edges of >= 1 token)."""
    n, pos = 0, 0
    while pos < len(key):
        kids = range(cb[n], cb[n + 1])
        nxt = [c for c in kids if edges[c][0] == key[pos]]
        if not nxt:
            return None
        n = nxt[0]
        e = edges[n]
        if key[pos:pos + len(e)] != e:
            return None
        pos += len(e)
    return n


def _brute(keys, cb, edges, term, ids, lp, tok_thr, sent_thr, alpha):
    """All keys whose every token is proposed at its step with logp >
    tok_thr and running sum > sent_thr; ascending (norm, node)."""
    res = []
    for key in keys:
        if len(key) > ids.shape[0] or len(key) == 0:
            continue
        s = 0.0
        ok = True
        for t, tok in enumerate(key):
            hit = np.nonzero(ids[t] == tok)[0]
            if hit.size == 0:
                ok = False
                break
            x = float(lp[t, hit[0]])
            if x <= tok_thr or s + x <= sent_thr:
                ok = False
                break
            s += x
        if not ok:
            continue
        node = _walk(cb, edges, key)
        norm = s * math.pow(6.0 / (5.0 + len(key)), alpha)
        res.append((norm, node, list(key)))
    res.sort(key=lambda r: (r[0], r[1]))
    return [r[2] for r in res], [r[0] for r in res]


@settings(max_examples=150, deadline=None,
          suppress_health_check=[HealthCheck.too_slow])
@given(data=st.data())
def test_bruteforce_no_pruning(po, data):
    vocab = data.draw(st.integers(2, 6))
    keys = data.draw(st.lists(st.lists(st.integers(0, vocab - 1), min_size=1,
                                       max_size=4), min_size=1, max_size=12))
    keys = sorted({tuple(k) for k in keys})
    keys = [list(k) for k in keys]
    tr = po.OracleTrie.from_keys(keys)
    cb, edges, term = oracle_logical(tr)
    # the brute force does not model the link quirk: require that no link
    # node has children
    for n in range(1, len(term)):
        if len(edges[n]) >= 2 and cb[n + 1] > cb[n]:
            return
    T = max(len(k) for k in keys)
    K = data.draw(st.integers(1, vocab))
    seed = data.draw(st.integers(0, 2 ** 31))
    rng = np.random.default_rng(seed)
    ids = np.stack([np.sort(rng.choice(vocab, K, replace=False))
                    for _ in range(T)]).astype(np.uint32)
    lp = (-rng.random((T, K)) * 3).astype(np.float32)
    alpha = data.draw(st.sampled_from([0.0, 1.0, 5.0]))
    big = 10 ** 6
    want = _brute(keys, cb, edges, term, ids, lp, -2.5, -6.0, alpha)
    for variant in (0, 1):
        got = tr.tbs([big] * T, ids, lp, -2.5, -6.0, alpha, False,
                     variant=variant)
        assert got[0] == want[0]
        assert np.array_equal(got[1], np.array(want[1]))


@settings(max_examples=60, deadline=None)
@given(st.lists(st.lists(st.integers(0, 9), min_size=0, max_size=6),
                min_size=1, max_size=40))
def test_build_invariants(po, keys):
    tr = po.OracleTrie.from_keys(keys)
    cb, edges, term = oracle_logical(tr)
    uniq = {tuple(k) for k in keys}
    assert tr.num_keys() == len(uniq) == int(term.sum())
    n = len(term)
    assert cb[0] == min(1, n) or n == 1
    assert cb[-1] == n
    assert all(cb[v] <= cb[v + 1] for v in range(n))  # breadth-first ids
    for v in range(n):
        kids = list(range(cb[v], cb[v + 1]))
        assert all(c > v for c in kids)
        firsts = [edges[c][0] for c in kids]
        assert firsts == sorted(set(firsts))   # label order, distinct
        for c in kids:
            assert len(edges[c]) >= 1
        # maximal path compression (louds-trie.cc:537-550): an edge stops
        # only where a key ends or the keys below it branch, so a non-root
        # node that ends no key has at least two children (a single child
        # would have been merged into its edge, and a childless one would
        # be a key)
        if v > 0 and not term[v]:
            assert len(kids) >= 2, (v, edges[v], kids)
    for k in uniq:
        node = _walk(cb, edges, list(k))
        assert node is not None and term[node] == 1


def test_variants_agree_on_regressions(po):
    for c in load_golden("oracle_regression.json"):
        tr = po.OracleTrie.from_keys(c["keys"])
        for variant in (0, 1):
            sents, norms = tr.tbs(c["beams"], np.array(c["topk_id"]),
                                  np.array(c["topk_logp"], dtype=np.float32),
                                  c["token_logp_threshold"],
                                  c["sents_logp_threshold"], c["length_norm"],
                                  c["early_exit"], variant=variant)
            assert sents == c["expect_sents"]
            assert [float(x).hex() for x in norms] == c["expect_norms_hex"]


def test_from_trie_equals_from_keys(ft, po):
    # the oracle over a flashtrie image (the scale tests' and the bench's
    # way) searches exactly as the oracle built from the same keys
    toks, offs = ft.synth_keys(3000, 512, 3, 7, 1.1, 5)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    a = po.OracleTrie.from_trie(t)
    b = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 4, 512, 6, 24, 8, 0.3, 2.0, True, 5)
    for r in range(4):
        ra = a.tbs([8] * 6, ids[r], lp[r], -10.0, -40.0, 5.0, False)
        rb = b.tbs([8] * 6, ids[r], lp[r], -10.0, -40.0, 5.0, False)
        assert ra[0] == rb[0] and np.array_equal(ra[1], rb[1])
