"""The closed form the kernel uses for a bounded heap, checked against a
direct simulation of the reference's Candidates (candidates.h:47-55) on
push sequences full of ties.

Pushes e_1..e_n (arrival order) of (norm, node), node ids distinct, into a
heap of capacity M keep: everything if n <= M; else, with v* the M-th
largest norm, all norm > v* items plus -- among the norm == v* items that
are among the first M items of {norm >= v*} in arrival order -- the
M - #{norm > v*} with the largest node ids.
"""

import heapq

from hypothesis import given, settings, strategies as st


def simulate(items, M):
    # heap of (norm, node): the top is the worst (smallest norm, then the
    # smallest node id), exactly AgentComparer's order
    h = []
    for norm, node in items:
        if len(h) < M or norm > h[0][0]:
            heapq.heappush(h, (norm, node))
        if len(h) > M:
            heapq.heappop(h)
    return sorted(h)


def closed_form(items, M):
    if len(items) <= M:
        return sorted(items)
    v = sorted((x[0] for x in items), reverse=True)[M - 1]
    greater = [x for x in items if x[0] > v]
    r = M - len(greater)
    ge = [x for x in items if x[0] >= v][:M]        # arrival order kept
    A = [x for x in ge if x[0] == v]
    keep = sorted(A, key=lambda x: x[1], reverse=True)[:r]
    return sorted(greater + keep)


@settings(max_examples=3000, deadline=None)
@given(st.data())
def test_closed_form_matches_heap(data):
    n = data.draw(st.integers(0, 30))
    nodes = data.draw(st.permutations(list(range(100)))) [:n]
    norms = data.draw(st.lists(st.integers(-4, 0), min_size=n, max_size=n))
    items = list(zip(norms, nodes))
    M = data.draw(st.integers(1, 12))
    assert closed_form(items, M) == simulate(items, M)


@settings(max_examples=1000, deadline=None)
@given(st.data())
def test_incremental_equals_one_shot(data):
    # `selected` is fed step by step; the state is the set, so merging the
    # kept set with the next step's pushes (old items first) is exact
    M = data.draw(st.integers(1, 8))
    steps = data.draw(st.integers(1, 4))
    seq, node = [], 0
    state = []
    for _ in range(steps):
        k = data.draw(st.integers(0, 10))
        batch = []
        for _ in range(k):
            batch.append((data.draw(st.integers(-3, 0)), node))
            node += 1
        seq += batch
        state = closed_form(state + batch, M)
    assert state == simulate(seq, M)
