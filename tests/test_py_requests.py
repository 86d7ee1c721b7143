"""The search entry points' argument reading (py_requests.h): Python lists,
tuples and numpy arrays of every common dtype, read in place, must give
exactly what pybind11's generic STL casters -- the reference module's
(tools/bindings.cpp:45-119) -- give, and reject what they reject.  CPU only
(flashtrie._convert_request runs the reader alone); the host search then
checks that numpy inputs search like lists."""

import numpy as np
import pytest

from helpers import assert_same_results

T, K = 5, 17


@pytest.fixture(scope="module")
def req():
    rng = np.random.default_rng(7)
    ids = np.sort(rng.choice(2**32 - 1, size=(T, K), replace=False), axis=1)
    ids[0, -1] = 2**32 - 1  # the largest uint32 (two 30-bit digits)
    ids[1, 0] = 0
    ids[2, 0] = 2**30 - 1  # one digit / two digits boundary
    ids[2, 1] = 2**30
    lp = rng.normal(0, 3, size=(T, K)).astype(np.float64)
    lp[0, 0] = 1e-46  # below float's subnormals: rounds to 0
    lp[0, 1] = -3.4028235e38
    lp[1, 2] = float(np.float32(0.1)) + 1e-17  # rounding of the double
    return [9, 8, 7, 6, 5], ids.astype(np.uint32), lp


def same(ft, *args):
    b, i, l = ft._convert_request(*args)
    b2, i2, l2 = ft._convert_request(*args, generic=True)
    assert b == b2
    assert i.dtype == np.uint32 and np.array_equal(i, i2)
    assert np.array_equal(l.view(np.uint32), l2.view(np.uint32))
    return b, i, l


def forms(beams, ids, lp):
    """Every argument form a caller might pass for one request."""
    il, ll = ids.tolist(), lp.tolist()
    l32 = lp.astype(np.float32)
    return {
        "lists": (beams, il, ll),
        "tuples": (tuple(beams), tuple(map(tuple, il)), tuple(map(tuple, ll))),
        "np_u32_f32": (np.array(beams, dtype=np.uint32), ids, l32),
        "np_f64": (beams, ids, lp),
        "np_f16": (beams, ids, np.clip(lp, -6e4, 6e4).astype(np.float16)),
        "np_i64": (beams, ids.astype(np.int64), l32),
        "np_u64": (beams, ids.astype(np.uint64), l32),
        "np_i32_small": (beams, (ids >> 2).astype(np.int32), l32),
        "np_u16": (beams, (ids & 0xFFFF).astype(np.uint16), l32),
        "rows_np": (beams, list(ids), list(l32)),
        "rows_np_f64": (beams, list(ids), list(lp)),
        "noncontig": (beams, np.asfortranarray(ids), np.asfortranarray(l32)),
        "strided": (beams, np.repeat(ids, 2, axis=1)[:, ::2], l32),
        "np_scalars": (beams, [list(r) for r in ids], [list(r) for r in l32]),
        "ints_as_logps": (beams, il, [[int(x) for x in r] for r in np.round(lp)]),
        "mixed": (beams, [ids[0]] + il[1:], [ll[0]] + list(l32[1:])),
        "extra_id_rows": (beams, il + [[1] * K], ll),
    }


@pytest.mark.parametrize("form", list(forms([1], np.zeros((1, 1), np.uint32),
                                            np.zeros((1, 1))).keys()))
def test_forms_match_generic(ft, req, form):
    beams, ids, lp = req
    args = forms(beams, ids, lp)[form]
    b, i, l = same(ft, *args)
    assert b == beams
    want_ids = np.asarray(args[1][:T] if form == "extra_id_rows" else args[1]).astype(np.uint64)
    assert np.array_equal(i.astype(np.uint64), want_ids[:T])
    # every form of the logps is the double (or float) rounded to float
    want_lp = np.array([[float(x) for x in r] for r in args[2]], dtype=np.float64)
    assert np.array_equal(l.view(np.uint32), want_lp.astype(np.float32).view(np.uint32))


def test_rejects_what_pybind_rejects(ft, req):
    beams, ids, lp = req
    bad = [
        (beams, ids.astype(np.int64) - 1, lp),          # negative id (ids[1, 0] = 0)
        (beams, ids.astype(np.uint64) + 2**32, lp),     # id >= 2^32
        (beams, [[float(x) for x in r] for r in ids], lp),  # floats for ids
        (beams, ids.astype(np.float64), lp),
        (beams, ids, [["x"] * K] * T),
        (beams, ids, [[None] * K] * T),
        ([-1] + beams[1:], ids, lp),
    ]
    for a in bad:
        with pytest.raises(TypeError):
            ft._convert_request(*a)
        with pytest.raises(TypeError):
            ft._convert_request(*a, generic=True)


def test_bools_and_index_objects(ft):
    class Idx:
        def __init__(self, v):
            self.v = v

        def __index__(self):
            return self.v

    b, i, l = same(ft, [2, 2], [[True, Idx(7)], [False, 3]], [[-1.0, -2.0], [-3.0, -4.0]])
    assert i.tolist() == [[1, 7], [0, 3]]


def test_shape_errors(ft):
    cases = [
        (([], [[1]], [[-1.0]]), "beams is empty"),
        (([2], [], [[-1.0]]), "topk rows are empty"),
        (([2], [[1]], []), "topk rows are empty"),
        (([2], [[]], [[]]), "row 0 is empty"),
        (([2, 2], [[1, 2]], [[-1.0, -1.0], [-1.0, -1.0]]), "fewer topk_id rows"),
        (([2], [[1], [2]], [[-1.0], [-1.0]]), "fewer beam widths"),
        (([2, 2], [[1, 2], [1]], [[-1.0, -1.0], [-1.0]]), "ragged"),
        (([2, 2], [[1, 2], [1, 2]], [[-1.0, -1.0], [-1.0]]), "ragged"),
        (([0, 2], [[1], [2]], [[-1.0], [-1.0]]), "beam width 0"),
        (([2, 2], np.ones((2, 3), np.uint32), np.ones((2, 2), np.float32)), "ragged"),
    ]
    for args, msg in cases:
        for generic in (False, True):
            with pytest.raises(RuntimeError, match=msg):
                ft._convert_request(*args, generic=generic)
    # final beam 0: no search and no shape checks (outputs stay empty), but
    # the rows must still convert, as the reference's signature requires
    for generic in (False, True):
        assert ft._convert_request([3, 0], [[1, 2], [1]], [[-1.0]],
                                   generic=generic)[1].shape == (0, 0)
        with pytest.raises(TypeError):
            ft._convert_request([3, 0], "not rows", None, generic=generic)


def test_host_search_numpy_equals_lists(ft, po):
    toks, offs = ft.synth_keys(5000, 512, 3, 7, 1.1, 11)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    o = po.OracleTrie.from_keys(toks=toks, offs=offs)
    ids, lp = ft.synth_requests(t, 0, 6, 512, 6, 24, 6, 0.3, 2.0, True, 5)
    for r in range(6):
        want = o.tbs([8] * 6, ids[r], lp[r], -10.0, -40.0, 5.0, False)
        for args in [([8] * 6, ids[r].tolist(), lp[r].tolist()),
                     (np.full(6, 8), ids[r], lp[r]),
                     ([8] * 6, ids[r].astype(np.int64), lp[r].astype(np.float64))]:
            got = ft.tbs(t, *args, -10.0, -40.0, 5.0, False, False)
            assert_same_results(got[:2], want, f"request {r}")


def test_result_lists(ft):
    # the lists bs_tbs_gpu returns: each result's first `length` tokens as
    # ints (ids up to 2^32 - 1), its norm as a float
    big = (1 << 32) - 1
    toks = np.array([[7, 2_000_000, 0], [2_000_000, 7, big], [big, 0, 0]], np.uint32)
    lens = np.array([2, 3, 1], np.uint32)
    norms = np.array([-1.5, -2.25, 0.0])
    sents, ns = ft._result_lists(lens, toks, norms)
    assert sents == [[7, 2_000_000], [2_000_000, 7, big], [big]]
    assert ns == [-1.5, -2.25, 0.0]
    assert all(type(x) is int for s in sents for x in s)
    assert all(type(x) is float for x in ns)
    e, en = ft._result_lists(np.zeros(0, np.uint32), np.zeros((0, 3), np.uint32),
                             np.zeros(0))
    assert e == [] and en == []
    with pytest.raises(ValueError):
        ft._result_lists(np.array([4, 0, 0], np.uint32), toks, norms)


def test_result_lists_leave_the_collector_as_found(ft):
    # the result lists are built with the cyclic collector held off; its
    # state is restored after, also when the call raises
    import gc
    toks = np.arange(12, dtype=np.uint32).reshape(4, 3)
    lens = np.array([3, 2, 1, 0], np.uint32)
    norms = np.zeros(4)
    was = gc.isenabled()
    try:
        gc.enable()
        ft._result_lists(lens, toks, norms)
        assert gc.isenabled()
        with pytest.raises(ValueError):
            ft._result_lists(np.array([9, 0, 0, 0], np.uint32), toks, norms)
        assert gc.isenabled()
        gc.disable()
        ft._result_lists(lens, toks, norms)
        assert not gc.isenabled()
    finally:
        (gc.enable if was else gc.disable)()


def test_host_search_leaves_the_collector_as_found(ft):
    import gc
    toks, offs = ft.synth_keys(2000, 256, 3, 6, 1.1, 3)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    ids, lp = ft.synth_requests(t, 0, 1, 256, 5, 16, 4, 0.3, 2.0, True, 1)
    assert gc.isenabled()
    ft.tbs(t, [4] * 5, ids[0], lp[0], -10.0, -40.0, 5.0, False, False)
    assert gc.isenabled()
