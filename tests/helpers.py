"""Helpers shared by the test modules."""

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

REC = np.dtype([("child_begin", "<u4"), ("first_tok", "<u4"),
                ("tail_off", "<u4"), ("meta", "<u4")])
TERMINAL = 0x80000000
LINK = 0x40000000


def decode_image(img):
    """Image blob (uint8 array) -> (num_nodes, records[N+1], parent, tail)."""
    img = np.asarray(img, dtype=np.uint8)
    hdr = np.frombuffer(img[:64].tobytes(), dtype="<u8", count=8)
    assert img[:7].tobytes() == b"FTIMG01"
    n, _, tl, ro, po_, to, tot = [int(x) for x in hdr[1:8]]
    assert tot == img.size
    recs = np.frombuffer(img[ro:ro + (n + 1) * 16].tobytes(), dtype=REC)
    parent = np.frombuffer(img[po_:po_ + n * 4].tobytes(), dtype="<u4")
    tail = np.frombuffer(img[to:to + tl * 4].tobytes(), dtype="<u4")
    return n, recs, parent, tail


def image_logical(img):
    """Image -> (child_begin[N+1], edges list, terminal[N]) in the oracle's
    logical form."""
    n, recs, _, tail = decode_image(img)
    meta = recs["meta"][:n].astype(np.uint64)
    elen = ((meta >> 16) & 0x3FFF).astype(np.int64)
    edges = []
    for v in range(n):
        if meta[v] & LINK:
            o = int(recs["tail_off"][v])
            edges.append(tail[o:o + elen[v]].tolist())
        elif v == 0:
            edges.append([])
        else:
            edges.append([int(recs["first_tok"][v])])
    term = ((meta >> 31) & 1).astype(np.uint8)
    return recs["child_begin"].copy(), edges, term


def oracle_logical(otrie):
    cb, eb, et, term = otrie.export()
    edges = [et[eb[v]:eb[v + 1]].tolist() for v in range(len(term))]
    return cb, edges, term


def load_golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def rows(ids, lp):
    return (np.asarray(ids, dtype=np.uint32).tolist(),
            np.asarray(lp, dtype=np.float32).tolist())


def assert_same_results(got, want, ctx=""):
    """got/want: (sents, norms).  Sequences bit-exact, norms bit-exact
    (the bar is 1e-5 relative; the host pow table makes them identical)."""
    gs, gn = got
    ws, wn = want
    assert len(gs) == len(ws), f"{ctx}: {len(gs)} results vs {len(ws)}"
    for i, (a, b) in enumerate(zip(gs, ws)):
        assert list(a) == list(b), f"{ctx}: sequence {i}: {a} vs {b}"
    gn = np.asarray(gn, dtype=np.float64)
    wn = np.asarray(wn, dtype=np.float64)
    assert np.allclose(gn, wn, rtol=1e-5, atol=0.0), f"{ctx}: norms differ"
    assert np.array_equal(gn, wn), f"{ctx}: norms not bit-identical"
