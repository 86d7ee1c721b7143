"""Shared code of the full-size GPU parity tests: the oracle over many
requests on host threads, and batched comparisons through the product's
two batch paths."""

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from helpers import assert_same_results

THREADS = min(16, os.cpu_count() or 1)


def oracle_all(ot, beams, ids, lp, rules):
    """Oracle results of every request (the ctypes call releases the GIL,
    so host threads run requests side by side)."""
    tok, sent, alpha, early = rules

    def one(r):
        return ot.tbs(beams[r], ids[r], lp[r], tok, sent, alpha, early)

    with ThreadPoolExecutor(THREADS) as ex:
        return list(ex.map(one, range(len(beams))))


def check_bs_tbs_gpu(ft, t, beams, ids, lp, rules, want, batch, what):
    """Requests through bs_tbs_gpu (Python lists in, the reference's
    surface), `batch` per call."""
    tok, sent, alpha, early = rules
    n = len(beams)
    nonempty = 0
    for b0 in range(0, n, batch):
        nb = min(batch, n - b0)
        got = ft.bs_tbs_gpu(t, nb, beams[b0:b0 + nb].tolist(), ids[b0:b0 + nb].tolist(),
                            lp[b0:b0 + nb].tolist(), tok, sent, alpha, early)
        for i in range(nb):
            assert_same_results((got[0][i], got[1][i]), want[b0 + i],
                                f"{what} request {b0 + i}")
            nonempty += len(want[b0 + i][0]) > 0
    return nonempty


def check_numpy_batches(ft, t, beams, ids, lp, rules, want, batch, what):
    """Requests through stage / launch / fetch (numpy arrays), `batch` per
    launch."""
    tok, sent, alpha, early = rules
    n = len(beams) - len(beams) % batch
    for b0 in range(0, n, batch):
        ft.stage(t, beams[b0:b0 + batch], ids[b0:b0 + batch], lp[b0:b0 + batch],
                 tok, sent, alpha, early)
        ft.launch(t)
        count, norms, lens, toks, _ = ft.fetch(t)
        for i in range(batch):
            c = int(count[i])
            got = ([toks[i, j, :lens[i, j]].tolist() for j in range(c)], norms[i, :c])
            assert_same_results(got, want[b0 + i], f"{what} request {b0 + i}")


def result_stats(want):
    n = np.array([len(w[0]) for w in want])
    return {"requests": len(want), "nonempty": int((n > 0).sum()),
            "mean_results": float(n.mean())}
