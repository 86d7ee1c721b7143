"""Benchmark harness over the flashtrie module: proposal files, request
preparation, batched search with timing, latency statistics.

Same behaviour and file formats as the reference's examples/flashtrie_bench.py
(read_topk_tsv :59-79, iter_batches :82-90, FlashTrieSearcher :93-281,
summarize_latency :289-316), so a run here and a run of the reference on the
same files print comparable numbers:

* proposal file: one ``query<TAB>json`` line per query, the JSON holding
  ``probs`` and ``indices`` (T x K) and optionally ``lcid``;
* ``superset_topk``: a row wider than K keeps its K highest-scoring columns;
* rows are sorted by token id before the search;
* a forced first step (``trie_start_token``: an int, or ``"lcid"`` for the
  record's field) prepends a row where only that token is live (logp 0, the
  other columns -inf) with beam width 1, and strips the token from every
  result;
* timing: the milliseconds ``bs_tbs_gpu`` reports per call (or host wall time
  for the CPU path), per-phase device times summed per call.
"""

import json
import math
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

__all__ = ["import_flashtrie", "read_topk_tsv", "iter_batches", "prepare_request",
           "Searcher", "summarize_latency", "latency_tsv", "phase_tsv",
           "PHASE_NAMES"]

PHASE_NAMES = ["expansion", "validation", "selection", "grid_overhead", "kernel"]


def import_flashtrie():
    """The flashtrie module: from FLASHTRIE_BUILD_DIR when set, else from this
    package (built by build.py)."""
    d = os.environ.get("FLASHTRIE_BUILD_DIR", HERE)
    if d not in sys.path:
        sys.path.insert(0, d)
    try:
        import flashtrie
    except ImportError as exc:
        raise SystemExit(f"cannot import flashtrie from {d} ({exc}); build it with "
                         f"python {os.path.join(HERE, 'build.py')}") from exc
    return flashtrie


def read_topk_tsv(path, max_queries=None):
    """Yields (query, record) from a ``query<TAB>json`` proposal file."""
    with open(path) as fh:
        for n, line in enumerate(fh):
            if max_queries is not None and n >= max_queries:
                return
            line = line.rstrip("\n")
            if not line:
                continue
            query, sep, payload = line.partition("\t")
            if not sep:
                raise ValueError(f"{path}:{n + 1}: expected 'query<TAB>json'")
            yield query, json.loads(payload)


def iter_batches(items, batch_size):
    """Consecutive lists of batch_size items (the last may be shorter)."""
    it = iter(items)
    while True:
        chunk = []
        for x in it:
            chunk.append(x)
            if len(chunk) == batch_size:
                break
        if not chunk:
            return
        yield chunk


def prepare_request(record, beam_size, topk, superset_topk=False, start_token=None):
    """One JSON record -> (beams, topk_id rows, topk_logp rows, forced).

    ``forced`` is True when a first step was prepended (its token is then
    stripped from the results)."""
    logp = np.asarray(record["probs"], dtype=np.float32)
    ids = np.asarray(record["indices"], dtype=np.uint32)
    if logp.shape != ids.shape or logp.ndim != 2:
        raise ValueError(f"probs {logp.shape} and indices {ids.shape} must be the "
                         "same 2-D shape")
    if superset_topk and ids.shape[1] > topk:
        # the K best columns of each row by score (the files are stored in
        # token order, not score order)
        keep = np.argpartition(-logp, topk - 1, axis=1)[:, :topk]
        logp = np.take_along_axis(logp, keep, axis=1)
        ids = np.take_along_axis(ids, keep, axis=1)
    if ids.shape[1] != topk:
        raise ValueError(f"data has K={ids.shape[1]} but topk={topk}; use "
                         "superset_topk to take the best K of a wider file")
    order = np.argsort(ids, axis=1, kind="stable")
    ids = np.take_along_axis(ids, order, axis=1)
    logp = np.take_along_axis(logp, order, axis=1)
    lead = record.get("lcid") if start_token == "lcid" else start_token
    forced = lead is not None
    if forced:
        lead = int(lead)
        # the forced token plus topk - 1 distinct fillers that never pass the
        # token threshold, in token order
        fill = [t for t in range(topk) if t != lead][:topk - 1]
        row_ids = np.array(sorted([lead] + fill), dtype=np.uint32)
        row_lp = np.where(row_ids == lead, np.float32(0.0),
                          np.float32(-math.inf)).astype(np.float32)
        ids = np.concatenate([row_ids[None, :], ids])
        logp = np.concatenate([row_lp[None, :], logp])
    beams = [beam_size] * ids.shape[0]
    if forced:
        beams[0] = 1
    return beams, ids.tolist(), logp.tolist(), forced


class Searcher:
    """Constrained beam search over one trie for a stream of batches.

    ``batch_times`` holds (milliseconds, requests) per call; ``phase_times``
    holds (summed phase vector, requests) per call."""

    def __init__(self, trie_path, beam_size=100, topk_tokens=8, batch_size=4,
                 max_seq_length=64, token_logp_threshold=-10.0,
                 sent_logp_threshold=-40.0, length_norm=5.0, early_exit=False,
                 use_gpu=True, superset_topk=False, trie_start_token=None,
                 verbose=True, trie=None, init_gpu=True):
        self.ft = import_flashtrie()
        self.beam_size = beam_size
        self.topk_tokens = topk_tokens
        self.batch_size = batch_size
        self.max_seq_length = max_seq_length
        self.thr = (token_logp_threshold, sent_logp_threshold)
        self.length_norm = length_norm
        self.early_exit = early_exit
        self.use_gpu = use_gpu
        self.superset_topk = superset_topk
        self.trie_start_token = trie_start_token
        self.batch_times, self.phase_times = [], []
        if trie is None:
            t0 = time.time()
            trie = self.ft.Trie()
            trie.load(trie_path)   # a MARISA trie.bin or a saved image
            if verbose:
                print(f"Loaded {trie_path} in {time.time() - t0:.2f}s: "
                      f"{trie.num_keys()} keys, {trie.num_nodes()} nodes, "
                      f"{trie.total_size() / (1 << 20):.2f} MiB")
        self.trie = trie
        if use_gpu and init_gpu:
            # one workspace for the widest call of the run (the forced step
            # counts in max_seq_length)
            trie.init_tbs_gpu(batch_size, topk_tokens, max_num_outpos=max_seq_length,
                              max_num_out_beams=beam_size,
                              max_num_out_tokens=beam_size * max_seq_length,
                              max_num_inter_beams=beam_size * max_seq_length)

    def search(self, records):
        """Searches a batch of JSON records; returns (sequences, scores) per
        record."""
        prep = [prepare_request(r, self.beam_size, self.topk_tokens,
                                self.superset_topk, self.trie_start_token)
                for r in records]
        tok_thr, sent_thr = self.thr
        if self.use_gpu:
            sents, norms, ms, phases = self.ft.bs_tbs_gpu(
                self.trie, len(prep), [p[0] for p in prep], [p[1] for p in prep],
                [p[2] for p in prep], tok_thr, sent_thr, self.length_norm,
                self.early_exit)
        else:
            sents, norms, phases = [], [], []
            t0 = time.perf_counter()
            for beams, ids, lps, _ in prep:
                s, n, _ = self.ft.tbs(self.trie, beams, ids, lps, tok_thr, sent_thr,
                                      self.length_norm, self.early_exit, False)
                sents.append(s)
                norms.append(n)
            ms = (time.perf_counter() - t0) * 1e3
        self.batch_times.append((ms, len(prep)))
        if phases and any(any(p) for p in phases):
            self.phase_times.append(([sum(p[k] for p in phases)
                                      for k in range(len(phases[0]))], len(phases)))
        for i, p in enumerate(prep):
            if p[3]:
                sents[i] = [s[1:] for s in sents[i]]
        return sents, [np.asarray(n) for n in norms]

    def reset_timers(self):
        self.batch_times, self.phase_times = [], []


def summarize_latency(per_run_ms, percentiles=(50, 90, 95, 99)):
    """Statistics within each measured run, then mean and sample standard
    deviation across runs (so the deviation is run-to-run variance)."""
    runs = [np.asarray(r, dtype=np.float64) for r in per_run_ms if len(r)]

    def across(vals):
        m = float(np.mean(vals)) if vals else 0.0
        s = float(np.std(vals, ddof=1)) if len(vals) > 1 else 0.0
        return m, s

    out = {"num_measured_runs": len(runs)}
    out["mean_ms"], out["std_ms"] = across([float(r.mean()) for r in runs])
    for p in percentiles:
        out[f"p{p}_ms"], out[f"std_p{p}_ms"] = across(
            [float(np.percentile(r, p)) for r in runs])
    return out


def latency_tsv(beam, topk, batch_size, batches_per_run, stats, mean_qps, std_qps,
                percentiles=(50, 90, 95, 99)):
    """(header, row) of the latency summary file, the reference's columns."""
    cols = ["beam", "topk", "batch_size", "batches_per_run", "num_measured_runs",
            "mean_ms", "std_ms"]
    vals = [beam, topk, batch_size, batches_per_run, stats["num_measured_runs"],
            f"{stats['mean_ms']:.3f}", f"{stats['std_ms']:.3f}"]
    for p in percentiles:
        cols += [f"p{p}_ms", f"std_p{p}_ms"]
        vals += [f"{stats[f'p{p}_ms']:.3f}", f"{stats[f'std_p{p}_ms']:.3f}"]
    cols += ["mean_qps", "std_qps"]
    vals += [f"{mean_qps:.3f}", f"{std_qps:.3f}"]
    return "\t".join(cols), "\t".join(str(v) for v in vals)


def phase_tsv(beam, topk, batch_size, phase_times):
    """(header, row) of the per-request phase file, or None without phases."""
    if not phase_times:
        return None
    total = np.zeros(len(PHASE_NAMES))
    n = 0
    for summed, count in phase_times:
        total += np.asarray(summed[:len(PHASE_NAMES)], dtype=np.float64)
        n += count
    means = total / max(n, 1)
    head = "beam\ttopk\tbatch_size\t" + "\t".join(f"{x}_ms" for x in PHASE_NAMES)
    row = f"{beam}\t{topk}\t{batch_size}\t" + "\t".join(f"{m:.4f}" for m in means)
    return head, row
