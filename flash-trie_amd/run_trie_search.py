#!/usr/bin/env python3
"""Constrained trie beam search over a top-K proposal file, with latency
statistics.

Same options, printed summary and output files as the reference's
examples/run_trie_search.py:

* ``--num-runs`` passes over the data; pass 1 is a warm-up whose results are
  written to ``--output-path`` (``query<TAB>count<TAB>seq | seq ...``) and
  whose times are dropped; percentiles are taken within each measured pass
  and averaged across passes;
* ``--latency-out`` writes one TSV row (beam, topk, batch_size,
  batches_per_run, num_measured_runs, mean/std and p50/p90/p95/p99 with their
  deviations, mean_qps, std_qps);
* ``--phase-out`` writes the mean device time per request by phase.

Example::

    python make_example_data.py --out-dir data --topk 100
    python run_trie_search.py --trie-path data/trie.bin --data-path data/topk.tsv \\
        --beam-size 100 --topk-tokens 100 --batch-size 8 --latency-out out/lat.tsv
"""

import argparse
import os
import sys
import time

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from ft_harness import (Searcher, iter_batches, latency_tsv, phase_tsv,  # noqa: E402
                        read_topk_tsv, summarize_latency)

PERCENTILES = (50, 90, 95, 99)


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__,
                                formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--trie-path", required=True,
                   help="MARISA trie.bin (or a trie image saved by this library)")
    p.add_argument("--data-path", required=True,
                   help="proposal TSV: 'query<TAB>json' per line")
    p.add_argument("--output-path", default=None, help="decoded sequences (warm-up pass)")
    p.add_argument("--latency-out", default=None, help="one-row latency summary TSV")
    p.add_argument("--phase-out", default=None, help="per-phase device time TSV")
    p.add_argument("--beam-size", type=int, default=100)
    p.add_argument("--topk-tokens", type=int, default=8)
    p.add_argument("--superset-topk", action="store_true",
                   help="rows wider than --topk-tokens keep their best columns")
    p.add_argument("--token-logp-threshold", type=float, default=-10.0)
    p.add_argument("--sent-logp-threshold", type=float, default=-40.0)
    p.add_argument("--length-norm", type=float, default=5.0)
    p.add_argument("--early-exit", action="store_true")
    p.add_argument("--trie-start-token", default=None,
                   help="force a first token with beam 1: an integer, or 'lcid' for "
                        "each record's lcid field")
    p.add_argument("--batch-size", type=int, default=1)
    p.add_argument("--max-seq-length", type=int, default=64,
                   help="steps per request the workspace holds (history = beam * this)")
    p.add_argument("--cpu", action="store_true", help="host search instead of the GPU")
    p.add_argument("--num-runs", type=int, default=11,
                   help="passes over the data, the first a warm-up")
    p.add_argument("--max-queries", type=int, default=None)
    p.add_argument("--logging-steps", type=int, default=1000)
    return p.parse_args(argv)


def start_token_arg(v):
    if v is None or v == "lcid":
        return v
    try:
        v = int(v)
    except ValueError:
        raise SystemExit("--trie-start-token must be an integer or 'lcid'")
    return v if v >= 0 else None


def run(args, searcher, dataset, log=print):
    """All passes over `dataset` with `searcher`; returns the summary dict
    (stats, qps, outputs per query, batches per run, phase times)."""
    per_run_ms, per_run_qps, outputs = [], [], []
    out_fh = None
    if args.output_path:
        os.makedirs(os.path.dirname(os.path.abspath(args.output_path)), exist_ok=True)
        out_fh = open(args.output_path, "w")
    phase_times = []
    try:
        for run_id in range(1, args.num_runs + 1):
            warm = run_id == 1
            searcher.reset_timers()
            t0 = time.time()
            for step, batch in enumerate(iter_batches(dataset, args.batch_size)):
                seqs, _ = searcher.search([rec for _, rec in batch])
                if warm:
                    for (query, _), s in zip(batch, seqs):
                        outputs.append(len(s))
                        if out_fh:
                            out_fh.write(f"{query}\t{len(s)}\t" +
                                         " | ".join(" ".join(map(str, x)) for x in s) + "\n")
                if args.logging_steps and step and step % args.logging_steps == 0:
                    log(f"  run {run_id}: {step} batches")
            wall = time.time() - t0
            ms = [m for m, _ in searcher.batch_times]
            log(f"  {'warm-up' if warm else f'run {run_id - 1}':>9}: {np.mean(ms):7.3f} "
                f"ms/batch  ({wall:.1f}s wall)")
            if not warm:
                per_run_ms.append(ms)
                per_run_qps.append(len(dataset) / wall if wall else 0.0)
                phase_times.extend(searcher.phase_times)
    finally:
        if out_fh:
            out_fh.close()
    return per_run_ms, per_run_qps, outputs, phase_times


def main(argv=None):
    args = parse_args(argv)
    if args.num_runs < 1:
        raise SystemExit("--num-runs must be >= 1")
    print(f"Reading {args.data_path} ...")
    dataset = list(read_topk_tsv(args.data_path, args.max_queries))
    if not dataset:
        raise SystemExit(f"no queries in {args.data_path}")
    print(f"  {len(dataset)} queries")
    searcher = Searcher(args.trie_path, beam_size=args.beam_size,
                        topk_tokens=args.topk_tokens, batch_size=args.batch_size,
                        max_seq_length=args.max_seq_length,
                        token_logp_threshold=args.token_logp_threshold,
                        sent_logp_threshold=args.sent_logp_threshold,
                        length_norm=args.length_norm, early_exit=args.early_exit,
                        use_gpu=not args.cpu, superset_topk=args.superset_topk,
                        trie_start_token=start_token_arg(args.trie_start_token))
    print(f"\nBeam width      : {args.beam_size}\nTop-K tokens    : {args.topk_tokens}\n"
          f"Batch size      : {args.batch_size}\n"
          f"Device          : {'CPU (host search)' if args.cpu else 'GPU'}\n"
          f"Runs            : {args.num_runs} (1 warm-up + {args.num_runs - 1} measured)\n")
    t_all = time.time()
    per_run_ms, per_run_qps, outputs, phase_times = run(args, searcher, dataset)
    if args.output_path:
        print(f"\nOutputs written to: {args.output_path}")
    print("\n" + "=" * 56 + "\nLatency summary\n" + "=" * 56)
    if outputs:
        print(f"Mean outputs/query    : {np.mean(outputs):.2f}")
    if not per_run_ms:
        print("No measured runs (use --num-runs >= 2 to collect latency).")
        return 0
    stats = summarize_latency(per_run_ms, PERCENTILES)
    qps = float(np.mean(per_run_qps))
    qps_sd = float(np.std(per_run_qps, ddof=1)) if len(per_run_qps) > 1 else 0.0
    print(f"Measured runs         : {stats['num_measured_runs']}")
    print(f"Batches per run       : {len(per_run_ms[0])}")
    print(f"Mean latency/batch    : {stats['mean_ms']:.3f} +/- {stats['std_ms']:.3f} ms")
    for p in PERCENTILES:
        print(f"  P{p:<3}                : {stats[f'p{p}_ms']:.3f} +/- "
              f"{stats[f'std_p{p}_ms']:.3f} ms")
    print(f"Mean throughput       : {qps:.1f} +/- {qps_sd:.1f} queries/s")
    print(f"Total elapsed         : {time.time() - t_all:.1f}s")
    if args.latency_out:
        os.makedirs(os.path.dirname(os.path.abspath(args.latency_out)), exist_ok=True)
        head, row = latency_tsv(args.beam_size, args.topk_tokens, args.batch_size,
                                len(per_run_ms[0]), stats, qps, qps_sd, PERCENTILES)
        with open(args.latency_out, "w") as fh:
            fh.write(head + "\n" + row + "\n")
        print(f"Latency written to    : {args.latency_out}")
    if args.phase_out:
        pt = phase_tsv(args.beam_size, args.topk_tokens, args.batch_size, phase_times)
        if pt is None:
            print("No phase timings recorded (the host search has none).")
        else:
            os.makedirs(os.path.dirname(os.path.abspath(args.phase_out)), exist_ok=True)
            with open(args.phase_out, "w") as fh:
                fh.write(pt[0] + "\n" + pt[1] + "\n")
            print(f"Phases written to     : {args.phase_out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
