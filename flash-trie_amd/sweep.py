#!/usr/bin/env python3
"""Beam-width / top-K / batch-size sweeps in one process.

Covers what the reference's examples/run_trie_search_BWsweep.py and
run_trie_search_BSsweep.py drive (one run_trie_search pass per
configuration, one latency row each), but loads the trie and sizes the GPU
workspace once for the widest configuration instead of once per run.

Inputs: ``--data-path`` is one proposal file, or a pattern with one ``*``
filled by each ``--file-values`` entry (``output_topk*.tsv``).  A
configuration is (file, beam, topk, batch): ``--beam-topk`` lists
``beam[:topk]`` pairs (topk defaults to beam); without it each file value is
both beam and topk.  ``--onemap`` pairs the i-th file with the i-th pair,
otherwise every file runs every pair.  ``--batch-sizes`` multiplies the
configurations.  Every configuration writes
``<output-dir>/latency_b{beam}_k{topk}_bs{batch}.tsv``; ``--latency-report``
collects all rows in one TSV.
"""

import argparse
import glob
import os
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import numpy as np  # noqa: E402
from ft_harness import (Searcher, import_flashtrie, latency_tsv,  # noqa: E402
                        phase_tsv, read_topk_tsv, summarize_latency)
import run_trie_search as rts  # noqa: E402


def parse_pairs(entries):
    out = []
    for e in entries or []:
        beam, _, topk = e.strip().partition(":")
        out.append((int(beam), int(topk or beam)))
    return out


def configs(args):
    if "*" in args.data_path:
        if not args.file_values:
            raise SystemExit("--data-path with '*' needs --file-values")
        files = [(v, args.data_path.replace("*", v)) for v in args.file_values]
    else:
        files = [(None, args.data_path)]
    pairs = parse_pairs(args.beam_topk)
    if not pairs:
        if any(v is None for v, _ in files):
            raise SystemExit("give --beam-topk, or file values that are the beam width")
        pairs = [(int(v), int(v)) for v, _ in files]
        combos = list(zip(files, pairs))
    elif args.onemap:
        if len(pairs) != len(files):
            raise SystemExit("--onemap needs as many --beam-topk pairs as files")
        combos = list(zip(files, pairs))
    else:
        combos = [(f, p) for f in files for p in pairs]
    bss = [int(x) for x in args.batch_sizes.split(",") if x.strip()]
    return [(path, beam, topk, bs) for (_, path), (beam, topk) in combos for bs in bss]


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__,
                                formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--trie-path", required=True)
    p.add_argument("--data-path", required=True)
    p.add_argument("--file-values", nargs="+", default=None)
    p.add_argument("--beam-topk", nargs="+", default=None)
    p.add_argument("--onemap", action="store_true")
    p.add_argument("--batch-sizes", default="1")
    p.add_argument("--superset-topk", action="store_true")
    p.add_argument("--output-dir", default="out/sweep")
    p.add_argument("--latency-report", default=None)
    p.add_argument("--token-logp-threshold", type=float, default=-10.0)
    p.add_argument("--sent-logp-threshold", type=float, default=-40.0)
    p.add_argument("--length-norm", type=float, default=5.0)
    p.add_argument("--early-exit", action="store_true")
    p.add_argument("--max-seq-length", type=int, default=64)
    p.add_argument("--num-runs", type=int, default=11)
    p.add_argument("--max-queries", type=int, default=None)
    p.add_argument("--cpu", action="store_true")
    p.add_argument("--phase-timing", action="store_true",
                   help="also write phase_b{beam}_k{topk}_bs{batch}.tsv per configuration")
    args = p.parse_args(argv)
    cfgs = configs(args)
    for path, *_ in cfgs:
        if not glob.glob(path):
            raise SystemExit(f"no such file: {path}")
    ft = import_flashtrie()
    trie = ft.Trie()
    t0 = time.time()
    trie.load(args.trie_path)
    print(f"Loaded {args.trie_path} in {time.time() - t0:.2f}s; {len(cfgs)} configurations")
    if not args.cpu:
        mb = max(c[1] for c in cfgs)
        trie.init_tbs_gpu(max(c[3] for c in cfgs), max(c[2] for c in cfgs),
                          max_num_outpos=args.max_seq_length, max_num_out_beams=mb,
                          max_num_out_tokens=mb * args.max_seq_length,
                          max_num_inter_beams=mb * args.max_seq_length)
    os.makedirs(args.output_dir, exist_ok=True)
    rows, head = [], None
    cache = {}
    for path, beam, topk, bs in cfgs:
        if path not in cache:
            cache[path] = list(read_topk_tsv(path, args.max_queries))
        data = cache[path]
        s = Searcher(None, beam_size=beam, topk_tokens=topk, batch_size=bs,
                     max_seq_length=args.max_seq_length,
                     token_logp_threshold=args.token_logp_threshold,
                     sent_logp_threshold=args.sent_logp_threshold,
                     length_norm=args.length_norm, early_exit=args.early_exit,
                     use_gpu=not args.cpu, superset_topk=args.superset_topk,
                     trie=trie, init_gpu=False, verbose=False)
        ra = argparse.Namespace(num_runs=args.num_runs, batch_size=bs, output_path=None,
                                logging_steps=0)
        print(f"beam {beam} topk {topk} batch {bs} ({os.path.basename(path)})")
        per_run_ms, per_run_qps, _, phases = rts.run(ra, s, data)
        if not per_run_ms:
            continue
        stats = summarize_latency(per_run_ms)
        qps = float(np.mean(per_run_qps))
        qsd = float(np.std(per_run_qps, ddof=1)) if len(per_run_qps) > 1 else 0.0
        head, row = latency_tsv(beam, topk, bs, len(per_run_ms[0]), stats, qps, qsd)
        rows.append(row)
        with open(os.path.join(args.output_dir, f"latency_b{beam}_k{topk}_bs{bs}.tsv"),
                  "w") as fh:
            fh.write(head + "\n" + row + "\n")
        if args.phase_timing:
            pt = phase_tsv(beam, topk, bs, phases)
            if pt:
                with open(os.path.join(args.output_dir,
                                       f"phase_b{beam}_k{topk}_bs{bs}.tsv"), "w") as fh:
                    fh.write(pt[0] + "\n" + pt[1] + "\n")
    if args.latency_report and head:
        os.makedirs(os.path.dirname(os.path.abspath(args.latency_report)), exist_ok=True)
        with open(args.latency_report, "w") as fh:
            fh.write(head + "\n" + "\n".join(rows) + "\n")
        print(f"Latency report: {args.latency_report}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
