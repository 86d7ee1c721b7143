#!/usr/bin/env python3
"""Synthetic example workload: a trie and top-K proposal files.

Same options and output files as the reference's
examples/make_example_data.py:

* ``trie.bin``: the trie of ``--num-keys`` unique keys, written as a MARISA
  trie file (readable by this library and by the reference);
* ``topk.tsv`` (or ``topk/output_topk{K}.tsv`` for every K of
  ``--per-topk-files``): ``query_<i><TAB>{"probs": T x K, "indices": T x K}``
  rows in token order;
* ``keys.txt`` with ``--write-keys``.

Keys: a length drawn from ``--length-weights`` (lengths 1, 2, ...), a shared
two-token stem from a pool of num_keys / 64 stems for the first tokens, then
uniform tokens.  Proposal rows: the tokens of ``--seeds-per-query`` random
keys at that step score U(-2.2, -0.2); random distractors fill the row with
U(-12, -4); a vocabulary too small to fill the row pads with low token ids at
-12.  Scores are rounded to 4 decimals.  The random streams are numpy's, so
the keys differ from the reference's for the same seed; the shapes and the
score model are the same.
"""

import argparse
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from ft_harness import import_flashtrie  # noqa: E402


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__,
                                formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--out-dir", default="data")
    p.add_argument("--num-keys", type=int, default=1000000)
    p.add_argument("--key-length", type=int, default=8, help="maximum tokens per key")
    p.add_argument("--length-weights", default="2,10,45,25,10,5,2,1",
                   help="relative frequency of key lengths 1, 2, 3, ...")
    p.add_argument("--vocab-size", type=int, default=262144)
    p.add_argument("--num-queries", type=int, default=2000)
    p.add_argument("--topk", type=int, default=100)
    p.add_argument("--per-topk-files", default=None,
                   help="comma-separated K values: topk/output_topk{K}.tsv each")
    p.add_argument("--seeds-per-query", type=int, default=128)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--write-keys", action="store_true")
    return p.parse_args(argv)


def make_keys(rng, num_keys, key_length, vocab, weights):
    """Unique keys as (tokens, offsets), sorted."""
    if vocab < 2:
        raise SystemExit("--vocab-size must be at least 2")
    w = np.asarray(weights[:key_length], dtype=np.float64)
    if w.size == 0 or w.sum() <= 0:
        raise SystemExit("--length-weights must contain a positive value")
    w /= w.sum()
    stems = rng.integers(0, vocab, size=(max(1, num_keys // 64), 2))
    L = w.size
    found = np.zeros((0, L + 1), dtype=np.int64)
    for _ in range(20):                      # bounded: a tiny vocab may not fill
        need = num_keys - len(found)
        if need <= 0:
            break
        m = int(need * 1.3) + 16
        lens = rng.choice(np.arange(1, L + 1), size=m, p=w)
        toks = rng.integers(0, vocab, size=(m, L))
        st = stems[rng.integers(0, len(stems), size=m)]
        toks[:, :2] = np.where(np.arange(2)[None, :] < np.minimum(lens, 2)[:, None],
                               st, toks[:, :2])
        toks = np.where(np.arange(L)[None, :] < lens[:, None], toks, -1)
        rows = np.concatenate([lens[:, None], toks], axis=1)
        found = np.unique(np.concatenate([found, rows]), axis=0)
    if len(found) > num_keys:
        found = found[rng.permutation(len(found))[:num_keys]]
    if len(found) < num_keys:
        print(f"warning: {len(found)} unique keys of the {num_keys} requested; "
              "raise --vocab-size or --key-length")
    keys = sorted(tuple(int(t) for t in r[1:1 + r[0]]) for r in found)
    offs = np.zeros(len(keys) + 1, dtype=np.uint64)
    offs[1:] = np.cumsum([len(k) for k in keys])
    toks = np.fromiter((t for k in keys for t in k), dtype=np.uint32, count=int(offs[-1]))
    return keys, toks, offs


def make_row(rng, seed_tokens, topk, vocab):
    """One proposal row in token order: (ids, logps)."""
    scored = {}
    for t in seed_tokens:
        scored.setdefault(int(t), round(float(-0.2 - 2.0 * rng.random()), 4))
    tries = 0
    while len(scored) < topk and tries < 50:
        tries += 1
        for t in rng.integers(0, vocab, size=2 * (topk - len(scored)) + 8):
            if len(scored) >= topk:
                break
            scored.setdefault(int(t), round(float(-4.0 - 8.0 * rng.random()), 4))
    t = 0
    while len(scored) < topk:
        scored.setdefault(t, -12.0)
        t += 1
    ids = sorted(scored)[:topk]
    return ids, [scored[i] for i in ids]


def write_topk_file(path, rng, keys, key_length, topk, vocab, num_queries, seeds):
    with open(path, "w") as fh:
        for q in range(num_queries):
            pick = [keys[i] for i in rng.integers(0, len(keys), size=min(seeds, len(keys)))]
            indices, probs = [], []
            for step in range(key_length):
                ids, lps = make_row(rng, [k[step] for k in pick if step < len(k)], topk, vocab)
                indices.append(ids)
                probs.append(lps)
            fh.write(f"query_{q}\t" + json.dumps({"probs": probs, "indices": indices}) + "\n")
    return os.path.getsize(path)


def main(argv=None):
    args = parse_args(argv)
    rng = np.random.default_rng(args.seed)
    os.makedirs(args.out_dir, exist_ok=True)
    ft = import_flashtrie()
    weights = [float(x) for x in args.length_weights.split(",") if x.strip()]
    print(f"Generating {args.num_keys} keys (max length {args.key_length}, "
          f"vocab {args.vocab_size}) ...")
    keys, toks, offs = make_keys(rng, args.num_keys, args.key_length, args.vocab_size,
                                 weights)
    hist = np.bincount([len(k) for k in keys])
    print("  length distribution: " +
          "  ".join(f"{n}:{c}" for n, c in enumerate(hist) if c))
    trie_path = os.path.join(args.out_dir, "trie.bin")
    trie = ft.Trie()
    trie.build_arrays(toks, offs)
    trie.save_marisa(trie_path)
    print(f"Built trie -> {trie_path}: {trie.num_keys()} keys, {trie.num_nodes()} nodes")
    if args.write_keys:
        with open(os.path.join(args.out_dir, "keys.txt"), "w") as fh:
            for k in keys:
                fh.write(" ".join(map(str, k)) + "\n")
    if args.per_topk_files:
        d = os.path.join(args.out_dir, "topk")
        os.makedirs(d, exist_ok=True)
        for k in (int(v) for v in args.per_topk_files.split(",") if v.strip()):
            path = os.path.join(d, f"output_topk{k}.tsv")
            size = write_topk_file(path, rng, keys, args.key_length, k, args.vocab_size,
                                   args.num_queries, args.seeds_per_query)
            print(f"  K={k:<6} {size / (1 << 20):8.2f} MiB  {os.path.basename(path)}")
        return 0
    path = os.path.join(args.out_dir, "topk.tsv")
    size = write_topk_file(path, rng, keys, args.key_length, args.topk, args.vocab_size,
                           args.num_queries, args.seeds_per_query)
    print(f"Wrote {args.num_queries} queries -> {path} ({size / (1 << 20):.2f} MiB, "
          f"shape ({args.key_length}, {args.topk}) per query)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
