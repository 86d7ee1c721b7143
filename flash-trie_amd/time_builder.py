"""Times the key-set builder (Trie.build_arrays: explicit keys -> trie
image, the work of louds-trie.cc:397-640) on N synthetic unique keys over
the paper trie's vocabulary (2.2M tokens, Zipf(1.05)), uniform length
3-9 (mean 6, the paper trie's mean key length), and reports wall time and
peak resident memory of key generation and of the build.

    python time_builder.py N [--vocab V] [--lmax L] [--seed S]
    python time_builder.py N --from-paper [--shuffle]

With --from-paper the keys are those of a paper-shape trie of about N
unique keys (synth_paper_trie, length 3-16 with mean ~6, Zipf(1.05)
prefix sharing), read back from its image in lexicographic order (with
--shuffle, in a seeded random order); the build from them must give the
same image, which is checked.

One JSON line: keys, tokens, generate_s, build_s, nodes, image_bytes,
rss_after_generate_gib, peak_rss_gib (the process's high-water mark after
the build; the generated keys stay resident during it)."""
import argparse
import json
import os
import resource
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import flashtrie as ft  # noqa: E402


def hwm_gib():
    # VmHWM: the peak resident set of this process
    with open("/proc/self/status") as f:
        for line in f:
            if line.startswith("VmHWM:"):
                return int(line.split()[1]) / (1 << 20)
    return resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / (1 << 20)


def rss_gib():
    with open("/proc/self/status") as f:
        for line in f:
            if line.startswith("VmRSS:"):
                return int(line.split()[1]) / (1 << 20)
    return 0.0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("n", type=int)
    ap.add_argument("--vocab", type=int, default=2_200_000)
    ap.add_argument("--lmax", type=int, default=9)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--from-paper", action="store_true")
    ap.add_argument("--shuffle", action="store_true")
    a = ap.parse_args()
    t0 = time.perf_counter()
    src = None
    if a.from_paper:
        # the paper workload's ratio of draws to unique keys (845.45M draws
        # give 799.49M unique keys)
        src = ft.Trie()
        ft.synth_paper_trie(src, int(a.n * 845.45 / 799.49), a.vocab, 1.05, a.seed)
        print(f"[time_builder] paper-shape trie of {src.num_keys()} keys made", file=sys.stderr,
              flush=True)
        toks, offs = ft.keys_of(src, a.seed if a.shuffle else 0, progress=True)
    else:
        toks, offs = ft.synth_keys(a.n, a.vocab, 3, a.lmax, 1.05, a.seed)
    t1 = time.perf_counter()
    rss_gen = rss_gib()
    print(f"[time_builder] generated {offs.size - 1} keys ({toks.size} tokens) in {t1 - t0:.1f} s",
          file=sys.stderr, flush=True)
    t = ft.Trie()
    t2 = time.perf_counter()
    t.build_arrays(toks, offs, progress=True)
    t3 = time.perf_counter()
    same = None
    if src is not None:
        import numpy as np
        same = bool(np.array_equal(src.image_view(), t.image_view()))
    out = {"keys": int(offs.size - 1), "tokens": int(toks.size), "generate_s": round(t1 - t0, 2),
           "build_s": round(t3 - t2, 2), "num_keys": int(t.num_keys()),
           "image_bytes": int(t.image_view().nbytes),
           "rss_after_generate_gib": round(rss_gen, 2), "peak_rss_gib": round(hwm_gib(), 2),
           "keys_from": ("paper-shape trie, " + ("shuffled" if a.shuffle else "sorted"))
           if a.from_paper else "synth_keys",
           "key_length": [3, 16] if a.from_paper else [3, a.lmax], "cpus": os.cpu_count(),
           "image_equals_source": same}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
