"""Per-step device profile of batch-1 searches, with a latency floor.

Runs `--requests` seeded requests of a workload one per launch (staged in
HBM, batch 1), `--reps` times, and prints the mean of each request's
device clocks (ft_fetch timing: expansion / selection / other / total) and
of its per-step counters (FT_STEP_STATS): parents, work items, next and
selected pushes, expansion and selection time, children scanned, bucket
reads, and for a shared step the leader's waits for the helpers' claims and
slices.

The floor is the time of each step's chain of dependent memory round trips
and cross-workgroup handshakes alone, with the latencies measured by
ft_copy_calib in the same run (chase: a dependent load over an image-sized
buffer, L_img, and an L2-resident one, L_l2; pingpong: a device-coherent
store seen on another XCD, L_post):

  general step  expansion: L_img x 2 when it reads hashed tables (the
                fingerprint word, then the bucket), else L_img (a scanned
                child's label); a shared step adds 2 L_post (the post seen
                by the helpers, their done count seen by the leader)
                selection: 2 L_l2 when it cuts (a histogram pass and a
                gather pass over the pushes)
                emit: L_l2 (the push) + 2 L_img (the node record, then the
                pending token of a link parent)
  step 0        with the root directory (a root that is not scanned, and
                FT_ROOT_DIR not 0): expansion L_img (the token's entry),
                emit 2 L_l2 (the push, then the same entry again)
  tail step     L_l2 / 4 (a round of up to four steps reads its rows once)
  start         L_img (the root's entry) ; output: (mean length / 2 + 1)
                L_l2 (the history walk, two tokens a record)

What the floor leaves out is the time the leader's single-CU phases spend
issuing their reads: a CU keeps a bounded number of reads in flight (the
calibrated gather rate), so a phase of R random reads costs about R x
(ns per read) beyond its chain.

    python step_profile.py [--config paper] [--model example] [--requests 256]
                           [--reps 3] [--no-calib]
"""
import argparse
import os
import re
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)


def calibrate():
    """(L_img, L_l2, L_post) in microseconds, from ft_copy_calib."""
    exe = os.path.join(HERE, "ft_copy_calib")
    out = {}
    for mib, key in ((32768, "img"), (4, "l2")):
        txt = subprocess.run([exe, "chase", str(mib), "100000"], check=True,
                             capture_output=True, text=True).stdout
        print("  " + txt.strip(), flush=True)
        out[key] = float(re.search(r"plain ([\d.]+) ns", txt).group(1)) / 1e3
    txt = subprocess.run([exe, "pingpong", "20000"], check=True, capture_output=True,
                         text=True).stdout
    print("  " + txt.strip().replace("\n", "\n  "), flush=True)
    other = re.findall(r"another XCD\): \d+ of \d+ rounds, ([\d.]+) ns", txt)
    out["post"] = float(other[0]) / 1e3 if other else 0.45
    for mode in (0, 1):
        txt = subprocess.run([exe, "gather", "32768", "1", "16", str(mode)], check=True,
                             capture_output=True, text=True).stdout
        print("  " + txt.strip(), flush=True)
    return out["img"], out["l2"], out["post"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="paper")
    ap.add_argument("--model", default="example")
    ap.add_argument("--requests", type=int, default=256)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--no-calib", action="store_true",
                    help="use L_img 0.40, L_l2 0.09, L_post 0.45 us")
    a = ap.parse_args()
    import flashtrie as ft
    import workloads as wl

    print(f"library {os.path.relpath(ft.__file__, os.path.dirname(HERE))} build "
          f"{ft.build_id()}", flush=True)
    if a.no_calib:
        L_img, L_l2, L_post = 0.40, 0.09, 0.45
    else:
        print("calibration (ft_copy_calib):", flush=True)
        L_img, L_l2, L_post = calibrate()
    print(f"L_img {L_img:.3f} us, L_l2 {L_l2:.3f} us, L_post {L_post:.3f} us", flush=True)

    beam = {"c1": 10, "c2": 100}.get(a.config, 1000)
    T = wl.STEPS[a.config]
    trie = wl.trie(ft, a.config)
    trie.init_tbs_gpu(8, max_num_topk=beam, max_num_outpos=T, max_num_out_beams=beam,
                      max_num_out_tokens=beam * T, max_num_inter_beams=beam * T * 4)
    beams, ids, lp = wl.requests(ft, trie, a.config, a.model, 0, a.requests, beam)
    tok_thr, sent_thr, alpha, early = wl.RULES[a.config]
    P = a.requests
    ft.reserve_staging(trie, P)
    ft.stage(trie, beams, ids, lp, tok_thr, sent_thr, alpha, early)
    for _ in range(a.reps):
        for first in range(P):
            ft.launch(trie, first, 1)
        ft.sync(trie)
    cnt, norms, lens, toks, timing = ft.fetch(trie)
    dev = timing["device_ms"] * 1e3
    ss = timing["step_stats"].astype(np.float64)
    tick_us = 0.01  # wall clock: 100 MHz
    print(f"\n{a.config} {a.model}, beam {beam}, {P} requests one per launch (last of "
          f"{a.reps} passes), device clocks (us): expansion {dev[:, 0].mean():.2f}, "
          f"selection {dev[:, 1].mean():.2f}, other {dev[:, 2].mean():.2f}, total "
          f"{dev[:, 3].mean():.2f}; results {cnt.mean():.1f}", flush=True)
    lens_mean = float(np.mean([lens[r, :cnt[r]].mean() for r in range(P) if cnt[r]]))
    print(" t  parents        W    next     new  children  buckets  exp_us  sel_us  "
          "claims_us slices_us  | floor: exp   sel  emit   (us)")
    floor = L_img  # start: the root's entry
    meas = 0.0
    for t in range(T):
        m = ss[:, t, :].mean(0)
        if m[0] == 0 and m[2] == 0 and m[4] == 0:
            continue
        general = ss[:, t, 5].max() > 0
        shared = m[8] > 0 or m[9] > 0
        cut = m[2] > ss[:, min(t + 1, T - 1), 0].mean() + 0.5 if t + 1 < T else False
        root_dir = t == 0 and m[6] == 0 and os.environ.get("FT_ROOT_DIR", "") != "0"
        if general:
            fe = L_img * (2 if m[7] > 0 and not root_dir else 1) + (2 * L_post if shared else 0.0)
            fs = 2 * L_l2 if cut else 0.0
            fm = 2 * L_l2 if root_dir else L_l2 + 2 * L_img
        else:
            fe, fs, fm = L_l2 / 4, 0.0, 0.0
        floor += fe + fs + fm
        meas += (m[4] + m[5]) * tick_us
        print(f"{t:2d} {m[0]:8.1f} {m[1]:8.0f} {m[2]:7.1f} {m[3]:7.1f} {m[6]:9.0f} {m[7]:8.0f} "
              f"{m[4] * tick_us:7.2f} {m[5] * tick_us:7.2f} {m[8] * tick_us:9.2f} "
              f"{m[9] * tick_us:9.2f}  |  {fe:5.2f} {fs:5.2f} {fm:5.2f}"
              + ("" if general else "   (single-wave tail)"))
    out_floor = (lens_mean / 2 + 1) * L_l2
    floor += out_floor
    print(f"\nsteps measured {meas:.2f} us (expansion + selection), device total "
          f"{dev[:, 3].mean():.2f} us")
    print(f"latency floor {floor:.2f} us = {floor / 1e3:.4f} ms (start {L_img:.2f}, output "
          f"{out_floor:.2f}, steps {floor - L_img - out_floor:.2f}); measured / floor = "
          f"{dev[:, 3].mean() / floor:.1f}")


if __name__ == "__main__":
    main()
