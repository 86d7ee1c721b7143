#!/usr/bin/env python3
"""Trie beam search benchmark on one MI355X.

The reference publishes its latency at the C++ boundary and its throughput
at harness wall time (its README.md:48-64; tools/bindings.cpp:90-100;
examples/run_trie_search.py:189-199).  Both are measured here, each at its
own boundary, with the reference's protocol (examples/flashtrie_bench.py:
270-291): per configuration one warm-up pass and --passes measured passes
over the configuration's seeded synthetic requests, statistics computed
within each pass and averaged across passes.

  value         peak requests/s over batch sizes 1, 2, 4, 8 at beam 1000 at
                the reference's throughput boundary, harness wall time: per
                batch the requests' numpy rows turned into Python lists
                (.tolist(), examples/flashtrie_bench.py:203) and
                flashtrie.bs_tbs_gpu called; q/s = requests of a pass / its
                wall time.  vs_baseline = value / the A100's 1,539 q/s.
  latency_ms    batch-1 latency at beam 1000 at the reference's latency
                boundary, C++ wall time around Trie::tbs_gpu_batched (mean
                and p99), plus the harness's per-call figures
  cpp_boundary  the peak q/s at the C++ boundary (no Python lists), with
                its own ratio to 1,539
  harness_numpy the harness loop passing the numpy arrays it holds to
                bs_tbs_gpu (which reads them in place) instead of lists
  boundary      every proposal model and beam width at both boundaries
  device_resident  kernel-only figures (inputs already in HBM, HIP events)
  roofline      algorithmic bytes per launch / average launch duration of
                the search kernel against the 8 TB/s HBM peak
  cpu_baseline  the CPU oracle (a restatement of the reference's
                LoudsTrie::tbs) on the host cores: the fast variant on a
                bounded sample on up to 16 threads, and the as-written cost
                model (a thread per parent, linear sibling scan) on a few
                requests
  configs       the other workloads (C2, the stress trie, C1), each with its
                own boundary sweep, kernel, roofline and CPU figures

steps / warmup / ms_per_step count harness calls at the peak batch (the
measured passes and the warm-up pass); --steps / --warmup size the
device-resident launches per batch size.

Workloads (--configs, the first is the headline):
  paper   800M unique keys over a 2.2M-token vocabulary, key length 3-16
          (mean ~6), Zipf(1.05) prefix sharing; beam = K = 1000, 16 steps
  c2      10M keys over a 256k vocabulary, length 4-12, Zipf(1.1); beam =
          K = 100, 12 steps
  stress  200M keys, 2.2M-child root, length 16-32; beam = K = 1000, 32
          steps, early exit, thresholds -4 / -20
  c1      100k keys over a 32k vocabulary, length 3-8; beam 10, K = 32,
          8 steps

Proposal models (--models): "example", the shape of the reference's example
generator (examples/make_example_data.py:119-145; one seeded key path per
beam slot, forced tokens U(-2.2,-0.2), distractors U(-12,-4)); "literal",
the configuration as stated: log-softmax of N(0, sigma^2) logits over the
vocabulary with 30% of the mass on one seeded key path.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs ...]
"""

import argparse
import gc
import json
import os
import re
import sys
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flash-trie_amd"))

METRIC = "mean/p99 trie-search ms @800M keys, beam 1000; peak q/s over batch 1-8"
HBM_PEAK_GBS = 8000.0
# the reference on an A100 (README.md:48-64): batch-1 mean / p99 ms and
# peak q/s over batch 1-8, per beam width
PUBLISHED = {1000: (1.91, 3.31, 1539.0), 500: (1.36, 2.04, 2571.0),
             100: (0.56, 0.70, 5754.0)}

import workloads as wl  # noqa: E402

ALPHA = 5.0
# per workload: token / sentence log-prob thresholds and early exit
RULES = {k: (v[0], v[1], v[3]) for k, v in wl.RULES.items()}

# per workload: description, beam, K, requests per pass, batch sizes,
# proposal models, other beam widths swept, as-written CPU sample
SPEC = {
    "paper": dict(desc="800M unique keys, 2.2M vocab, key length 3-16 (mean ~6), "
                       "Zipf(1.05) prefix sharing", beam=1000, topk=1000,
                  requests=13000, batches=(1, 2, 4, 8), models=("example", "literal"),
                  widths=(100, 500), as_written=2),
    "c2": dict(desc="10M-key trie, 256k vocab, key length 4-12, Zipf(1.1)", beam=100,
               topk=100, requests=1000, batches=(1, 2, 4, 8), models=("literal", "example"),
               widths=(), as_written=8),
    "stress": dict(desc="stress: 200M-key trie, 2.2M vocab (heavy-fanout root), key "
                        "length 16-32, Zipf(1.05) prefix sharing; early exit, "
                        "thresholds -4 / -20", beam=1000, topk=1000, requests=1000,
                   batches=(1, 8), models=("literal", "example"), widths=(), as_written=2),
    "c1": dict(desc="100k-key trie, 32k vocab, key length 3-8, Zipf(1.1) (the CPU "
                    "plumbing configuration)", beam=10, topk=32, requests=200,
               batches=(1, 8), models=("literal",), widths=(), as_written=200),
}


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200,
                   help="timed device-resident launches per batch size")
    p.add_argument("--warmup", type=int, default=20,
                   help="untimed device-resident launches per batch size")
    p.add_argument("--configs", default="paper,c2,stress,c1",
                   help="workloads, the first one the headline")
    p.add_argument("--config", default=None, help="one workload only (= --configs X)")
    p.add_argument("--requests", type=int, default=0,
                   help="requests per pass of the headline workload (0: its own)")
    p.add_argument("--passes", type=int, default=2, help="measured passes")
    p.add_argument("--models", default="", help="proposal models (empty: the workload's)")
    p.add_argument("--batches", default="", help="batch sizes (empty: the workload's)")
    p.add_argument("--beam-sweep", default=None,
                   help="other beam widths of the headline (K = beam), empty to skip")
    p.add_argument("--sweep-requests", type=int, default=4000,
                   help="requests per pass for the other beam widths")
    p.add_argument("--no-harness", action="store_true",
                   help="skip the harness-wall (Python) sweeps")
    p.add_argument("--pool", type=int, default=512,
                   help="requests staged in HBM for the device-resident runs")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--cpu-threads", type=int, default=16,
                   help="cap on CPU-baseline threads (the box's CPU share)")
    p.add_argument("--as-written-seconds", type=float, default=30.0,
                   help="time cap of the as-written CPU sample per workload")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--child-index", default="records", choices=["records", "louds"],
                   help="child ranges from the node records or from the LOUDS "
                        "rank/select directory (switched off: its kernel faulted "
                        "once and the cause is not found)")
    return p.parse_args()


def device_free_bytes():
    """Free device memory (hipMemGetInfo on the current device), or None."""
    import ctypes
    try:
        hip = ctypes.CDLL("libamdhip64.so")
    except OSError:
        return None
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    if hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) != 0:
        return None
    return free.value


def measured_traffic(cfg, batch, build_id):
    """HBM bytes per launch of the search kernel at this batch size, from
    rocprofv3 FETCH_SIZE + WRITE_SIZE runs scaled by the same counters of a
    copy kernel of known size, as committed in the counter summary -- only
    when that summary was recorded on the library measured here (its
    build_id line); None otherwise."""
    path = os.path.join(ROOT, "profiles", f"tbs_kernel_{cfg}_traffic.txt")
    if not os.path.exists(path):
        return None
    text = open(path).read()
    m = re.search(r"^build_id\s*=\s*([0-9a-f]+)", text, re.M)
    if not m or m.group(1) != build_id:
        return None
    pat = re.compile(r"^traffic_bytes_per_launch\[(\d+)\]\s*=\s*(\d+)", re.M)
    for b, v in pat.findall(text):
        if int(b) == batch:
            return int(v)
    return None


def pass_stats(call_ms, batch):
    """Per-pass statistics averaged across passes (flashtrie_bench.py:
    270-291): q/s = requests of a pass / the sum of its call times; mean
    and p99 of the per-call milliseconds."""
    qps = [batch * len(r) / (r.sum() * 1e-3) for r in call_ms]
    return {"qps": float(np.mean(qps)),
            "mean_ms": float(np.mean([r.mean() for r in call_ms])),
            "p99_ms": float(np.mean([np.percentile(r, 99) for r in call_ms])),
            "qps_passes": [round(x, 1) for x in qps]}


def boundary_sweep(ft, trie, beams, ids, lp, batches, rules, passes, what):
    """The C++ boundary: bench_boundary times each Trie::tbs_gpu_batched call
    where bs_tbs_gpu times it; returns per batch size the pass statistics
    and the results' hashes (last pass)."""
    tok_thr, sent_thr, early = rules
    out, hashes = {}, {}
    for b in batches:
        n = len(beams) - len(beams) % b
        cm, ps, cnt, hs = ft.bench_boundary(trie, beams[:n], ids[:n], lp[:n], b,
                                            tok_thr, sent_thr, ALPHA, early, 1,
                                            passes)
        st = pass_stats(cm, b)
        st["wall_qps"] = float(np.mean(n / ps))
        out[b] = st
        hashes[b] = (cnt, hs)
        log(f"{what} batch {b}: {st['qps']:.0f} q/s at the C++ boundary "
            f"(passes {st['qps_passes']}), mean {st['mean_ms']:.3f} ms "
            f"p99 {st['p99_ms']:.3f} ms per call")
    b0 = batches[0]
    same = all(np.array_equal(hashes[b][1], hashes[b0][1][:len(hashes[b][1])])
               for b in batches)
    return out, hashes, same


def harness_sweep(ft, trie, beams, ids, lp, batches, rules, passes, lists, what):
    """Harness wall time (examples/run_trie_search.py:189-199): per batch,
    the requests' rows handed to flashtrie.bs_tbs_gpu -- as Python lists
    made by .tolist() when `lists` (what examples/flashtrie_bench.py:203
    does), else as the numpy arrays -- and the call's results dropped.  One
    warm-up pass and `passes` measured ones; q/s = requests / pass wall."""
    tok_thr, sent_thr, early = rules
    out = {}
    for b in batches:
        n = len(beams) - len(beams) % b
        walls, calls = [], []
        for p in range(1 + passes):
            cms = np.empty(n // b)
            t0 = time.perf_counter()
            for k, b0 in enumerate(range(0, n, b)):
                c0 = time.perf_counter()
                if lists:
                    r = ft.bs_tbs_gpu(trie, b, beams[b0:b0 + b].tolist(),
                                      ids[b0:b0 + b].tolist(), lp[b0:b0 + b].tolist(),
                                      tok_thr, sent_thr, ALPHA, early)
                else:
                    r = ft.bs_tbs_gpu(trie, b, beams[b0:b0 + b], ids[b0:b0 + b],
                                      lp[b0:b0 + b], tok_thr, sent_thr, ALPHA, early)
                del r
                cms[k] = (time.perf_counter() - c0) * 1e3
            wall = time.perf_counter() - t0
            if p >= 1:
                walls.append(wall)
                calls.append(cms)
        qps = [n / w for w in walls]
        out[b] = {"qps": float(np.mean(qps)), "qps_passes": [round(x, 1) for x in qps],
                  "mean_ms": float(np.mean([c.mean() for c in calls])),
                  "p99_ms": float(np.mean([np.percentile(c, 99) for c in calls])),
                  "calls_per_pass": n // b}
        if lists:
            # the caller's own share of a call: the three .tolist() and the
            # release of the lists, with no search -- the wall this harness
            # cannot go below on this host
            fw = []
            for p in range(1 + passes):
                t0 = time.perf_counter()
                for b0 in range(0, n, b):
                    x = (beams[b0:b0 + b].tolist(), ids[b0:b0 + b].tolist(),
                         lp[b0:b0 + b].tolist())
                    del x
                if p >= 1:
                    fw.append(time.perf_counter() - t0)
            out[b]["caller_ms"] = float(np.mean(fw)) / (n // b) * 1e3
            out[b]["caller_only_qps"] = float(n / np.mean(fw))
            out[b]["search_ms"] = out[b]["mean_ms"] - out[b]["caller_ms"]
        log(f"{what} batch {b}: {out[b]['qps']:.0f} q/s harness wall "
            f"({'lists' if lists else 'numpy'}; passes {out[b]['qps_passes']}), "
            f"mean {out[b]['mean_ms']:.3f} ms p99 {out[b]['p99_ms']:.3f} ms per call"
            + (f"; the lists alone {out[b]['caller_ms']:.3f} ms a call "
               f"({out[b]['caller_only_qps']:.0f} q/s with no search)" if lists else ""))
    return out


def fnv_results(sents, norms):
    """The hash bench_boundary computes over one request's results."""
    h = 0xcbf29ce484222325
    m = (1 << 64) - 1

    def mix(w):
        nonlocal h
        h = ((h ^ w) * 0x100000001b3) & m
    mix(len(sents))
    bits = np.asarray(norms, dtype=np.float64).view(np.uint64)
    for s, nb in zip(sents, bits):
        mix(len(s))
        for tk in s:
            mix(int(tk))
        nb = int(nb)
        mix(nb & 0xFFFFFFFF)
        mix(nb >> 32)
    return h


def oracle_of(trie):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    return pyoracle, pyoracle.OracleTrie.from_trie(trie)


def cpu_info():
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    return model, os.cpu_count() or 1, aff


def run_oracle(ot, reqs, rules, seconds, threads, with_work=False, variant=None):
    """Runs the oracle over reqs (list of (beams, ids, lp)) on `threads`
    host threads until done or `seconds` pass (a request started is
    finished); returns ({index: (sents, norms)}, works, elapsed seconds)."""
    tok_thr, sent_thr, early = rules
    done, works, lock, nxt = {}, [], threading.Lock(), [0]
    deadline = time.time() + seconds
    kw = {} if variant is None else {"variant": variant}

    def worker():
        while time.time() < deadline:
            with lock:
                r = nxt[0]
                nxt[0] += 1
            if r >= len(reqs):
                return
            bm, i_, l_ = reqs[r]
            res = ot.tbs(bm, i_, l_, tok_thr, sent_thr, ALPHA, early,
                         with_work=with_work, **kw)
            with lock:
                done[r] = res[:2]
                if with_work:
                    works.append(res[2])

    t0 = time.time()
    th = [threading.Thread(target=worker) for _ in range(threads)]
    [x.start() for x in th]
    [x.join() for x in th]
    return done, works, time.time() - t0


def check_hashes(chk, hashes):
    """Requests of `chk` ({r: (sents, norms)}) whose results differ from the
    timed results' hashes at any batch size."""
    bad = 0
    for r, (s_, n_) in chk.items():
        hv = fnv_results(s_, n_)
        for b, (cn, hs) in hashes.items():
            if r < len(hs) and (int(hs[r]) != hv or int(cn[r]) != len(s_)):
                bad += 1
                break
    return bad


def fmt_sweep(sw):
    keys = ("qps", "mean_ms", "p99_ms", "wall_qps")
    return {str(b): {k: round(v[k], 4 if k.endswith("_ms") else 1) for k in keys if k in v}
            for b, v in sw.items()}


def run_workload(ft, cfg, args, headline):
    """Every measurement of one workload; returns its record and the
    headline figures."""
    spec = SPEC[cfg]
    rules = RULES[cfg]
    B, K, T = spec["beam"], spec["topk"], wl.STEPS[cfg]
    n_req = (args.requests or spec["requests"]) if headline else spec["requests"]
    batches = ([int(x) for x in args.batches.split(",")] if args.batches and headline
               else list(spec["batches"]))
    models = ([m for m in args.models.split(",") if m] if args.models and headline
              else list(spec["models"]))
    widths = (list(spec["widths"]) if args.beam_sweep is None
              else [int(x) for x in args.beam_sweep.split(",") if x.strip()])
    widths = [w for w in widths if w < B] if headline else list(spec["widths"])
    t0 = time.time()
    os.environ["FT_SYNTH_VERBOSE"] = "1"  # per-level progress on stderr
    trie = wl.trie(ft, cfg)
    log(f"{cfg}: trie of {trie.num_keys()} keys, {trie.num_nodes()} nodes, "
        f"{trie.total_size() / 2**30:.2f} GiB image, {time.time() - t0:.1f}s")
    if args.child_index == "louds":
        os.environ["FT_CHILD_INDEX"] = "louds"
    free0 = device_free_bytes()
    t0 = time.time()
    # (at least 3: an untimed 3-request launch separates the runs of a trace)
    trie.init_tbs_gpu(max(max(batches), 3), max_num_topk=K, max_num_outpos=T,
                      max_num_out_beams=B, max_num_out_tokens=B * T,
                      max_num_inter_beams=B * T)
    free1 = device_free_bytes()
    info = trie.device_info()
    dev_bytes = (free0 - free1) if free0 is not None and free1 is not None else None
    log(f"{cfg}: device {info}; context ready in {time.time() - t0:.1f}s; "
        f"{(dev_bytes or 0) / 2**30:.2f} GiB of device memory")

    # ---- both boundaries, per proposal model --------------------------------
    boundary, reqsets, hashsets = {}, {}, {}
    for model in models:
        t0 = time.time()
        beams, ids, lp = wl.requests(ft, trie, cfg, model, 0, n_req, B, K)
        log(f"{cfg} {model}: {n_req} requests generated in {time.time() - t0:.1f}s")
        what = f"{cfg} {model} beam {B}"
        sweep, hashes, same = boundary_sweep(ft, trie, beams, ids, lp, batches, rules,
                                             args.passes, what)
        rec = {"cpp_boundary": fmt_sweep(sweep), "same_results_every_batch": same}
        if not args.no_harness:
            # (the headline model over every request; the others over at
            # most --sweep-requests, as the other beam widths)
            nh = n_req if model == models[0] else min(n_req, args.sweep_requests)
            rec["harness_lists"] = harness_sweep(ft, trie, beams[:nh], ids[:nh], lp[:nh],
                                                 batches, rules, args.passes, True, what)
            rec["harness_numpy"] = harness_sweep(ft, trie, beams[:nh], ids[:nh], lp[:nh],
                                                 batches, rules, args.passes, False, what)
        boundary[model] = {B: rec}
        reqsets[model] = (beams, ids, lp)
        hashsets[model] = hashes
        boundary[model][B]["_sweep"] = sweep
    head = models[0]

    # ---- device-resident runs (kernel-only figures) --------------------------
    beams, ids, lp = reqsets[head]
    P = min(args.pool, n_req)
    ft.reserve_staging(trie, P)
    ft.stage(trie, beams[:P], ids[:P], lp[:P], *rules[:2], ALPHA, rules[2])
    ft.launch(trie, 0, 1)
    ft.sync(trie)
    dev_qps, kern_ms = {}, {}
    for b in batches:
        nb = P // b
        # an untimed batch-3 launch before each batch size splits a kernel
        # trace into one run of dispatches per batch size
        ft.launch(trie, 0, min(3, P))
        for i in range(args.warmup):
            ft.launch(trie, (i % nb) * b, b)
        ft.sync(trie)
        t1 = time.perf_counter()
        for i in range(args.steps):
            ft.launch(trie, (i % nb) * b, b)
        ft.sync(trie)
        el = time.perf_counter() - t1
        dev_qps[b] = args.steps * b / el
        kern_ms[b] = ft.launch_times(trie, min(args.steps, 1024))
        log(f"{cfg} device-resident batch {b}: {dev_qps[b]:.0f} q/s, kernel mean "
            f"{kern_ms[b].mean():.3f} ms p99 {np.percentile(kern_ms[b], 99):.3f} ms")
    dev_peak = max(dev_qps, key=dev_qps.get)
    tick_ms = 1.0 / info["wall_clock_khz"]
    # per-step device profile of the pool at batch 1 and at the largest batch
    phase = {}
    for pb in sorted({1, max(batches)}):
        ft.launch(trie, 0, min(3, P))  # a separator in kernel traces
        used = P - P % pb
        for first in range(0, used, pb):
            ft.launch(trie, first, pb)
        if used < P:
            ft.launch(trie, used, P - used)
        ft.sync(trie)
        cnt, norms, lens, toks, timing = ft.fetch(trie)
        dev = timing["device_ms"]
        phase[str(pb)] = {"expand_ms": float(dev[:, 0].mean()),
                          "select_ms": float(dev[:, 1].mean()),
                          "other_ms": float(dev[:, 2].mean()),
                          "device_total_ms": float(dev[:, 3].mean())}
        ss = timing["step_stats"].astype(np.float64)
        if headline:
            log(f"per step at batch {pb} (mean over the pool): parents, work, next, "
                "sel, expand_ms, select_ms, children, probes, claim_wait_ms, "
                "done_wait_ms")
        steps_tab = []
        for t in range(ss.shape[1]):
            m = ss[:, t, :].mean(axis=0)
            steps_tab.append([round(float(x), 1) for x in m[:4]] +
                             [round(float(x * tick_ms), 4) for x in (m[4], m[5])] +
                             [round(float(x), 1) for x in m[6:8]] +
                             [round(float(x * tick_ms), 4) for x in m[8:10]])
            if headline:
                log(f"  step {t:2d}: {m[0]:7.1f} {m[1]:9.1f} {m[2]:7.1f} {m[3]:6.1f} "
                    f"{m[4] * tick_ms:7.4f} {m[5] * tick_ms:7.4f} {m[6]:9.1f} {m[7]:9.1f} "
                    f"{m[8] * tick_ms:7.4f} {m[9] * tick_ms:7.4f}")
        phase[str(pb)]["steps"] = steps_tab
        log(f"{cfg} phases per request at batch {pb} (ms): "
            f"{ {k: round(v, 4) for k, v in phase[str(pb)].items() if k != 'steps'} }")

    # ---- other beam widths at both boundaries --------------------------------
    for w in widths:
        for model in models:
            bw, iw, lw = wl.requests(ft, trie, cfg, model, 100000 * w, args.sweep_requests, w)
            what = f"{cfg} {model} beam {w}"
            sweep, hashes, same = boundary_sweep(ft, trie, bw, iw, lw, batches, rules,
                                                 args.passes, what)
            rec = {"cpp_boundary": fmt_sweep(sweep), "same_results_every_batch": same,
                   "_sweep": sweep}
            if not args.no_harness:
                rec["harness_lists"] = harness_sweep(ft, trie, bw, iw, lw, batches, rules,
                                                     args.passes, True, what)
                rec["harness_numpy"] = harness_sweep(ft, trie, bw, iw, lw, batches, rules,
                                                     args.passes, False, what)
            boundary[model][w] = rec
            reqsets[(model, w)] = (bw, iw, lw)
            hashsets[(model, w)] = hashes

    # ---- CPU oracle: both variants, parity, work counters ---------------------
    cpu, parity, algo_bytes, wstats = None, {}, None, {}
    if not args.no_cpu:
        pyoracle, ot = oracle_of(trie)
        model_name, nproc, aff = cpu_info()
        threads = max(1, min(args.cpu_threads, aff))
        hb, hi, hl = reqsets[head]
        sample = [(hb[r], hi[r], hl[r]) for r in range(n_req)]
        log(f"{cfg} cpu baseline (fast variant): {threads} threads for at most "
            f"{args.cpu_seconds:.0f}s")
        done, works, cpu_el = run_oracle(ot, sample, rules, args.cpu_seconds,
                                         threads, with_work=True)
        lat1 = []
        for r in range(min(3, n_req)):
            t1 = time.perf_counter()
            ot.tbs(hb[r], hi[r], hl[r], *rules[:2], ALPHA, rules[2])
            lat1.append((time.perf_counter() - t1) * 1e3)
        # the reference's own cost model: requests one after another (it
        # spawns and joins a thread per parent, so one core at a time)
        n_aw = min(spec["as_written"], n_req)
        aw_thr = min(n_aw, threads) if n_aw <= 4 else 1
        log(f"{cfg} cpu baseline (as-written variant): up to {n_aw} requests on "
            f"{aw_thr} thread(s), at most {args.as_written_seconds:.0f}s")
        t1 = time.time()
        aw_done, _, aw_el = run_oracle(ot, sample[:n_aw], rules, args.as_written_seconds,
                                       aw_thr, variant=pyoracle.AS_WRITTEN)
        aw_el = time.time() - t1
        # per-request time: the sample's requests ran aw_thr at a time, each
        # on one core at a time (its per-parent threads are joined at once)
        aw_ms = aw_el * 1e3 * aw_thr / len(aw_done) if aw_done else None
        cpu = {
            "value": len(done) / cpu_el, "unit": "q/s", "cores": threads, "kind": "port",
            "sample": f"{len(done)} of the {n_req} {head}-model requests at beam {B} in "
                      f"{cpu_el:.1f}s on {threads} threads (oracle, fast variant: binary "
                      f"sibling search, one thread per request); 1-thread latency "
                      f"{np.mean(lat1):.2f} ms",
            "fast": {"qps": round(len(done) / cpu_el, 2), "threads": threads,
                     "requests": len(done), "seconds": round(cpu_el, 2),
                     "latency_ms_1thread": round(float(np.mean(lat1)), 3)},
            "as_written": {"qps_per_core": round(1e3 / aw_ms, 4) if aw_ms else None,
                           "ms_per_request": round(aw_ms, 1) if aw_ms else None,
                           "requests": len(aw_done), "seconds": round(aw_el, 2),
                           "cores": aw_thr,
                           "what": "the reference's cost model (louds-trie.cc:120, 155-163, "
                                   "810-856): a thread spawned and joined per parent, "
                                   "linear sibling scan; one core per request, "
                                   f"{aw_thr} request(s) at a time"},
            "host": {"cpu_model": model_name, "nproc": nproc, "affinity_cpus": aff,
                     "thread_cap": args.cpu_threads,
                     "pinning": "none (the process's affinity mask)"}}
        log(f"{cfg} cpu: fast {cpu['fast']['qps']} q/s on {threads} threads; as-written "
            f"{cpu['as_written']['ms_per_request']} ms per request")
        # parity: every sampled request's timed results (last pass, at every
        # batch size) against the oracle's, both variants
        for model in models:
            mb_, mi, ml = reqsets[model]
            if model == head:
                chk = done
            else:
                chk, _, _ = run_oracle(ot, [(mb_[r], mi[r], ml[r])
                                            for r in range(min(512, n_req))],
                                       rules, args.cpu_seconds, threads)
            bad = check_hashes(chk, hashsets[model])
            parity[model] = {"checked": len(chk), "mismatches": bad, "batches": batches}
            log(f"{cfg} parity {model}: {len(chk)} requests, {bad} mismatches")
        parity["as_written"] = {"checked": len(aw_done),
                                "mismatches": check_hashes(aw_done, hashsets[head])}
        for key in [k for k in reqsets if isinstance(k, tuple)]:
            bw, iw, lw = reqsets[key]
            chk, _, _ = run_oracle(ot, [(bw[r], iw[r], lw[r]) for r in range(16)],
                                   rules, args.cpu_seconds, threads)
            bad = check_hashes(chk, hashsets[key])
            boundary[key[0]][key[1]]["parity"] = {"checked": len(chk), "mismatches": bad}
        # device-resident results of the pool against the oracle
        bad = 0
        for r, (s_, n_) in done.items():
            if r >= P:
                continue
            c = int(cnt[r])
            g = [toks[r, j, :lens[r, j]].tolist() for j in range(c)]
            bad += int(g != s_ or not np.array_equal(norms[r, :c], n_))
        parity["device_resident"] = {"checked": sum(r < P for r in done),
                                     "mismatches": bad}
        # algorithmic bytes per request (oracle work counters): 8K per row +
        # 16 per parent + 16 per non-link parent + 4 per child label touched
        # + 32 per candidate + 16 per survivor + result bytes
        W = np.array(works, dtype=np.float64)
        res_b = np.array([16 + 16 * len(s) + 4 * sum(map(len, s))
                          for s, _ in done.values()], dtype=np.float64)
        per_req = (W[:, 6] + 16 * W[:, 1] + 16 * (W[:, 1] - W[:, 2]) +
                   4 * W[:, 3] + 32 * W[:, 4] + 16 * W[:, 5] + res_b)
        algo_bytes = float(per_req.mean())
        wstats = {"steps": float(W[:, 0].mean()), "parents": float(W[:, 1].mean()),
                  "link_parents": float(W[:, 2].mean()),
                  "candidates": float(W[:, 4].mean()),
                  "results": float(np.mean([len(s) for s, _ in done.values()]))}

    build_id = ft.build_id()
    kb = kern_ms[dev_peak]
    roof = None
    if algo_bytes is not None:
        achieved = algo_bytes * dev_peak / (kb.mean() * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                "traffic": measured_traffic(cfg, dev_peak, build_id),
                "algorithmic_bytes_per_request": round(algo_bytes),
                "requests_per_launch": dev_peak,
                "launch_ms": round(float(kb.mean()), 4),
                "build_id": build_id}

    hs = boundary[head][B]["_sweep"]
    cpp_peak = max(hs, key=lambda b: hs[b]["qps"])
    l1 = hs.get(1, hs[cpp_peak])
    rec = {
        "workload": spec["desc"], "beam": B, "topk": K, "steps": T,
        "requests_per_pass": n_req, "passes": args.passes, "warmup_passes": 1,
        "batch_sizes": batches, "models": models, "headline_model": head,
        "thresholds": list(rules[:2]), "length_norm": ALPHA, "early_exit": rules[2],
        "latency_ms": {"mean": round(l1["mean_ms"], 4), "p99": round(l1["p99_ms"], 4),
                       "boundary": "C++ wall time around Trie::tbs_gpu_batched, batch 1",
                       "kernel_mean": round(float(kern_ms.get(1, kb).mean()), 4),
                       "kernel_p99": round(float(np.percentile(kern_ms.get(1, kb), 99)), 4)},
        "cpp_boundary_peak": {"qps": round(hs[cpp_peak]["qps"], 1), "batch": cpp_peak},
        "boundary": {m: {str(w): {k: v for k, v in d2.items() if not k.startswith("_")}
                         for w, d2 in d.items()} for m, d in boundary.items()},
        "device_resident": {"qps_by_batch": {str(b): round(v, 1) for b, v in dev_qps.items()},
                            "kernel_ms_by_batch": {str(b): round(float(v.mean()), 4)
                                                   for b, v in kern_ms.items()},
                            "kernel_p99_ms_by_batch": {
                                str(b): round(float(np.percentile(v, 99)), 4)
                                for b, v in kern_ms.items()},
                            "requests_pooled": P, "launches": args.steps,
                            "warmup_launches": args.warmup},
        "phases_ms_per_request": phase,
        "workload_stats": wstats,
        "parity": parity,
        "memory": {"image_bytes": trie.total_size(), "context_device_bytes": dev_bytes,
                   "child_index": args.child_index},
        "roofline": roof,
        "cpu_baseline": cpu,
        "device": info,
    }
    if not args.no_harness:
        hl_ = boundary[head][B]["harness_lists"]
        hp = max(hl_, key=lambda b: hl_[b]["qps"])
        rec["harness_peak"] = {"qps": round(hl_[hp]["qps"], 1), "batch": hp,
                               "mean_ms": round(hl_[hp]["mean_ms"], 4),
                               "calls_per_pass": hl_[hp]["calls_per_pass"]}
        hn = boundary[head][B]["harness_numpy"]
        hnp = max(hn, key=lambda b: hn[b]["qps"])
        rec["harness_numpy_peak"] = {"qps": round(hn[hnp]["qps"], 1), "batch": hnp}
        if 1 in hl_:
            rec["latency_ms"]["harness_mean"] = round(hl_[1]["mean_ms"], 4)
            rec["latency_ms"]["harness_p99"] = round(hl_[1]["p99_ms"], 4)
    for m in rec["boundary"].values():
        for w in m.values():
            for k in ("harness_lists", "harness_numpy"):
                if k in w:
                    w[k] = {str(b): {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                                     for kk, vv in v.items()} for b, v in w[k].items()}
    return rec


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: the search shards by request "
              "(a replicated trie, no exchange between GPUs), so the "
              f"aggregate is the per-GPU rate times the GPU count; --gpus "
              f"{args.gpus} is not run here", file=sys.stderr)
        sys.exit(2)
    import build as ftbuild
    if not ftbuild.built():
        ftbuild.build()
    import flashtrie as ft

    cfgs = [args.config] if args.config else [c for c in args.configs.split(",") if c]
    for c in cfgs:
        if c not in SPEC:
            sys.exit(f"unknown workload {c}")
    t_all = time.time()
    recs = {}
    for i, cfg in enumerate(cfgs):
        t0 = time.time()
        recs[cfg] = run_workload(ft, cfg, args, headline=(i == 0))
        gc.collect()  # the workload's trie and context are gone before the next
        log(f"{cfg}: measured in {time.time() - t0:.0f}s")
    head_cfg = cfgs[0]
    h = recs[head_cfg]
    B = h["beam"]
    pub = PUBLISHED.get(B) if head_cfg == "paper" else None
    if "harness_peak" in h:
        value, peak_b = h["harness_peak"]["qps"], h["harness_peak"]["batch"]
        ms_step, calls = h["harness_peak"]["mean_ms"], h["harness_peak"]["calls_per_pass"]
        value_def = ("harness wall q/s: per batch, the requests' numpy rows -> Python "
                     "lists (.tolist()) -> flashtrie.bs_tbs_gpu, results dropped; "
                     "requests of a pass / its wall time (examples/flashtrie_bench.py:203, "
                     "examples/run_trie_search.py:189-199)")
    else:
        value, peak_b = h["cpp_boundary_peak"]["qps"], h["cpp_boundary_peak"]["batch"]
        sw = h["boundary"][h["headline_model"]][str(B)]["cpp_boundary"][str(peak_b)]
        ms_step, calls = sw["mean_ms"], h["requests_per_pass"] // peak_b
        value_def = "C++ boundary q/s (--no-harness)"
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "q/s",
        "n_gpus": 1,
        "steps": calls * args.passes,
        "warmup": calls,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / pub[2], 3) if pub else None,
        "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": h["workload"], "beam": B, "topk": h["topk"],
                   "steps": h["steps"], "batch_sizes": h["batch_sizes"],
                   "peak_batch": peak_b, "requests_per_pass": h["requests_per_pass"],
                   "passes": args.passes, "warmup_passes": 1,
                   "headline_model": h["headline_model"], "models": h["models"],
                   "value": value_def,
                   "latency_boundary": "C++ wall time around Trie::tbs_gpu_batched "
                                       "(tools/bindings.cpp:90-100): staging, the kernel, "
                                       "output vectors",
                   "thresholds": h["thresholds"], "length_norm": ALPHA,
                   "early_exit": h["early_exit"]},
        "steps_count": "steps = harness calls timed at the peak batch (the measured "
                       "passes), warmup = those of the warm-up pass, ms_per_step = their "
                       "mean; --steps / --warmup size the device-resident launches per "
                       "batch size (device_resident.launches / warmup_launches)",
        "latency_ms": h["latency_ms"],
        "cpp_boundary": dict(h["cpp_boundary_peak"],
                             vs_published_a100_qps=round(h["cpp_boundary_peak"]["qps"] / pub[2], 3)
                             if pub else None),
        "harness_numpy": dict(h.get("harness_numpy_peak", {}),
                              vs_published_a100_qps=round(h["harness_numpy_peak"]["qps"] / pub[2], 3)
                              if pub and "harness_numpy_peak" in h else None),
        "published_a100": ({str(k): {"mean_ms": v[0], "p99_ms": v[1], "peak_qps": v[2]}
                            for k, v in PUBLISHED.items()} if head_cfg == "paper" else None),
        "boundary": h["boundary"],
        "device_resident": h["device_resident"],
        "phases_ms_per_request": h["phases_ms_per_request"],
        "workload_stats": h["workload_stats"],
        "parity": h["parity"],
        "device": h["device"],
        "memory": h["memory"],
        "roofline": h["roofline"],
        "cpu_baseline": h["cpu_baseline"],
        "configs": {c: r for c, r in recs.items() if c != head_cfg},
        "build_id": ft.build_id(),
        "bench_seconds": round(time.time() - t_all, 1),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
