"""Per-kernel duration summary of a rocprofv3 results database.

rocprofv3 --kernel-trace writes a rocpd SQLite database; its --stats CSV is
written at process exit, which a cooperative launch can pre-empt (rocprofv3
then ends with SIGSEGV after the program's own exit).  This prints the same
figures from the database: calls, total, mean, min, max, p50 and p99 of the
dispatch durations per kernel and grid size.

With --runs it prints the same figures per run of consecutive dispatches
that share kernel and grid size, in dispatch order (the benchmark separates
its batch sizes with one launch of a different grid).

With --pmc it prints, per kernel, grid size and counter, the mean value per
dispatch of the counters a `rocprofv3 --pmc` run collected (FETCH_SIZE and
WRITE_SIZE are in KiB); with --pmc --runs, per run of consecutive dispatches
(in dispatch order) that share kernel and grid size.

Usage: python flash-trie_amd/rocpd_summary.py [--runs] [--pmc] <results.db> [name-filter]
"""

import sqlite3
import sys

import numpy as np


def summary(db, name_filter=""):
    con = sqlite3.connect(db)
    rows = con.execute(
        "select name, grid_x, workgroup_x, lds_size, vgpr_count, sgpr_count, "
        "duration from kernels").fetchall()
    groups = {}
    for name, gx, wx, lds, vgpr, sgpr, dur in rows:
        if name_filter and name_filter not in name:
            continue
        key = (name, gx // max(wx, 1), wx, lds, vgpr, sgpr)
        groups.setdefault(key, []).append(dur)
    out = []
    for (name, wgs, wx, lds, vgpr, sgpr), d in sorted(
            groups.items(), key=lambda kv: -sum(kv[1])):
        d = np.array(d, dtype=np.float64) / 1e3  # ns -> us
        out.append({"kernel": name, "workgroups": wgs, "wg_size": wx,
                    "lds": lds, "vgpr": vgpr, "sgpr": sgpr, "calls": d.size,
                    "total_us": d.sum(), "mean_us": d.mean(), "min_us": d.min(),
                    "max_us": d.max(), "p50_us": np.percentile(d, 50),
                    "p99_us": np.percentile(d, 99)})
    return out


def run_summary(db, name_filter=""):
    con = sqlite3.connect(db)
    rows = con.execute(
        "select name, grid_x, workgroup_x, lds_size, vgpr_count, sgpr_count, "
        "duration from kernels order by start").fetchall()
    runs = []
    for name, gx, wx, lds, vgpr, sgpr, dur in rows:
        if name_filter and name_filter not in name:
            continue
        key = (name, gx // max(wx, 1), wx, lds, vgpr, sgpr)
        if not runs or runs[-1][0] != key:
            runs.append((key, []))
        runs[-1][1].append(dur)
    out = []
    for i, ((name, wgs, wx, lds, vgpr, sgpr), d) in enumerate(runs):
        d = np.array(d, dtype=np.float64) / 1e3
        out.append({"kernel": name, "run": i, "workgroups": wgs, "wg_size": wx,
                    "lds": lds, "vgpr": vgpr, "sgpr": sgpr, "calls": d.size,
                    "total_us": d.sum(), "mean_us": d.mean(), "min_us": d.min(),
                    "max_us": d.max(), "p50_us": np.percentile(d, 50),
                    "p99_us": np.percentile(d, 99)})
    return out


def pmc_summary(db, name_filter="", runs=False):
    """Mean counter value per dispatch, per (kernel, grid size) -- or, with
    runs, per run of consecutive dispatches of one kernel and grid size
    (a dispatch's counters are taken together, whatever their number)."""
    con = sqlite3.connect(db)
    rows = con.execute(
        "select dispatch_id, kernel_name, grid_size, workgroup_size, counter_name, value "
        "from counters_collection order by dispatch_id").fetchall()
    disp = {}
    for did, name, grid, wg, counter, value in rows:
        if name_filter and name_filter not in name:
            continue
        d = disp.setdefault(did, [(name, grid // max(wg, 1)), {}])
        d[1][counter] = d[1].get(counter, 0.0) + value
    groups = []  # [(key, {counter: [values]})]
    index = {}
    for did in sorted(disp):
        key, vals = disp[did]
        if runs:
            if not groups or groups[-1][0] != key:
                groups.append((key, {}))
            g = groups[-1][1]
        else:
            if key not in index:
                index[key] = len(groups)
                groups.append((key, {}))
            g = groups[index[key]][1]
        for c, v in vals.items():
            g.setdefault(c, []).append(v)
    out = []
    for (name, wgs), counters in groups:
        for counter in sorted(counters):
            v = np.array(counters[counter], dtype=np.float64)
            out.append({"kernel": name, "workgroups": wgs, "counter": counter,
                        "dispatches": v.size, "mean": v.mean(), "min": v.min(),
                        "max": v.max()})
    return out


def main():
    args = [a for a in sys.argv[1:] if a not in ("--pmc", "--runs")]
    if not args:
        print(__doc__)
        sys.exit(1)
    if "--pmc" in sys.argv:
        res = pmc_summary(args[0], args[1] if len(args) > 1 else "", "--runs" in sys.argv)
        print(f"{'kernel':<40} {'WGs':>5} {'counter':<12} {'dispatches':>10} "
              f"{'mean':>14} {'min':>14} {'max':>14}")
        for r in res:
            print(f"{r['kernel'][:40]:<40} {r['workgroups']:>5} {r['counter']:<12} "
                  f"{r['dispatches']:>10} {r['mean']:>14.1f} {r['min']:>14.1f} "
                  f"{r['max']:>14.1f}")
        return
    runs = "--runs" in sys.argv
    res = (run_summary if runs else summary)(args[0], args[1] if len(args) > 1 else "")
    if runs:
        print(f"{'run':>3} ", end="")
    print(f"{'kernel':<40} {'WGs':>4} {'calls':>6} {'total_us':>11} "
          f"{'mean_us':>9} {'min_us':>9} {'p50_us':>9} {'p99_us':>9} "
          f"{'max_us':>9}  lds/vgpr/sgpr")
    for r in res:
        if runs:
            print(f"{r['run']:>3} ", end="")
        print(f"{r['kernel'][:40]:<40} {r['workgroups']:>4} {r['calls']:>6} "
              f"{r['total_us']:>11.1f} {r['mean_us']:>9.2f} {r['min_us']:>9.2f} "
              f"{r['p50_us']:>9.2f} {r['p99_us']:>9.2f} {r['max_us']:>9.2f}  "
              f"{r['lds']}/{r['vgpr']}/{r['sgpr']}")


if __name__ == "__main__":
    main()
