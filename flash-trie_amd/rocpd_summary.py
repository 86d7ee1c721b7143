"""Per-kernel duration summary of a rocprofv3 results database.

rocprofv3 --kernel-trace writes a rocpd SQLite database; its --stats CSV is
written at process exit, which a cooperative launch can pre-empt (rocprofv3
then ends with SIGSEGV after the program's own exit).  This prints the same
figures from the database: calls, total, mean, min, max, p50 and p99 of the
dispatch durations per kernel and grid size.

Usage: python flash-trie_amd/rocpd_summary.py <results.db> [name-filter]
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


def main():
    if len(sys.argv) < 2:
        print(__doc__)
        sys.exit(1)
    res = summary(sys.argv[1], sys.argv[2] if len(sys.argv) > 2 else "")
    print(f"{'kernel':<40} {'WGs':>4} {'calls':>6} {'total_us':>11} "
          f"{'mean_us':>9} {'min_us':>9} {'p50_us':>9} {'p99_us':>9} "
          f"{'max_us':>9}  lds/vgpr/sgpr")
    for r in res:
        print(f"{r['kernel'][:40]:<40} {r['workgroups']:>4} {r['calls']:>6} "
              f"{r['total_us']:>11.1f} {r['mean_us']:>9.2f} {r['min_us']:>9.2f} "
              f"{r['p50_us']:>9.2f} {r['p99_us']:>9.2f} {r['max_us']:>9.2f}  "
              f"{r['lds']}/{r['vgpr']}/{r['sgpr']}")


if __name__ == "__main__":
    main()
