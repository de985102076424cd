"""Summarise rocprofv3 result databases (rocpd SQLite) as short text.

    python rocprof_summary.py stats <run_results.db> [--top N]
    python rocprof_summary.py pmc <run_results.db> [--kernel REGEX]

``stats`` prints per-kernel call count, total and average duration (us, as
rocprofv3 stores them in ``top_kernels``);
``pmc`` prints the per-dispatch average of each collected counter per kernel.
"""

from __future__ import annotations

import argparse
import collections
import re
import sqlite3


def _short(name: str, width: int = 70) -> str:
    name = re.sub(r"\(anonymous namespace\)::", "", name)
    base = name.split("(")[0]
    return base[:width]


def stats(db: str, top: int) -> str:
    c = sqlite3.connect(db)
    rows = list(c.execute(
        "select name, total_calls, total_duration, average, percentage from top_kernels"))
    out = [f"{'kernel':70s} {'calls':>6s} {'total_us':>10s} {'avg_us':>9s} {'pct':>6s}"]
    for name, calls, total, avg, pct in rows[:top]:
        out.append(f"{_short(name):70s} {calls:6d} {total:10.1f} {avg:9.3f} {pct:6.2f}")
    return "\n".join(out)


def pmc(db: str, kernel: str | None) -> str:
    c = sqlite3.connect(db)
    agg = collections.defaultdict(list)
    for k, n, v in c.execute("select kernel_name, counter_name, value from counters_collection"):
        if kernel and not re.search(kernel, k):
            continue
        agg[(_short(k), n)].append(v)
    out = [f"{'kernel':60s} {'counter':>11s} {'n':>4s} {'avg':>12s} {'median':>12s} {'max':>12s}"]
    for (k, n), vs in agg.items():
        med = sorted(vs)[len(vs) // 2]
        out.append(f"{k[:60]:60s} {n:>11s} {len(vs):4d} {sum(vs)/len(vs):12.1f} {med:12.1f} "
                   f"{max(vs):12.1f}")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("what", choices=["stats", "pmc"])
    ap.add_argument("db")
    ap.add_argument("--top", type=int, default=15)
    ap.add_argument("--kernel", default=None)
    a = ap.parse_args()
    print(stats(a.db, a.top) if a.what == "stats" else pmc(a.db, a.kernel))


if __name__ == "__main__":
    main()
