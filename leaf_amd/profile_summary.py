"""Summarize a rocprofv3 kernel-trace database (rocpd SQLite) per kernel.

    python -m leaf_amd.profile_summary path/to/run_results.db [--top N]

Prints launches, average / min / total duration per kernel name, sorted by
total time: the same figures `rocprofv3 --stats` reports.
"""
from __future__ import annotations

import argparse
import sqlite3


def summarize(db_path: str, top: int = 30) -> str:
    db = sqlite3.connect(db_path)
    rows = db.execute("select name, count(*), avg(end - start), min(end - start), sum(end - start) "
                      "from kernels group by name order by sum(end - start) desc").fetchall()
    total = sum(r[4] for r in rows) or 1
    out = [f"{'launches':>9} {'avg_us':>9} {'min_us':>9} {'total_ms':>10} {'share':>6}  kernel"]
    for name, n, avg, mn, tot in rows[:top]:
        short = name.replace("leafhip::(anonymous namespace)::", "")
        short = short.split("(")[0] if "(" in short else short
        out.append(f"{n:9d} {avg / 1e3:9.2f} {mn / 1e3:9.2f} {tot / 1e6:10.3f} {100 * tot / total:5.1f}%  {short}")
    return "\n".join(out)


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("db")
    parser.add_argument("--top", type=int, default=30)
    args = parser.parse_args()
    print(summarize(args.db, args.top))


if __name__ == "__main__":
    main()
