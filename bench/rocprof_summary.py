#!/usr/bin/env python
"""Summarize a rocprofv3 kernel trace (the *_kernel_trace.csv of `rocprofv3 --kernel-trace`) per kernel
and launch shape: dispatches, mean / median / min / max duration (End - Start).  Writes a markdown
table, and with --json the same figures as JSON (bench.py reads the headline GEMM's mean from
profiles/gemm_prefill_p512_kernel_trace.json as the roofline's primary kernel time).

    python bench/rocprof_summary.py TRACE.csv [--top 12] [--match SUBSTR] [--json OUT.json --source MD]
"""
from __future__ import annotations

import argparse
import csv
import json
import re
import statistics


def short(name):
    """Kernel name without its parameter list and the leading 'void '."""
    n = re.sub(r"^void ", "", name)
    depth, out = 0, []
    for ch in n:
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    return "".join(out).strip()


def summarize(path, match=None):
    groups = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = short(row["Kernel_Name"])
            if match and match not in name:
                continue
            key = (name, int(row["Grid_Size_X"]), int(row["Workgroup_Size_X"]))
            groups.setdefault(key, []).append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    out = []
    for (name, grid, wg), d in groups.items():
        out.append({"kernel": name, "grid_x": grid, "workgroup_x": wg, "work_groups": grid // max(wg, 1),
                    "dispatches": len(d), "total_us": round(sum(d), 1), "mean_us": round(statistics.fmean(d), 3),
                    "median_us": round(statistics.median(d), 3), "min_us": round(min(d), 3), "max_us": round(max(d), 3)})
    out.sort(key=lambda r: -r["total_us"])
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("trace")
    ap.add_argument("--top", type=int, default=12)
    ap.add_argument("--match", default=None, help="only kernels whose name contains this")
    ap.add_argument("--json", default=None, help="also write the rows as JSON to this path")
    ap.add_argument("--source", default=None, help="the markdown summary the JSON belongs to")
    args = ap.parse_args()
    rows = summarize(args.trace, args.match)
    total = sum(r["total_us"] for r in rows) or 1.0
    print("| kernel | work-groups x threads | dispatches | mean us | median us | min us | max us | share |")
    print("|---|---|---|---|---|---|---|---|")
    for r in rows[:args.top]:
        print(f"| `{r['kernel']}` | {r['work_groups']} x {r['workgroup_x']} | {r['dispatches']} | {r['mean_us']} | "
              f"{r['median_us']} | {r['min_us']} | {r['max_us']} | {100 * r['total_us'] / total:.1f}% |")
    if args.json:
        json.dump({"source": args.source, "trace": args.trace.split("/")[-1], "kernels": rows[:args.top]},
                  open(args.json, "w"), indent=1)


if __name__ == "__main__":
    main()
