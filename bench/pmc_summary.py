#!/usr/bin/env python
"""Summaries of rocprofv3 counter runs (`--pmc`, *_counter_collection.csv) of the prefill GEMM set, per
GEMM shape.  The shape of each kernel comes from the bench line the profiled run printed (its
`gemm_shapes`: every trunk config serves one shape of the set).

  python bench/pmc_summary.py mfma PMC.csv RUN.json [--bench BENCH.json] [--clock-mhz 2400]
      SQ_INSTS_VALU_MFMA_MOPS_F16 (units of 512 FLOP), SQ_VALU_MFMA_BUSY_CYCLES (summed over the 1024
      SIMDs) per dispatch: FLOP issued against 2MNK, busy cycles per 1024 FLOP, and the matrix cores'
      utilisation over the dispatch (End - Start at the given clock).  --bench: an untraced bench line
      whose per-launch times are shown beside it.
  python bench/pmc_summary.py traffic FETCH.csv WRITE.csv RUN.json [--copy-bytes N] [--json OUT --source MD]
      FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled by what the same counter reads for the
      harness's copy kernel of N bytes (k_copy16, `bench.py --copy-probe N`), against the algorithmic
      bytes (A, W and bias read, C written once).  --json writes what bench.py's roofline reads.
"""
from __future__ import annotations

import argparse
import csv
import importlib.util
import json
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, HERE)
from rocprof_summary import short  # noqa: E402

LABEL = {"qkv": "QKV", "attn_proj": "attn-proj", "fc": "fc", "mlp_proj": "mlp-proj"}


def bench_module():
    spec = importlib.util.spec_from_file_location("bench_main", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def last_json(path):
    with open(path) as f:
        lines = [ln for ln in f.read().splitlines() if ln.startswith("{")]
    return json.loads(lines[-1])


def shapes_by_kernel(run_json):
    """{template name (as rocprofv3 prints it, without the namespace): shape dict} from a bench line."""
    cfg_tag = bench_module().cfg_tag
    out = {}
    for x in last_json(run_json)["gemm_shapes"]:
        tag = cfg_tag(x["kernel"])
        if tag:
            out[tag] = x
    return out


def counters(path):
    """{(kernel, counter): [value per dispatch]} and {kernel: [duration us per dispatch]}."""
    vals, dur, seen = {}, {}, set()
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            name = short(r["Kernel_Name"]).removeprefix("g2::")
            vals.setdefault((name, r["Counter_Name"]), []).append(float(r["Counter_Value"]))
            key = (name, r["Dispatch_Id"])
            if key not in seen:
                seen.add(key)
                dur.setdefault(name, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return vals, dur


def shape_label(x):
    return f"{LABEL.get(x['gemm'], x['gemm'])} {x['M']}x{x['N']}x{x['K']}"


def cmd_mfma(a):
    vals, dur = counters(a.csv)
    shapes = shapes_by_kernel(a.run)
    bench_us = {}
    if a.bench:
        for x in last_json(a.bench)["gemm_shapes"]:
            bench_us[(x["N"], x["K"])] = x["us"]
    print("| kernel | shape | dispatches | MOPS_F16 x 512 (FLOP) | algorithmic 2MNK | MFMA busy cycles | "
          "busy x 1024 / FLOP | kernel us (counter run) | MFMA util over kernel | bench us per launch | "
          "FLOP / (peak x launch) |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    for tag, x in shapes.items():
        mops = vals.get((tag, "SQ_INSTS_VALU_MFMA_MOPS_F16"))
        busy = vals.get((tag, "SQ_VALU_MFMA_BUSY_CYCLES"))
        if not mops or not busy:
            continue
        flop = statistics.fmean(mops) * 512
        algo = 2.0 * x["M"] * x["N"] * x["K"]
        b = statistics.fmean(busy)
        us = statistics.median(dur[tag])
        util = b / (1024 * us * a.clock_mhz)
        bu = bench_us.get((x["N"], x["K"]))
        frac = f"{algo / (2500e12 * bu * 1e-6):.3f}" if bu else "-"
        print(f"| `{tag}` | {shape_label(x)} | {len(mops)} | {flop:.4g} | {algo:.4g} | {b:.4g} | "
              f"{b * 1024 / flop:.3f} | {us:.2f} | {util:.3f} | {bu if bu else '-'} | {frac} |")


def cmd_traffic(a):
    fv, _ = counters(a.fetch)
    wv, _ = counters(a.write)
    copy_f = statistics.fmean(fv[("k_copy16", "FETCH_SIZE")])
    copy_w = statistics.fmean(wv[("k_copy16", "WRITE_SIZE")])
    kib = a.copy_bytes / 1024
    fs, ws = kib / copy_f, kib / copy_w
    print(f"Calibration: `k_copy16` copies {a.copy_bytes} B ({kib:.0f} KiB read + {kib:.0f} KiB written). It reads "
          f"FETCH_SIZE = {copy_f:.1f} KiB and WRITE_SIZE = {copy_w:.1f} KiB, so the scale factors are {fs:.3f} (fetch) "
          f"and {ws:.3f} (write).\n")
    print("| kernel | shape | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | scaled read MB | scaled write MB | "
          "algorithmic read MB | algorithmic write MB | traffic / algorithmic |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    out = {"source": a.source, "fetch_scale": fs, "write_scale": ws, "per_shape": {}}
    for tag, x in shapes_by_kernel(a.run).items():
        f = fv.get((tag, "FETCH_SIZE"))
        w = wv.get((tag, "WRITE_SIZE"))
        if not f or not w:
            continue
        M, N, K = x["M"], x["N"], x["K"]
        fk, wk = statistics.fmean(f), statistics.fmean(w)
        rd, wr = fk * fs * 1024, wk * ws * 1024
        ard, awr = (M * K + N * K + N) * 2, M * N * 2
        print(f"| `{tag}` | {shape_label(x)} | {len(f)} | {fk:.1f} | {wk:.1f} | {rd / 1e6:.2f} | {wr / 1e6:.2f} | "
              f"{ard / 1e6:.2f} | {awr / 1e6:.2f} | {(rd + wr) / (ard + awr):.2f} |")
        out["per_shape"][shape_label(x)] = {"kernel": tag, "fetch_kib": fk, "write_kib": wk, "bytes": round(rd + wr),
                                            "read_bytes": round(rd), "write_bytes": round(wr),
                                            "algo_read_bytes": ard, "algo_write_bytes": awr}
    if a.json:
        with open(a.json, "w") as fo:
            json.dump(out, fo, indent=1)
            fo.write("\n")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("mfma")
    p.add_argument("csv")
    p.add_argument("run", help="stdout of the profiled bench.py run (its JSON line)")
    p.add_argument("--bench", default=None, help="an untraced bench line, for the per-launch times")
    p.add_argument("--clock-mhz", type=float, default=2400.0)
    p = sub.add_parser("traffic")
    p.add_argument("fetch")
    p.add_argument("write")
    p.add_argument("run", help="stdout of one of the profiled bench.py runs (its JSON line)")
    p.add_argument("--copy-bytes", type=int, default=268435456)
    p.add_argument("--json", default=None)
    p.add_argument("--source", default=None)
    a = ap.parse_args()
    {"mfma": cmd_mfma, "traffic": cmd_traffic}[a.cmd](a)


if __name__ == "__main__":
    main()
