#!/usr/bin/env python
"""Summaries of rocprofv3 counter runs (`--pmc`, *_counter_collection.csv): the prefill GEMM set per GEMM
shape (the shape of each kernel comes from the bench line the profiled run printed, its
`gemm_shapes`: every trunk config serves one shape of the set), and the decode GEMV legs.

  python bench/pmc_summary.py mfma PMC.csv RUN.json [--bench BENCH.json] [--clock-mhz 2400]
      SQ_INSTS_VALU_MFMA_MOPS_F16 (units of 512 FLOP), SQ_VALU_MFMA_BUSY_CYCLES (summed over the 1024
      SIMDs) per dispatch: FLOP issued against 2MNK, busy cycles per 1024 FLOP, and the matrix cores'
      utilisation over the dispatch (End - Start at the given clock).  --bench: an untraced bench line
      whose per-launch times are shown beside it.
  python bench/pmc_summary.py traffic FETCH.csv WRITE.csv RUN.json [--copy-bytes N] [--json OUT --source MD]
      FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled by what the same counter reads for the
      harness's copy kernel of N bytes (k_copy16, `bench.py --copy-probe N`), against the algorithmic
      bytes (A, W and bias read, C written once).  --json writes what bench.py's roofline reads.
  python bench/pmc_summary.py gemv FETCH.csv WRITE.csv TRACE.csv [--copy-bytes N]
      the decode GEMV legs (`bench.py --gemv-only`): per k_gemv kernel and grid, the shape from its
      template arguments and grid (N rows of K), FETCH_SIZE / WRITE_SIZE (median per dispatch),
      scaled, against the algorithmic bytes, with the kernel-trace median duration.
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


GEMV_LEGS = {(2304, 768): "QKV", (768, 768): "attn-proj", (3072, 768): "fc", (768, 3072): "mlp-proj",
             (50257, 768): "tied head"}


def gemv_shape(name, grid, wg):
    """(N, K, INT8) of a k_gemv<LPR, CPL, U, QW, ...> dispatch: rows per work-group (64/LPR) * U *
    (wg/64), K = LPR * CPL * 16 bytes of weights per row; N = the rows the grid covers (a multiple of
    the rows per work-group: the last one may be partial, so N is matched to the known legs)."""
    import re
    m = re.search(r"k_gemv<(\d+), (\d+), (\d+), (true|false)", name)
    if not m:
        return None
    lpr, cpl, u, qw = int(m.group(1)), int(m.group(2)), int(m.group(3)), m.group(4) == "true"
    rows_wg = (64 // lpr) * u * (wg // 64)
    k = lpr * cpl * 16 // (1 if qw else 2)
    cover = (grid // wg) * rows_wg
    for (n, kk) in GEMV_LEGS:
        if kk == k and cover - rows_wg < n <= cover:
            return n, k, qw
    return None


def cmd_gemv(a):
    def rows(path):
        with open(path, newline="") as f:
            return list(csv.DictReader(f))
    fet, wri, tr = rows(a.fetch), rows(a.write), rows(a.trace)
    def copy_val(rs, counter):
        v = [float(r["Counter_Value"]) for r in rs if short(r["Kernel_Name"]) == "k_copy16" and r["Counter_Name"] == counter]
        return statistics.fmean(v)
    kib = a.copy_bytes / 1024
    fs, ws = kib / copy_val(fet, "FETCH_SIZE"), kib / copy_val(wri, "WRITE_SIZE")
    def by_leg(rs, key_grid, key_wg, val):
        out = {}
        for r in rs:
            nm = short(r["Kernel_Name"])
            if "k_gemv<" not in nm:
                continue
            sh = gemv_shape(nm, int(r[key_grid]), int(r[key_wg]))
            if sh:
                out.setdefault((nm, sh), []).append(val(r))
        return out
    f = by_leg(fet, "Grid_Size", "Workgroup_Size", lambda r: float(r["Counter_Value"]))
    w = by_leg(wri, "Grid_Size", "Workgroup_Size", lambda r: float(r["Counter_Value"]))
    t = by_leg(tr, "Grid_Size_X", "Workgroup_Size_X", lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print(f"Calibration: `k_copy16` copying {a.copy_bytes} B reads FETCH_SIZE = {kib / fs:.1f} KiB and WRITE_SIZE = "
          f"{kib / ws:.1f} KiB, so the scale factors are {fs:.3f} (fetch) and {ws:.3f} (write).\n")
    print("| leg | kernel | dispatches | FETCH_SIZE KiB (median) | WRITE_SIZE KiB | scaled bytes | algorithmic bytes "
          "| ratio | kernel us (trace median) |")
    print("|---|---|---|---|---|---|---|---|---|")
    order = sorted(f, key=lambda k: (not k[1][2], k[1][0] == 50257, list(GEMV_LEGS).index(k[1][:2])))
    for key in order:
        nm, (n, k, qw) = key
        fk, wk = statistics.median(f[key]), statistics.median(w.get(key, [0.0]))
        scaled = fk * fs * 1024 + wk * ws * 1024
        head = n == 50257
        bias = 0 if head else 2 * n
        algo = (n * k + 4 * n + 2 * k + 2 * n + bias) if qw else (2 * n * k + 2 * k + 2 * n + bias)
        us = statistics.median(t[key]) if key in t else float("nan")
        leg = f"{'INT8' if qw else 'fp16'} {GEMV_LEGS[(n, k)]} {k}x{n}"
        print(f"| {leg} | `{nm}` | {len(f[key])} | {fk:.1f} | {wk:.2f} | {scaled / 1e6:.3f} MB | {algo / 1e6:.3f} MB | "
              f"{scaled / algo:.3f} | {us:.2f} |")


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
    p = sub.add_parser("gemv")
    p.add_argument("fetch")
    p.add_argument("write")
    p.add_argument("trace")
    p.add_argument("--copy-bytes", type=int, default=268435456)
    p = sub.add_parser("traffic")
    p.add_argument("fetch")
    p.add_argument("write")
    p.add_argument("run", help="stdout of one of the profiled bench.py runs (its JSON line)")
    p.add_argument("--copy-bytes", type=int, default=268435456)
    p.add_argument("--json", default=None)
    p.add_argument("--source", default=None)
    a = ap.parse_args()
    {"mfma": cmd_mfma, "traffic": cmd_traffic, "gemv": cmd_gemv}[a.cmd](a)


if __name__ == "__main__":
    main()
