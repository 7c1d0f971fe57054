#!/usr/bin/env python
"""Kernel-by-kernel attribution of the prefill forward, with a sum-of-parts validity guard after the
reference's bench/profile_forward.cu:153-189: the per-kernel times of one forward, summed, against the
whole forward timed without the tracer.

Three steps (the first two on the GPU box, the third anywhere):

  python bench/prefill_breakdown.py whole --backend int8 --T 512 --out gpurun_out/whole.json
      times N forwards untraced, one hipEvent pair per forward on the library's stream (median,
      [min, max]); nothing else runs between them.
  rocprofv3 --kernel-trace -d gpurun_out/pb -o run -f csv -- \\
      python3 bench/prefill_breakdown.py marked --backend int8 --T 512
      runs N forwards with a burst of empty marker kernels between them, so the trace splits into
      forwards.
  python bench/prefill_breakdown.py attribute gpurun_out/pb/run_kernel_trace.csv gpurun_out/whole.json
      per kernel (name and grid): calls per forward, median time per forward and share; then
      SUM = median over forwards of the summed kernel times, and the guard on SUM / whole:
      < 0.97 -> time between kernels that no kernel accounts for (launch gaps, host), shares of the
      whole are not shares of the kernels; > 1.25 -> the tracer serialized the forward, shares are
      weak evidence; else OK.  SUM is not a latency; the whole is.

The forward is gpt2_prefill_fill_cache on BASELINE's synthetic GPT-2-124M (plain body, seed 1234,
random ids), logits of the last row, the library's default settings.
"""
from __future__ import annotations

import argparse
import csv
import ctypes as C
import json
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
MARKER = "k_empty"


def setup(args):
    sys.path.insert(0, ROOT)
    sys.path.insert(0, HERE)
    import importlib

    import numpy as np

    import __graft_entry__
    pkg = __graft_entry__.load_package()
    synth = importlib.import_module(pkg.__name__ + ".synth")
    L = pkg.lib()
    model = pkg.Model(synth.make_body(seed=1234, plain=True))
    if args.backend == "int8":
        model.quantize()
    T = args.T
    kv, scr = pkg.KVCache(T), pkg.Scratch(T)
    d_ids = pkg.Dev.from_numpy(np.asarray(synth.token_ids(T, seed=1), np.int32))
    logits = pkg.Dev(50257 * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all = logits.ptr, 0
    be = pkg.backend(args.backend)

    def forward():
        L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, T, C.byref(scr.s), C.byref(caps))

    keep = (model, kv, scr, d_ids, logits, caps)
    return pkg, L, forward, keep


def cmd_whole(args):
    pkg, L, forward, keep = setup(args)
    hip = C.CDLL("libamdhip64.so")
    for name in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime", "hipEventDestroy"):
        getattr(hip, name).restype = C.c_int
    stream = C.c_void_p(L.gpt2_get_stream() if hasattr(L, "gpt2_get_stream") else None)
    for _ in range(args.warmup):
        forward()
    L.gpt2_sync()
    ev = [(C.c_void_p(), C.c_void_p()) for _ in range(args.iters)]
    for a, b in ev:
        assert hip.hipEventCreate(C.byref(a)) == 0 and hip.hipEventCreate(C.byref(b)) == 0
    for a, b in ev:
        hip.hipEventRecord(a, stream)
        forward()
        hip.hipEventRecord(b, stream)
    L.gpt2_sync()
    pkg.check("whole")
    ms = []
    for a, b in ev:
        t = C.c_float()
        assert hip.hipEventElapsedTime(C.byref(t), a, b) == 0
        ms.append(t.value)
        hip.hipEventDestroy(a)
        hip.hipEventDestroy(b)
    out = {"backend": args.backend, "T": args.T, "iters": args.iters, "median_ms": statistics.median(ms),
           "min_ms": min(ms), "max_ms": max(ms), "mean_ms": statistics.fmean(ms)}
    text = json.dumps(out)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")


def cmd_marked(args):
    pkg, L, forward, keep = setup(args)
    import harness
    H = harness.lib(pkg)
    ms = C.c_float()
    for _ in range(args.warmup):
        forward()
    for _ in range(args.iters):
        if H.gpt2_bench_empty(1, C.byref(ms)):
            raise RuntimeError("gpt2_bench_empty")
        forward()
    H.gpt2_bench_empty(1, C.byref(ms))
    L.gpt2_sync()
    pkg.check("marked")
    print(f"marked {args.iters} forwards ({args.backend}, T={args.T})", flush=True)


def short(name):
    sys.path.insert(0, HERE)
    from rocprof_summary import short as s
    return s(name)


def cmd_attribute(args):
    with open(args.whole) as f:
        whole = json.load(f)
    rows = []
    with open(args.trace, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), short(r["Kernel_Name"]),
                         int(r["Grid_Size_X"]) // max(int(r["Workgroup_Size_X"]), 1)))
    rows.sort()
    # forwards: the dispatches between two marker bursts
    fwds, cur, seen_marker = [], [], False
    for s, e, name, wgs in rows:
        if name == MARKER:
            if seen_marker and cur:
                fwds.append(cur)
            cur, seen_marker = [], True
            continue
        if seen_marker:
            cur.append((name, wgs, (e - s) / 1e3))
    n0 = len(fwds)
    fwds = fwds[args.skip:]
    if not fwds:
        raise SystemExit("no marked forwards in the trace")
    ops = {}
    for i, fw in enumerate(fwds):
        for name, wgs, us in fw:
            d = ops.setdefault((name, wgs), {})
            d[i] = d.get(i, 0.0) + us
    calls = {}
    for name, wgs, _ in fwds[0]:
        calls[(name, wgs)] = calls.get((name, wgs), 0) + 1
    sums = [sum(us for _, _, us in fw) for fw in fwds]
    sum_med = statistics.median(sums)
    table = []
    for key, per in ops.items():
        med = statistics.median([per.get(i, 0.0) for i in range(len(fwds))])
        table.append((med, key, calls.get(key, 0)))
    table.sort(key=lambda t: -t[0])
    attributed = sum(t[0] for t in table) or 1.0
    w_us = whole["median_ms"] * 1e3
    print(f"Prefill forward, backend {whole['backend']}, T={whole['T']}: {len(fwds)} traced forwards "
          f"({n0} marked, {args.skip} skipped), {len(fwds[0])} kernels per forward.\n")
    print("| kernel | work-groups | calls | median us / forward | us / call | share |")
    print("|---|---|---|---|---|---|")
    for med, (name, wgs), c in table:
        print(f"| `{name}` | {wgs} | {c} | {med:.1f} | {med / max(c, 1):.2f} | {100 * med / attributed:.1f}% |")
    print(f"| SUM (per forward, median) | | {len(fwds[0])} | {sum_med:.1f} | | 100% |")
    ratio = sum_med / w_us
    print(f"\nWhole forward, untraced (hipEvent pair per forward, N={whole['iters']}): median {w_us:.1f} us "
          f"[{whole['min_ms'] * 1e3:.1f}, {whole['max_ms'] * 1e3:.1f}].")
    print(f"Validity: SUM / whole = {sum_med:.1f} / {w_us:.1f} = {ratio:.3f}")
    if ratio < 0.97:
        print(f"  SUM < whole by {100 * (1 - ratio):.1f}%: {w_us - sum_med:.1f} us per forward run no kernel "
              f"({w_us - sum_med:.1f} / {len(fwds[0]) - 1} = {(w_us - sum_med) / max(len(fwds[0]) - 1, 1):.2f} us "
              "per kernel boundary): the shares are shares of kernel time, not of the forward.")
    elif ratio > 1.25:
        print("  SUM > whole by more than 25%: the tracer serialized the forward; the shares are weak evidence.")
    else:
        print("  OK: the kernels account for the whole forward (within the tracer's own overhead); the shares "
              "are shares of the forward.  SUM is not a latency: the whole is.")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    for name in ("whole", "marked"):
        p = sub.add_parser(name)
        p.add_argument("--backend", default="int8", choices=["int8", "flash", "gemv", "tiled"])
        p.add_argument("--T", type=int, default=512)
        p.add_argument("--iters", type=int, default=50)
        p.add_argument("--warmup", type=int, default=5)
        if name == "whole":
            p.add_argument("--out", default=None)
    p = sub.add_parser("attribute")
    p.add_argument("trace")
    p.add_argument("whole")
    p.add_argument("--skip", type=int, default=2, help="marked forwards to drop at the start")
    args = ap.parse_args()
    {"whole": cmd_whole, "marked": cmd_marked, "attribute": cmd_attribute}[args.cmd](args)


if __name__ == "__main__":
    main()
