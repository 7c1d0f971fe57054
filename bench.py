#!/usr/bin/env python
"""Benchmark of the MI355X matmul path of bare-metal-gpt2 (BASELINE.json metric).

Headline (`value`): fp16 prefill GEMM TFLOP/s at P=512 -- one step is the prefill's trunk GEMM set,
12 layers x {QKV 512x2304x768, attn-proj 512x768x768, fc 512x3072x768, mlp-proj 512x768x3072}
(+bias), each layer with its own weights, run back to back through gpt2_matmul_tiled.  Inputs are
resident in HBM before the timed region; timing is hipEvents on the launch stream around K steps.

Also reported in the same JSON line:
  step_stats    one hipEvent pair per step: mean (= ms_per_step), median and [min, max], with the
                TFLOP/s at each
  clock         the gfx clock amd-smi reports while the step runs back to back (median, [min, max])
  launch_floor_us  an empty kernel launched back to back (the per-launch floor of this box)
  roofline      the GEMM kernel with the largest share of the step, against 2500 TFLOP/s fp16 MFMA:
                `achieved` from its rocprof mean in profiles/gemm_prefill_p512_kernel_trace.json
                (the primary kernel time), this run's hipEvent launch average beside it
  gemm_set_graph_replay  the same step captured once as a hipGraph and replayed (no faster: the
                gap between dependent launches is the same inside a graph)
  gemv_int8     INT8 decode GEMV GB/s per trunk shape, cold (rotating > 512 MB of weight copies,
                so every launch streams from HBM) and warm (same weights every launch), beside the
                same shape with fp16 weights in alternating rounds (medians, [min, max], verdict), the
                48-GEMV trunk chain of one decode step, and the same kernel on the INT8 tied head
                (38.6 MB per launch, where the launch floor no longer hides the streaming rate)
  head_gemv     fp16 tied-head GEMV (77.3 MB) cold / warm
  gemm_int8_set the same P=512 trunk set with INT8 weights (the config-5 prefill GEMMs)
  head_gemm     the tied head as a prefill GEMM, [512x768] . [768x50257]^T (39.5 GFLOP)
  gemm_m_sweep  the four trunk GEMMs at M in {1, 16, 32, 64, 128, 256, 512, 1024}, fp16 and INT8
                weights, with the kernel each M takes (GEMV at M = 1, the skinny GEMM for short prompts)
  measured_peaks  this box's HBM read stream and fp16 MFMA issue rate, beside the datasheet peaks
  bandwidth_guard  every cold (HBM) GB/s leg against the measured read stream (the reference's bug
                line): legs above it are listed as suspicious
  attention_prefill  causal MFMA prefill attention per launch at T=512 and T=1024 (12 heads x 64)
  forward_t64   config 1 on the GPU: the fp16 forward at T=64 with logits for all 64 rows
  prefill       the whole prefill at P=512 (fp16 and INT8 trunk weights) and at P=128 with the
                LayerNorm fold at its default and off; prefill_trunk_gemm_tflops = the trunk's
                86.97 GFLOP / the fp16 P=512 forward (a lower bound: attention, LayerNorms, head row
                in the denominator)
  decode        GPT-2-124M decode tok/s @ctx=512: INT8 trunk + fp16 head, one hipGraph replay per
                token, after a P=512 prefill (the prefill itself is timed too); plus the mean over
                the 511-step greedy run, and (decode.cold) the same step with its weights cold:
                four uploads of the model stepped round robin, 650 MB of weights past the 256 MB MALL
  decode_fp16_vs_int8  the persistent step with fp16 and with INT8 trunk weights at ctx 128, 512 and
                1023, warm and cold, the fp16 and INT8 48-GEMV chains, and the INT8/fp16 ratios
  cpu_baseline  the reference's own cpu/forward_cpu.c matmul (oracle/_ref, if built) or the oracle
                restatement, on the same four GEMM shapes, on this host's cores
  cpu_forward_t64  config 1 on the CPU: the reference's forward at T=64 with logits_all (median of
                5 on every thread, one run on one thread), beside forward_t64
  cpu_decode_baseline  the reference's CPU decode @ctx=512 (no KV cache: a full forward over 513
                positions per token), tok/s beside the GPU decode leg

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extras]
       (--gemv-only and --decode-only run one leg, as the drivers of the committed counter profiles)
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "prefill GEMM TFLOP/s @P=512; INT8 decode GEMV HBM GB/s; decode tok/s @ctx=512"
PEAK_FP16_TFLOPS = 2500.0      # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
M_PREFILL = 512
GEMM_SET = [("qkv", 2304, 768), ("attn_proj", 768, 768), ("fc", 3072, 768), ("mlp_proj", 768, 3072)]
TRUNK_GEMV = [("qkv", 2304, 768), ("attn_proj", 768, 768), ("fc", 3072, 768), ("mlp_proj", 768, 3072)]
N_LAYER, VOCAB, N_EMBD = 12, 50257, 768


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_harness():
    """bench/harness.py (the binding of bench/libgpt2bench.so, the native timing loops)."""
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bench")
    if here not in sys.path:
        sys.path.insert(0, here)
    return importlib.import_module("harness")


class Bench:
    def __init__(self, pkg):
        self.pkg = pkg
        self.L = pkg.lib()
        self.harness = load_harness()
        self.H = self.harness.lib(pkg)    # timing loops and microbenchmarks (not the product library)
        self.keep = []

    def dev(self, a):
        d = self.pkg.Dev.from_numpy(a)
        self.keep.append(d)
        return d

    def empty(self, nbytes):
        d = self.pkg.Dev(nbytes)
        self.keep.append(d)
        return d

    def op(self, kind, Cb, A, W, Ws, bias, M, N, K):
        return self.harness.GPT2BenchOp(kind, Cb, A, W, Ws, bias, M, N, K)

    def run_ops(self, ops, warmup, iters, per_op=False):
        arr = (self.harness.GPT2BenchOp * len(ops))(*ops)
        ms = C.c_float()
        per = (C.c_float * len(ops))() if per_op else None
        rc = self.H.gpt2_bench_ops(arr, len(ops), warmup, iters, C.byref(ms),
                                   C.cast(per, C.POINTER(C.c_float)) if per_op else None)
        if rc:
            self.pkg.check("gpt2_bench_ops")
            raise RuntimeError(f"gpt2_bench_ops rc={rc}")
        return ms.value, (list(per) if per_op else None)

    def run_steps(self, ops, warmup, iters):
        """Per-round times (ms) of `iters` rounds of ops, each between its own pair of events on the
        launch stream, and the first-to-last total."""
        arr = (self.harness.GPT2BenchOp * len(ops))(*ops)
        per = (C.c_float * iters)()
        tot = C.c_float()
        rc = self.H.gpt2_bench_ops_steps(arr, len(ops), warmup, iters, per, C.byref(tot))
        if rc:
            self.pkg.check("gpt2_bench_ops_steps")
            raise RuntimeError(f"gpt2_bench_ops_steps rc={rc}")
        return list(per), tot.value

    def run_ops_graph(self, ops, warmup, iters):
        """Mean ms per round when one round is captured once as a hipGraph and replayed."""
        arr = (self.harness.GPT2BenchOp * len(ops))(*ops)
        ms = C.c_float()
        rc = self.H.gpt2_bench_ops_graph(arr, len(ops), warmup, iters, C.byref(ms))
        if rc:
            self.pkg.check("gpt2_bench_ops_graph")
            raise RuntimeError(f"gpt2_bench_ops_graph rc={rc}")
        return ms.value


def f16(rng, shape, std):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float16)


# ------------------------------------------------------------------------------ prefill GEMM set
def bench_gemm_set(B, steps, warmup, clock=True):
    rng = np.random.default_rng(1234)
    L = B.L
    X = B.dev(f16(rng, (M_PREFILL, 768), 1.0))
    Xf = B.dev(f16(rng, (M_PREFILL, 3072), 1.0))
    outs = {name: B.empty(M_PREFILL * N * 2) for name, N, K in GEMM_SET}
    ops = []
    for layer in range(N_LAYER):
        for name, N, K in GEMM_SET:
            W = B.dev(f16(rng, (N, K), 0.02))
            b = B.dev(f16(rng, N, 0.01))
            A = Xf if K == 3072 else X
            ops.append(B.op(0, outs[name].ptr, A.ptr, W.ptr, None, b.ptr, M_PREFILL, N, K))
    flops_step = sum(2.0 * M_PREFILL * N * K for _, N, K in GEMM_SET) * N_LAYER
    per_ms, total_ms = B.run_steps(ops, warmup, steps)
    ms_step = total_ms / steps
    tf = lambda ms: round(flops_step / (ms * 1e-3) / 1e12, 2)
    step_stats = {"mean_ms": round(ms_step, 5), "median_ms": round(float(np.median(per_ms)), 5),
                  "min_ms": round(min(per_ms), 5), "max_ms": round(max(per_ms), 5), "n": steps,
                  "tflops_median": tf(float(np.median(per_ms))), "tflops_at_min_max_ms": [tf(min(per_ms)), tf(max(per_ms))],
                  "timing": "one hipEvent pair per step on the launch stream (steps share their boundary events); "
                            "ms_per_step and value use the mean"}
    if clock:
        clock = sustained_clock(B, ops)
    else:
        clock = {"sclk_mhz": None, "method": "skipped (--no-clock)"}
    ms_graph = B.run_ops_graph(ops, warmup, steps)
    # Per-kernel launch durations for the roofline, under the step's own conditions: each shape's
    # 12 layer GEMMs (distinct weights, so the weights are not L2-resident) back to back.
    shapes = []
    by_cfg = {}
    for j, (name, N, K) in enumerate(GEMM_SET):
        ms_shape, _ = B.run_ops(ops[j::4], 3, max(20, steps // 4))
        ms = ms_shape / N_LAYER
        cfg = L.gpt2_tune_gemm_pick(M_PREFILL, N, K)
        cname = L.gpt2_tune_gemm_name(cfg).decode()
        fl = 2.0 * M_PREFILL * N * K
        shapes.append({"gemm": name, "M": M_PREFILL, "N": N, "K": K, "kernel": cname, "us": round(ms * 1e3, 3),
                       "tflops": round(fl / (ms * 1e-3) / 1e12, 2)})
        c = by_cfg.setdefault(cname, {"flops": 0.0, "ms": 0.0, "launches": 0})
        c["flops"] += fl
        c["ms"] += ms
        c["launches"] += 1
    dom = max(by_cfg.items(), key=lambda kv: kv[1]["ms"])
    d = dom[1]
    flops_launch = d["flops"] / d["launches"]
    live_us = d["ms"] / d["launches"] * 1e3
    achieved_live = flops_launch / (live_us * 1e-6) / 1e12
    # Primary time: the rocprofv3 kernel duration of this kernel in the committed trace of the same
    # workload (profiles/gemm_prefill_p512_kernel_trace.json); the hipEvent figure of this run beside it.
    prof = rocprof_kernel_time(dom[0])
    if prof:
        achieved = flops_launch / (prof["mean_us"] * 1e-6) / 1e12
        src = {"time_source": "rocprofv3 kernel duration (mean over dispatches)", "rocprof_mean_us": prof["mean_us"],
               "rocprof_median_us": prof["median_us"], "rocprof_dispatches": prof["dispatches"],
               "rocprof_profile": prof["source"]}
    else:
        achieved = achieved_live
        src = {"time_source": "hipEvents in this run (no committed rocprofv3 trace covers this kernel config)"}
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP16_TFLOPS, 4), "traffic": None,
                "kernel": dom[0], "flops_per_launch": flops_launch, **src,
                "avg_launch_us": round(live_us, 3), "achieved_live": round(achieved_live, 2),
                "frac_live": round(achieved_live / PEAK_FP16_TFLOPS, 4),
                "live_method": "hipEvents around 12 back-to-back launches of this shape (distinct weights), this run"}
    roofline.update(measured_traffic(dom[0], [x for x in shapes if x["kernel"] == dom[0]]))
    return flops_step, ms_step, shapes, roofline, ms_graph, step_stats, clock


def cfg_tag(cfg_name):
    """The kernel's template name (as rocprofv3 prints it) of a GEMM tile config name."""
    import re
    m = re.fullmatch(r"dl_bn(\d+)_bm(\d+)_w(\d+)x(\d+)_s(\d+)(?:_k(\d+))?(?:_u(\d+))?", cfg_name)
    if m:
        g = m.groups()
        return "k_gemm_dl<{}, {}, {}, {}, {}, false, {}, {}, 0>".format(*g[:5], g[5] or 1, g[6] or 1)
    m = re.fullmatch(r"bn(\d+)_bm(\d+)_bk(\d+)_w(\d+)x(\d+)_d(\d+)", cfg_name)
    if m:
        return "k_gemm_mfma<{}, {}, {}, {}, {}, false, {}, false>".format(*m.groups())
    return None


def rocprof_kernel_time(cfg_name):
    """Mean / median kernel duration of a GEMM config in the committed rocprofv3 trace of the headline
    workload (written by bench/rocprof_summary.py), or None when the trace does not cover it."""
    path = os.path.join(ROOT, "profiles", "gemm_prefill_p512_kernel_trace.json")
    try:
        prof = json.load(open(path))
    except (OSError, ValueError):
        return None
    tag = cfg_tag(cfg_name)
    for k in prof.get("kernels", []):
        if tag and k["kernel"].endswith(tag):
            return {"mean_us": k["mean_us"], "median_us": k["median_us"], "dispatches": k["dispatches"],
                    "source": prof["source"]}
    return None


def measured_traffic(cfg_name, shapes):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs (profiles/gemm_prefill_p512_hbm_traffic.md), averaged over the shapes that kernel
    serves in the step; null when that profile does not cover this kernel config."""
    path = os.path.join(ROOT, "profiles", "gemm_prefill_p512_hbm_traffic.json")
    try:
        prof = json.load(open(path))
    except (OSError, ValueError):
        return {}
    key = {(2304, 768): "QKV 512x2304x768", (3072, 768): "fc 512x3072x768", (768, 768): "attn-proj 512x768x768",
           (768, 3072): "mlp-proj 512x768x3072"}
    want = [prof["per_shape"].get(key.get((x["N"], x["K"]), ""), {}) for x in shapes]
    tag = cfg_tag(cfg_name)
    if not tag or not want or any(not w or w.get("kernel") != tag for w in want):
        return {}
    return {"traffic": round(sum(w["bytes"] for w in want) / len(want)), "traffic_source": prof["source"]}


def launch_floor_us(B, iters=2000):
    """An empty kernel (1 work-group) launched back to back on the launch stream: the per-launch floor
    every GEMM, GEMV and graph node of this line pays."""
    ms = C.c_float()
    if B.H.gpt2_bench_empty(iters, C.byref(ms)):
        B.pkg.check("gpt2_bench_empty")
    return round(ms.value * 1e3, 3)


def sustained_clock(B, ops, seconds=1.5):
    """The shader clock under the headline workload: the same step run back to back for `seconds`
    (untimed) while a second thread samples `amd-smi metric --clock` (one reading per XCD per sample);
    median / min / max over every XCD reading.  The timed steps themselves last milliseconds, shorter
    than one amd-smi call, so the clock is read under the same load right after them."""
    import threading
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            c = amd_smi_clocks()
            if not c:
                return
            samples.extend(v for k, v in c.items() if k.endswith(".clk.value") and isinstance(v, (int, float)))

    t = threading.Thread(target=sampler, daemon=True)
    t0 = time.perf_counter()
    t.start()
    n = 0
    while time.perf_counter() - t0 < seconds:
        B.run_ops(ops, 0, 20)
        n += 1
    stop.set()
    t.join(timeout=30)
    if not samples:
        return {"sclk_mhz": None, "method": "amd-smi unavailable"}
    return {"sclk_mhz_median": float(np.median(samples)), "sclk_mhz_min_max": [min(samples), max(samples)],
            "readings": len(samples), "load_s": round(time.perf_counter() - t0, 2),
            "method": "amd-smi metric --clock (every XCD's gfx clock) sampled in a thread while the headline step "
                      f"ran back to back ({n * 20} steps, untimed) right after the timed region"}


def amd_smi_clocks():
    """The GPU clocks as `amd-smi metric --clock` reports them right after the headline's timed region
    (the reference records the clock with every number, BENCH_PROTOCOL.md:64-72): the gfx entries of
    its JSON, flattened; None where amd-smi is absent or refuses."""
    import subprocess
    try:
        out = subprocess.run(["amd-smi", "metric", "--clock", "--json"], capture_output=True, text=True, timeout=20)
        data = json.loads(out.stdout)
    except (OSError, ValueError, subprocess.SubprocessError):
        return None
    flat = {}

    def walk(x, path):
        if isinstance(x, dict):
            for k, v in x.items():
                walk(v, f"{path}.{k}" if path else str(k))
        elif isinstance(x, list):
            for i, v in enumerate(x):
                walk(v, f"{path}[{i}]")
        elif "gfx" in path.lower() and len(flat) < 48:
            flat[path] = x
    walk(data, "")
    return flat or None


# ------------------------------------------------------------------------------ INT8 / fp16 GEMVs
def quantize_dev(B, w16_dev, N, K):
    q = B.empty(N * K)
    s = B.empty(N * 4)
    B.L.gpt2_quantize_rows(q.ptr, s.ptr, w16_dev.ptr, N, K)
    B.L.gpt2_sync()
    B.pkg.check("quantize")
    return q, s


def copies_for(nbytes, floor=600e6):
    return max(4, int(np.ceil(floor / nbytes)))


def bench_gemv(B, quick=False):
    """quick: a few launches per leg (the counter runs profile every dispatch).

    Per trunk shape, INT8 (gpt2_gemv_int8) against fp16 weights (gpt2_gemv_fp16), cold and warm, in
    alternating rounds (INT8 first on even rounds) so that a change of the box's state during the leg
    lands on both sides alike: a cold sample is one pass over the rotating copies (us per launch), a
    warm one the mean of a burst of launches on one copy; median and [min, max] per side, and the
    overlap verdict of bench/ab.py."""
    ab = importlib.import_module("ab")
    rng = np.random.default_rng(4321)
    rounds, n_cold, n_warm, n_chain, n_head = (1, 1, 20, 2, 10) if quick else (7, 5, 300, 200, 200)
    L = B.L
    res = {}
    x768 = B.dev(f16(rng, 768, 1.0))
    x3072 = B.dev(f16(rng, 3072, 1.0))
    y = B.empty(VOCAB * 2)
    chain = []

    for name, N, K in TRUNK_GEMV:
        x = x3072 if K == 3072 else x768
        w16 = B.dev(f16(rng, (N, K), 0.02))
        q, s = quantize_dev(B, w16, N, K)
        b = B.dev(f16(rng, N, 0.01))
        algo = N * K + 4 * N + 2 * K + 2 * N + 2 * N
        algo16 = 2 * N * K + 2 * K + 2 * N + 2 * N
        R, R16 = copies_for(N * K), copies_for(2 * N * K)
        big, big16 = B.empty(R * N * K), B.empty(R16 * N * K * 2)
        for r in range(R):
            L.gpt2_d2d(big.at(r * N * K), q.ptr, N * K)
        for r in range(R16):
            L.gpt2_d2d(big16.at(r * N * K * 2), w16.ptr, N * K * 2)
        L.gpt2_sync()
        cold = {8: [B.op(3, y.ptr, x.ptr, big.at(r * N * K), s.ptr, b.ptr, 1, N, K) for r in range(R)],
                16: [B.op(2, y.ptr, x.ptr, big16.at(r * N * K * 2), None, b.ptr, 1, N, K) for r in range(R16)]}
        warm = {8: [B.op(3, y.ptr, x.ptr, q.ptr, s.ptr, b.ptr, 1, N, K)], 16: [B.op(2, y.ptr, x.ptr, w16.ptr, None, b.ptr, 1, N, K)]}
        for d in (8, 16):
            B.run_ops(cold[d], 0, 1)
            B.run_ops(warm[d], 5, 5)
        sc, sw = {8: [], 16: []}, {8: [], 16: []}
        for rnd in range(rounds):
            for d in ((8, 16) if rnd % 2 == 0 else (16, 8)):
                ms, _ = B.run_ops(cold[d], 0, 1)
                sc[d].append(ms * 1e3 / len(cold[d]))
                ms, _ = B.run_ops(warm[d], 0, n_warm)
                sw[d].append(ms * 1e3)
        big.free()
        big16.free()
        c8, c16, w8, w16s = ab.stats(sc[8]), ab.stats(sc[16]), ab.stats(sw[8]), ab.stats(sw[16])
        res[name] = {"N": N, "K": K, "bytes": algo, "copies": R,
                     "cold_us": round(c8["median"], 3), "cold_us_min_max": [round(c8["min"], 3), round(c8["max"], 3)],
                     "cold_GBs": round(algo / (c8["median"] * 1e-6) / 1e9, 1),
                     "warm_us": round(w8["median"], 3), "warm_GBs": round(algo / (w8["median"] * 1e-6) / 1e9, 1)}
        res[name]["fp16"] = {"bytes": algo16, "copies": R16, "cold_us": round(c16["median"], 3),
                             "cold_us_min_max": [round(c16["min"], 3), round(c16["max"], 3)],
                             "cold_GBs": round(algo16 / (c16["median"] * 1e-6) / 1e9, 1),
                             "warm_us": round(w16s["median"], 3),
                             "warm_GBs": round(algo16 / (w16s["median"] * 1e-6) / 1e9, 1)}
        v = ab.verdict(c16, c8)
        res[name]["int8_speedup_cold"] = v["speedup_b_vs_a"]
        res[name]["cold_verdict"] = v["verdict"] if rounds >= 3 else "one round (quick run): no verdict"
        res[name]["int8_speedup_warm"] = ab.verdict(w16s, w8)["speedup_b_vs_a"]
        log(f"gemv {name}: {res[name]}")
    res["per_shape_method"] = (f"{rounds} alternating rounds per shape, INT8 first on even rounds; cold sample = one pass "
                               f"over the rotating copies, warm sample = mean of {n_warm} launches; medians")
    # the 48 INT8 GEMVs of one decode step, distinct weights per layer, back to back
    chain_bytes = 0
    for layer in range(N_LAYER):
        for name, N, K in TRUNK_GEMV:
            x = x3072 if K == 3072 else x768
            q = B.dev(rng.integers(-127, 128, (N, K), dtype=np.int8))
            s = B.dev(np.full(N, 1e-3, np.float32))
            b = B.dev(f16(rng, N, 0.01))
            chain.append(B.op(3, y.ptr, x.ptr, q.ptr, s.ptr, b.ptr, 1, N, K))
            chain_bytes += N * K + 4 * N + 2 * K + 4 * N
    ms_chain, _ = B.run_ops(chain, 2 if quick else 20, n_chain)
    res["trunk_chain_48"] = {"bytes": chain_bytes, "us": round(ms_chain * 1e3, 2),
                             "GBs": round(chain_bytes / (ms_chain * 1e-3) / 1e9, 1)}
    if not quick:
        res["trunk_chain_48"]["fp16_vs_int8"] = chain_fp16_vs_int8(B, chain, chain_bytes, x768, x3072, y, rng)
    # the same kernel on the INT8 tied head (38.6 MB, no bias): large enough that the launch floor
    # no longer hides the streaming rate
    N, K = VOCAB, 768
    w16 = B.dev(f16(rng, (N, K), 0.02))
    q, s = quantize_dev(B, w16, N, K)
    w16.free()
    algo = N * K + 4 * N + 2 * K + 2 * N
    R = copies_for(N * K)
    big = B.empty(R * N * K)
    for r in range(R):
        L.gpt2_d2d(big.at(r * N * K), q.ptr, N * K)
    L.gpt2_sync()
    log(f"gemv chain: {res['trunk_chain_48']}")
    ms_cold, _ = B.run_ops([B.op(3, y.ptr, x768.ptr, big.at(r * N * K), s.ptr, None, 1, N, K) for r in range(R)], 1, n_cold)
    ms_cold /= R
    ms_warm, _ = B.run_ops([B.op(3, y.ptr, x768.ptr, q.ptr, s.ptr, None, 1, N, K)], 2 if quick else 10, n_head)
    res["head"] = {"N": N, "K": K, "bytes": algo, "copies": R,
                   "cold_us": round(ms_cold * 1e3, 3), "cold_GBs": round(algo / (ms_cold * 1e-3) / 1e9, 1),
                   "cold_frac_of_8TBs": round(algo / (ms_cold * 1e-3) / 8e12, 3),
                   "warm_us": round(ms_warm * 1e3, 3), "warm_GBs": round(algo / (ms_warm * 1e-3) / 1e9, 1)}
    big.free()
    # fp16 tied head: [1x768] . [768x50257], 77.3 MB; cold rotates >= 600 MB of copies (8), well past
    # the 256 MB MALL
    N, K = VOCAB, 768
    algo = 2 * N * K + 2 * K + 2 * N
    R = copies_for(2 * N * K)
    big = B.empty(R * N * K * 2)
    head = f16(rng, (N, K), 0.02)
    for r in range(R):
        L.gpt2_h2d(big.at(r * N * K * 2), head.ctypes.data, head.nbytes)
    log(f"gemv int8 head: {res['head']}")
    ms_cold, _ = B.run_ops([B.op(2, y.ptr, x768.ptr, big.at(r * N * K * 2), None, None, 1, N, K) for r in range(R)], 1,
                           2 * n_cold)
    ms_cold /= R
    ms_warm, _ = B.run_ops([B.op(2, y.ptr, x768.ptr, big.ptr, None, None, 1, N, K)], 2 if quick else 10, n_head)
    head_res = {"N": N, "K": K, "bytes": algo, "copies": R, "cold_us": round(ms_cold * 1e3, 2),
                "cold_GBs": round(algo / (ms_cold * 1e-3) / 1e9, 1), "warm_us": round(ms_warm * 1e3, 2),
                "warm_GBs": round(algo / (ms_warm * 1e-3) / 1e9, 1)}
    big.free()
    return res, head_res


def chain_fp16_vs_int8(B, chain8, bytes8, x768, x3072, y, rng, rounds=12, burst=20):
    """The 48 trunk GEMVs of one decode step with fp16 weights against the same chain with INT8 weights
    (the reference's [C] comparison, BENCHMARKS.md:932: 0.9764 against 0.6948 ms), in alternating rounds
    (fp16 first on even rounds); one sample = the mean of `burst` chains; median and [min, max] per side
    and the overlap verdict (bench/ab.py)."""
    ab = importlib.import_module("ab")
    chain16, bytes16 = [], 0
    for layer in range(N_LAYER):
        for name, N, K in TRUNK_GEMV:
            x = x3072 if K == 3072 else x768
            W = B.dev(f16(rng, (N, K), 0.02))
            b = B.dev(f16(rng, N, 0.01))
            chain16.append(B.op(2, y.ptr, x.ptr, W.ptr, None, b.ptr, 1, N, K))
            bytes16 += 2 * N * K + 2 * K + 4 * N
    s16, s8 = [], []
    B.run_ops(chain16, 5, 5)
    for r in range(rounds):
        for side in ((0, 1) if r % 2 == 0 else (1, 0)):
            ms, _ = B.run_ops(chain16 if side == 0 else chain8, 2, burst)
            (s16 if side == 0 else s8).append(ms * 1e3)
    a, b8 = ab.stats(s16), ab.stats(s8)
    v = ab.verdict(a, b8)
    return {"fp16_us": {k: round(v_, 2) for k, v_ in a.items()}, "int8_us": {k: round(v_, 2) for k, v_ in b8.items()},
            "fp16_bytes": bytes16, "int8_bytes": bytes8, "bytes_ratio": round(bytes16 / bytes8, 3),
            "fp16_GBs": round(bytes16 / (a["median"] * 1e-6) / 1e9, 1),
            "int8_GBs": round(bytes8 / (b8["median"] * 1e-6) / 1e9, 1),
            "int8_speedup": v["speedup_b_vs_a"], "verdict": v["verdict"],
            "rounds": rounds, "sample": f"mean of {burst} chains back to back, 48 distinct weights per chain"}


# ------------------------------------------------------------------------------ INT8 GEMM set, head GEMM
def bench_gemm_extra(B, steps):
    """The same P=512 trunk set with INT8 weights (gpt2_matmul_int8, the config-5 prefill path), and
    the tied head as a prefill GEMM: [512x768] . [768x50257]^T (config 4, logits for every row)."""
    rng = np.random.default_rng(4242)
    L = B.L
    X = B.dev(f16(rng, (M_PREFILL, 768), 1.0))
    Xf = B.dev(f16(rng, (M_PREFILL, 3072), 1.0))
    outs = {name: B.empty(M_PREFILL * N * 2) for name, N, K in GEMM_SET}
    ops = []
    for layer in range(N_LAYER):
        for name, N, K in GEMM_SET:
            q = B.dev(rng.integers(-127, 128, (N, K), dtype=np.int8))
            s = B.dev((rng.random(N, dtype=np.float32) * np.float32(2e-4) + np.float32(1e-4)).astype(np.float32))
            b = B.dev(f16(rng, N, 0.01))
            ops.append(B.op(1, outs[name].ptr, (Xf if K == 3072 else X).ptr, q.ptr, s.ptr, b.ptr, M_PREFILL, N, K))
    flops = sum(2.0 * M_PREFILL * N * K for _, N, K in GEMM_SET) * N_LAYER
    ms, _ = B.run_ops(ops, 5, max(20, steps // 2))
    per = []
    for j, (name, N, K) in enumerate(GEMM_SET):
        ms_shape, _ = B.run_ops(ops[j::4], 3, max(20, steps // 4))
        us = ms_shape / N_LAYER * 1e3
        per.append({"gemm": name, "us": round(us, 3), "tflops": round(2.0 * M_PREFILL * N * K / (us * 1e-6) / 1e12, 2)})
    int8 = {"us_per_step": round(ms * 1e3, 2), "tflops": round(flops / (ms * 1e-3) / 1e12, 2), "shapes": per}
    B.keep.clear()
    # head GEMM: fp16 wte [50257, 768], A = 512 LayerNorm-like rows, no bias
    N, K = VOCAB, 768
    A = B.dev(f16(rng, (M_PREFILL, K), 1.0))
    W = B.dev(f16(rng, (N, K), 0.02))
    Cm = B.empty(M_PREFILL * N * 2)
    ms_h, _ = B.run_ops([B.op(0, Cm.ptr, A.ptr, W.ptr, None, None, M_PREFILL, N, K)], 3, 50)
    fl = 2.0 * M_PREFILL * N * K
    achieved = fl / (ms_h * 1e-3) / 1e12
    head = {"M": M_PREFILL, "N": N, "K": K, "gflop": round(fl / 1e9, 3), "us": round(ms_h * 1e3, 2),
            "tflops": round(achieved, 1), "frac_of_peak": round(achieved / PEAK_FP16_TFLOPS, 4),
            "kernel": L.gpt2_tune_gemm_name(L.gpt2_tune_gemm_pick(M_PREFILL, N, K)).decode()}
    B.keep.clear()
    return int8, head


# ------------------------------------------------------------------------------ M sweep
def bench_m_sweep(B, Ms=(1, 16, 32, 64, 128, 256, 512, 1024), iters=30):
    """The four trunk GEMMs across prompt lengths (the reference's bench/profile_matmul.cu:6-16 sweep):
    per shape, 12 layers' distinct weights back to back through gpt2_matmul_tiled / gpt2_matmul_int8,
    per-launch microseconds and TFLOP/s (M = 1 runs the GEMV path and short prompts the skinny GEMM,
    as the launchers route them)."""
    rng = np.random.default_rng(555)
    L = B.L
    out = {}
    for kind in ("fp16", "int8"):
        rows = []
        for name, N, K in GEMM_SET:
            if kind == "int8":
                Ws = [B.dev(rng.integers(-127, 128, (N, K), dtype=np.int8)) for _ in range(N_LAYER)]
                sc = B.dev(np.full(N, 1e-3, np.float32))
            else:
                Ws = [B.dev(f16(rng, (N, K), 0.02)) for _ in range(N_LAYER)]
                sc = None
            b = B.dev(f16(rng, N, 0.01))
            for M in Ms:
                A = B.dev(f16(rng, (M, K), 1.0))
                Cm = B.empty(M * N * 2)
                ops = [B.op(1 if kind == "int8" else 0, Cm.ptr, A.ptr, w.ptr, sc.ptr if sc else None, b.ptr, M, N, K)
                       for w in Ws]
                ms, _ = B.run_ops(ops, 3, iters)
                us = ms * 1e3 / N_LAYER
                cfg = L.gpt2_tune_gemm_pick_q(M, N, K, 1 if kind == "int8" else 0)
                skinny = hasattr(L, "gpt2_tune_gemm_skinny_max") and 2 <= M <= L.gpt2_tune_gemm_skinny_max(kind == "int8")
                rows.append({"gemm": name, "M": M, "us": round(us, 3),
                             "tflops": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 2),
                             "kernel": "gemv" if M == 1 else "skinny" if skinny else L.gpt2_tune_gemm_name(cfg).decode()})
            B.keep.clear()
        out[kind] = rows
    return out


# ------------------------------------------------------------------------------ prefill attention
def bench_attention(B):
    """Causal prefill attention (gpt2_attention_flash) over qkv[T, 2304], 12 heads x 64 dims.  FLOPs
    counted over the causal triangle: 2 (q.k) + 2 (p.v) per (query, key <= query, dim, head)."""
    rng = np.random.default_rng(99)
    res = {}
    for T in (512, 1024):
        qkv = B.dev(f16(rng, (T, 2304), 1.0))
        att = B.empty(T * 768 * 2)
        ms, _ = B.run_ops([B.op(4, att.ptr, qkv.ptr, None, None, None, T, 0, 0)], 20, 500)
        fl = 4.0 * 12 * 64 * T * (T + 1) / 2
        res[f"T{T}"] = {"us": round(ms * 1e3, 3), "gflop": round(fl / 1e9, 4),
                        "tflops": round(fl / (ms * 1e-3) / 1e12, 2)}
    return res


# ------------------------------------------------------------------------------ seeded body
_BODY = None


def seeded_body():
    """The seeded GPT-2-124M body (base seed 1234, N(0,0.02) weights, zero biases, LN 1/0), built once
    and shared by the forward, decode and CPU legs."""
    global _BODY
    if _BODY is None:
        _BODY = importlib.import_module("bare_metal_gpt2_amd.synth").make_body(seed=1234, plain=True)
    return _BODY


# ------------------------------------------------------------------------------ forward (config 1)
def bench_forward_t64(B, reps=20):
    """Config 1 on the GPU: the fp16 forward (flash backend, fp16 weights) at T=64 with logits for
    every row [64 x 50257] (forward_cuda.cu:77-116 with logits_all), host-timed per call around a
    device sync; median, min and max of `reps` calls after 3 untimed ones."""
    pkg, L = B.pkg, B.L
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    model = pkg.Model(seeded_body())
    T = 64
    d_ids = B.dev(synth.token_ids(T, seed=1234))
    logits = B.empty(T * VOCAB * 2)
    scr = pkg.Scratch(T)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all = logits.ptr, 1
    be = pkg.backend("flash")
    ms = []
    for i in range(reps + 3):
        L.gpt2_sync()
        t = time.perf_counter()
        L.gpt2_forward_cuda(be, C.byref(model.gpu), d_ids.ptr, T, C.byref(scr.s), C.byref(caps))
        L.gpt2_sync()
        if i >= 3:
            ms.append((time.perf_counter() - t) * 1e3)
    pkg.check("forward T=64")
    model.free()
    scr.free()
    return {"T": T, "logits_all": True, "backend": "flash (fp16)", "gflop": 15.89,
            "ms_median": round(float(np.median(ms)), 4), "ms_min_max": [round(min(ms), 4), round(max(ms), 4)]}


def bench_prefill(B, reps=30):
    """The whole prefill (gpt2_prefill_fill_cache: embedding, 12 layers with attention and the K/V
    fill, final LayerNorm, last-row logits) at P=512 with fp16 and with INT8 trunk weights, and at
    P=128 with the LayerNorm fold at its default (on there) and off, and at P=16 with the skinny GEMM
    at its default (on there) and off; one hipEvent pair per forward on the library's stream, median
    and [min, max] of `reps` forwards after 3 untimed ones.
    prefill_trunk_gemm_tflops = the 48 trunk GEMMs' 86.97 GFLOP / the fp16 P=512 forward: attention,
    LayerNorms and the head row sit in the denominator, so it is a lower bound on the trunk rate."""
    pkg, L = B.pkg, B.L
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    hip = C.CDLL("libamdhip64.so")
    for fn in ("hipEventCreate", "hipEventRecord", "hipEventElapsedTime", "hipEventDestroy"):
        getattr(hip, fn).restype = C.c_int
    stream = C.c_void_p(L.gpt2_get_stream())

    def run(model, backend, T, lnfold=-1, skinny=-1):
        kv, scr = pkg.KVCache(T), pkg.Scratch(T)
        d_ids = B.dev(synth.token_ids(T, seed=1234))
        logits = B.empty(VOCAB * 2)
        caps = pkg.GPT2CapsGPU()
        caps.logits, caps.logits_all = logits.ptr, 0
        be = pkg.backend(backend)
        L.gpt2_tune_prefill_lnfold(lnfold)
        L.gpt2_tune_gemm_skinny(skinny)
        ev = [(C.c_void_p(), C.c_void_p()) for _ in range(reps)]
        for a, b in ev:
            hip.hipEventCreate(C.byref(a))
            hip.hipEventCreate(C.byref(b))
        try:
            for _ in range(3):
                L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, T, C.byref(scr.s),
                                          C.byref(caps))
            for a, b in ev:
                hip.hipEventRecord(a, stream)
                L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, T, C.byref(scr.s),
                                          C.byref(caps))
                hip.hipEventRecord(b, stream)
            L.gpt2_sync()
            pkg.check(f"prefill {backend} T={T}")
            ms = []
            for a, b in ev:
                t = C.c_float()
                hip.hipEventElapsedTime(C.byref(t), a, b)
                ms.append(t.value)
        finally:
            L.gpt2_tune_prefill_lnfold(-1)
            L.gpt2_tune_gemm_skinny(-1)
            for a, b in ev:
                hip.hipEventDestroy(a)
                hip.hipEventDestroy(b)
            kv.free()
            scr.free()
        return {"ms_median": round(float(np.median(ms)), 4), "ms_min_max": [round(min(ms), 4), round(max(ms), 4)]}

    model = pkg.Model(seeded_body())
    out = {"fp16_p512": run(model, "flash", 512), "fp16_p128": run(model, "flash", 128),
           "fp16_p128_lnfold_off": run(model, "flash", 128, 0), "fp16_p16": run(model, "flash", 16),
           "fp16_p16_skinny_off": run(model, "flash", 16, skinny=0)}
    model.quantize()
    out["int8_p512"] = run(model, "int8", 512)
    out["int8_p128"] = run(model, "int8", 128)
    out["int8_p128_lnfold_off"] = run(model, "int8", 128, 0)
    out["int8_p16"] = run(model, "int8", 16)
    out["int8_p16_skinny_off"] = run(model, "int8", 16, skinny=0)
    model.free()
    trunk_flop = N_LAYER * sum(2.0 * M_PREFILL * N * K for _, N, K in GEMM_SET)
    out["prefill_trunk_gemm_tflops"] = round(trunk_flop / (out["fp16_p512"]["ms_median"] * 1e-3) / 1e12, 2)
    for w in ("fp16", "int8"):
        out[f"{w}_p128_lnfold_speedup"] = round(out[f"{w}_p128_lnfold_off"]["ms_median"] / out[f"{w}_p128"]["ms_median"], 3)
        out[f"{w}_p16_skinny_speedup"] = round(out[f"{w}_p16_skinny_off"]["ms_median"] / out[f"{w}_p16"]["ms_median"], 3)
    return out


def cpu_forward_t64():
    """Config 1 on the CPU: the reference's forward (cpu/forward_cpu.c:118-166 via oracle/_ref, or the
    restatement) at T=64 with logits_all, on the same seeded body and ids as bench_forward_t64.  Warmup
    1, median of 5 on every thread, then one run on one thread (correctness.c:240-250 pattern)."""
    import oracle
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    body, ids = seeded_body(), synth.token_ids(64, seed=1234)
    use_ref = oracle.ref_available()
    off = oracle.oracle_offsets() if use_ref else None

    def run():
        t = time.perf_counter()
        if use_ref:
            oracle.ref_forward(body, off, ids, logits_all=True)
        else:
            oracle.forward(body, ids, logits_all=True)
        return (time.perf_counter() - t) * 1e3

    threads = int(os.environ.get("OMP_NUM_THREADS", "1"))
    run()
    ms = [run() for _ in range(5)]
    one = None
    try:
        gomp = C.CDLL("libgomp.so.1")
        gomp.omp_set_num_threads(1)
        one = round(run(), 1)
        gomp.omp_set_num_threads(threads)
    except OSError:
        pass
    return {"T": 64, "logits_all": True, "kind": "reference" if use_ref else "port", "cores": threads,
            "ms_median": round(float(np.median(ms)), 1), "ms_min_max": [round(min(ms), 1), round(max(ms), 1)],
            "ms_one_thread": one, "gflop": 15.89, "cpu": cpu_model()}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


# ------------------------------------------------------------------------------ decode (config 5)
def bench_decode(B, steady_reps=64, greedy=True, cold_copies=4, cold_reps=48):
    """Config 5 decode: the P=512 prefill, then the step at pos 512 (multi-kernel graph, persistent
    step, eager), the 511-step greedy run, and the persistent step with its weights cold (see
    decode_cold)."""
    pkg, L = B.pkg, B.L
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    t0 = time.time()
    model = pkg.Model(seeded_body())
    model.quantize()                       # 48 trunk tensors INT8, head fp16
    kv = pkg.KVCache(1024)
    scr = pkg.Scratch(1024)
    P = 512
    ids = synth.token_ids(P, seed=1234)
    d_ids = B.dev(ids)
    logits = B.empty(VOCAB * 2)
    tokens = B.empty(1024 * 4)
    be = pkg.backend("int8")
    caps = pkg.GPT2CapsGPU()
    caps.logits = logits.ptr
    caps.logits_all = 0
    # the P=512 prefill itself (INT8 trunk GEMMs, attention, head row, K/V fill), host-timed per call
    pre = []
    for i in range(6):
        L.gpt2_sync()
        t = time.perf_counter()
        L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, P, C.byref(scr.s), C.byref(caps))
        L.gpt2_sync()
        if i >= 1:
            pre.append((time.perf_counter() - t) * 1e3)
    pkg.check("prefill")
    first = int(np.argmax(pkg.half_bits_to_f32(logits.numpy(np.uint16, (VOCAB,)))))
    ms = C.c_float()

    def steady(mode):
        """Median ms per replay at pos 512 (cache length 512), each replay re-pinned to pos 512."""
        g = L.gpt2_decode_graph_create_mode(be, C.byref(model.gpu), C.byref(kv.kv), C.byref(scr.s), logits.ptr,
                                            tokens.ptr, mode)
        if not g:
            pkg.check("graph create")
            raise RuntimeError("graph create failed")
        got_mode = L.gpt2_decode_graph_mode(g)
        samples = []
        for i in range(steady_reps + 5):
            L.gpt2_decode_graph_set(g, first, P)
            L.gpt2_decode_graph_time(g, 1, C.byref(ms))
            if i >= 5:
                samples.append(ms.value)
        tok, pos = C.c_int(), C.c_int()
        if L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)):
            pkg.check("steady decode")
        pkg.check("steady decode")
        return g, got_mode, samples

    # multi-kernel captured step (reference point), then the persistent step (the default)
    g_multi, _, samples_multi = steady(pkg.DECODE_MULTI)
    L.gpt2_decode_graph_destroy(g_multi)
    g, mode, samples = steady(pkg.DECODE_AUTO)
    # eager (non-graph) step at the same position, for the launch-overhead comparison
    eager = []
    for i in range(12):
        kv.kv.len = P
        L.gpt2_sync()
        t = time.perf_counter()
        L.gpt2_decode_step_cuda(be, C.byref(model.gpu), C.byref(kv.kv), first, P, C.byref(scr.s), logits.ptr, None)
        L.gpt2_sync()
        if i >= 2:
            eager.append((time.perf_counter() - t) * 1e3)
    pkg.check("eager decode")
    # the full greedy run: 511 steps from pos 512 (ctx 512 -> 1023)
    tok, pos = C.c_int(), C.c_int()
    greedy_ms = None
    if greedy:
        kv.kv.len = P
        L.gpt2_decode_graph_set(g, first, P)
        L.gpt2_decode_graph_time(g, 511, C.byref(ms))
        if L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)):
            pkg.check("greedy run")
        pkg.check("greedy run")
        greedy_ms = ms.value
    L.gpt2_decode_graph_destroy(g)
    streamed = model.q.streamed_bytes
    kv_bytes = L.gpt2_kv_step_bytes(C.byref(kv.kv), P + 1)
    med = float(np.median(samples))
    med_multi = float(np.median(samples_multi))
    res = {"prefill_ms_at_512": round(float(np.median(pre)), 4),
           "step": "persistent (one kernel per token)" if mode == pkg.DECODE_PERSISTENT else "multi-kernel graph",
           "tok_s_at_512": round(1000.0 / med, 1), "ms_step_at_512": round(med, 4),
           "ms_step_min_max": [round(min(samples), 4), round(max(samples), 4)],
           "multi_kernel_graph_tok_s_at_512": round(1000.0 / med_multi, 1),
           "eager_ms_step_at_512": round(float(np.median(eager)), 4),
           "greedy_511_tok_s": round(1000.0 / greedy_ms, 1) if greedy_ms else None,
           "greedy_final_pos": pos.value if greedy_ms else None,
           "weight_bytes": int(streamed), "kv_bytes_at_513": int(kv_bytes),
           "step_GBs_at_512": round((streamed + kv_bytes) / (med * 1e-3) / 1e9, 1),
           "setup_s": round(time.time() - t0, 1)}
    kv.free()
    model.free()
    if cold_copies:
        res["cold"] = decode_cold(B, scr, first, logits, tokens, streamed, kv_bytes, med, cold_copies, cold_reps)
    scr.free()
    return res


def decode_cold(B, scr, first, logits, tokens, streamed, kv_bytes, warm_ms, copies, reps, backend="int8"):
    """The default (persistent) step with its weights cold: `copies` uploads of the same model, each
    with its own K/V cache (the P=512 prefill) and graph, stepped round robin at pos 512, so the weights
    a step reads (162 MB INT8 trunk + fp16 head, 247 MB all fp16) were last read copies-1 steps earlier,
    past the 256 MB MALL.  backend "int8" quantizes the trunk, "gemv" keeps every weight fp16.  With
    first / streamed / kv_bytes / warm_ms left 0 / None, the step's own prefill token and byte counts
    are used and no cold/warm ratio is given."""
    pkg, L = B.pkg, B.L
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    P = 512
    ids = synth.token_ids(P, seed=1234)
    d_ids = B.dev(ids)
    be = pkg.backend(backend)
    caps = pkg.GPT2CapsGPU()
    caps.logits = logits.ptr
    caps.logits_all = 0
    models, kvs, graphs = [], [], []
    ms = C.c_float()
    try:
        for _ in range(copies):
            m = pkg.Model(seeded_body())
            if backend == "int8":
                m.quantize()
            kv = pkg.KVCache(1024)
            models.append(m)
            kvs.append(kv)
            L.gpt2_prefill_fill_cache(be, C.byref(m.gpu), C.byref(kv.kv), d_ids.ptr, P, C.byref(scr.s), C.byref(caps))
            g = L.gpt2_decode_graph_create_mode(be, C.byref(m.gpu), C.byref(kv.kv), C.byref(scr.s), logits.ptr,
                                                tokens.ptr, pkg.DECODE_AUTO)
            if not g:
                pkg.check("cold graph create")
                raise RuntimeError("graph create failed")
            graphs.append(g)
        L.gpt2_sync()
        pkg.check("cold setup")
        if not first:
            first = int(np.argmax(pkg.half_bits_to_f32(logits.numpy(np.uint16, (VOCAB,)))))
        if streamed is None:
            streamed = models[0].q.streamed_bytes if backend == "int8" else FP16_STEP_WEIGHT_BYTES
        if not kv_bytes:
            kv_bytes = L.gpt2_kv_step_bytes(C.byref(kvs[0].kv), P + 1)
        samples = []
        for i in range(reps + copies):
            g = graphs[i % copies]
            L.gpt2_decode_graph_set(g, first, P)
            L.gpt2_decode_graph_time(g, 1, C.byref(ms))
            if i >= copies:
                samples.append(ms.value)
        tok, pos = C.c_int(), C.c_int()
        for g in graphs:
            if L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)):
                pkg.check("cold decode")
        pkg.check("cold decode")
        med = float(np.median(samples))
        res = {"backend": backend, "copies": copies, "rotated_weight_MB": round(copies * streamed / 1e6, 1),
               "ms_step_at_512": round(med, 4), "ms_step_min_max": [round(min(samples), 4), round(max(samples), 4)],
               "tok_s_at_512": round(1000.0 / med, 1), "weight_bytes": int(streamed),
               "step_GBs_at_512": round((streamed + kv_bytes) / (med * 1e-3) / 1e9, 1)}
        if warm_ms:
            res["cold_over_warm"] = round(med / warm_ms, 3)
        return res
    finally:
        for g in graphs:
            L.gpt2_decode_graph_destroy(g)
        for kv in kvs:
            kv.free()
        for m in models:
            m.free()


FP16_STEP_WEIGHT_BYTES = 2 * 12 * (2304 * 768 + 768 * 768 + 3072 * 768 + 768 * 3072) + 2 * VOCAB * 768


def bench_decode_compare(B, rounds=24, ctxs=(128, 512, 1023), cold_copies=4, cold_reps=32):
    """fp16 against INT8 trunk weights in the decode step (the reference's central decode comparison,
    BENCHMARKS.md:914-917): GPT-2-124M with fp16 trunk GEMVs (gemv backend) and with INT8 trunk GEMVs
    (int8 backend), both with the fp16 head and the default (persistent) graph step; one P=1023 prefill
    each, then single steps re-pinned at ctx 128, 512 and 1023 in alternating rounds (fp16 first on
    even rounds).  Per (side, ctx): median and [min, max] of the single-step times; the INT8 speedup
    and the overlap verdict.  Then both at ctx 512 with their weights cold (decode_cold)."""
    pkg, L = B.pkg, B.L
    ab = importlib.import_module("ab")
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    P = 1023
    ids = synth.token_ids(P, seed=1234)
    d_ids = B.dev(ids)
    sides, out = {}, {}
    ms = C.c_float()
    try:
        for name, backend in (("fp16", "gemv"), ("int8", "int8")):
            model = pkg.Model(seeded_body())
            if backend == "int8":
                model.quantize()
            kv, scr = pkg.KVCache(1024), pkg.Scratch(1024)
            logits, tokens = B.empty(VOCAB * 2), B.empty(1024 * 4)
            caps = pkg.GPT2CapsGPU()
            caps.logits, caps.logits_all = logits.ptr, 0
            be = pkg.backend(backend)
            sides[name] = {"model": model, "kv": kv, "scr": scr, "g": None}
            L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, P, C.byref(scr.s), C.byref(caps))
            L.gpt2_sync()
            pkg.check("prefill")
            first = int(np.argmax(pkg.half_bits_to_f32(logits.numpy(np.uint16, (VOCAB,)))))
            g = L.gpt2_decode_graph_create_mode(be, C.byref(model.gpu), C.byref(kv.kv), C.byref(scr.s), logits.ptr,
                                                tokens.ptr, pkg.DECODE_AUTO)
            if not g:
                pkg.check("graph create")
                raise RuntimeError("graph create failed")
            sides[name].update(g=g, first=first, mode=L.gpt2_decode_graph_mode(g),
                               weight_bytes=model.q.streamed_bytes if backend == "int8" else FP16_STEP_WEIGHT_BYTES)
        samples = {(n, c): [] for n in sides for c in ctxs}
        for r in range(rounds + 2):
            for c in ctxs:
                for n in (("fp16", "int8") if r % 2 == 0 else ("int8", "fp16")):
                    sd = sides[n]
                    L.gpt2_decode_graph_set(sd["g"], sd["first"], c)
                    L.gpt2_decode_graph_time(sd["g"], 1, C.byref(ms))
                    if r >= 2:
                        samples[(n, c)].append(ms.value * 1e3)
        tok, pos = C.c_int(), C.c_int()
        for n, sd in sides.items():
            if L.gpt2_decode_graph_sync(sd["g"], C.byref(tok), C.byref(pos)):
                pkg.check(f"decode {n}")
                raise RuntimeError("decode step failed")
        for c in ctxs:
            a, b = ab.stats(samples[("fp16", c)]), ab.stats(samples[("int8", c)])
            v = ab.verdict(a, b)
            kvb = L.gpt2_kv_step_bytes(C.byref(sides["int8"]["kv"].kv), c + 1)
            row = {}
            for n, st in (("fp16", a), ("int8", b)):
                wb = sides[n]["weight_bytes"]
                row[n] = {"us_median": round(st["median"], 2), "us_min_max": [round(st["min"], 2), round(st["max"], 2)],
                          "tok_s": round(1e6 / st["median"], 1), "weight_bytes": wb,
                          "step_GBs": round((wb + kvb) / (st["median"] * 1e-6) / 1e9, 1)}
            row.update(int8_speedup=v["speedup_b_vs_a"], verdict=v["verdict"], kv_bytes=int(kvb))
            out[f"ctx{c}"] = row
        out["steps"] = {n: ("persistent (one kernel per token)" if sd["mode"] == pkg.DECODE_PERSISTENT
                            else "multi-kernel graph") for n, sd in sides.items()}
        out["rounds"] = rounds
    finally:
        for sd in sides.values():
            if sd["g"]:
                L.gpt2_decode_graph_destroy(sd["g"])
            sd["kv"].free()
            sd["scr"].free()
            sd["model"].free()
    if cold_copies:
        scr = pkg.Scratch(1024)
        logits, tokens = B.empty(VOCAB * 2), B.empty(1024 * 4)
        try:
            cold = {}
            for n, backend in (("fp16", "gemv"), ("int8", "int8")):
                cold[n] = decode_cold(B, scr, 0, logits, tokens, None, 0, None, cold_copies, cold_reps, backend=backend)
            cold["int8_speedup"] = round(cold["fp16"]["ms_step_at_512"] / cold["int8"]["ms_step_at_512"], 3)
            out["cold_ctx512"] = cold
        finally:
            scr.free()
    return out


# ------------------------------------------------------------------------------ persistent prefill trace
def prefill_trace(B, T=512, backend="int8"):
    """The persistent prefill (csrc/prefill.hip, opt-in) beside the launch sequence at one T, and its
    per-task trace (gpt2_tune_prefill_trace): for each task type the mean time waiting for inputs,
    before the k-loop (the LayerNorm panel), in the k-loop (attention: the whole block), in the
    epilogue, draining the stores and bumping the counter; the gap between a work-group's tasks."""
    pkg, L = B.pkg, B.L
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    model = pkg.Model(seeded_body())
    if backend == "int8":
        model.quantize()
    ids = synth.token_ids(T, seed=1)
    d_ids = B.dev(np.asarray(ids, np.int32))
    scr, kv = pkg.Scratch(T), pkg.KVCache(T)
    logits = B.empty(VOCAB * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all = logits.ptr, 0
    ntask = L.gpt2_tune_prefill_trace(None, 0, T)
    buf = B.empty(ntask * 64)
    be = pkg.backend(backend)

    def run(persistent, trace=False):
        L.gpt2_tune_prefill_persistent(1 if persistent else 0)
        L.gpt2_tune_prefill_trace(buf.ptr if trace else None, ntask, T)
        L.gpt2_sync()
        t = time.perf_counter()
        L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, T, C.byref(scr.s), C.byref(caps))
        L.gpt2_sync()
        pkg.check("prefill")
        return (time.perf_counter() - t) * 1e3

    try:
        for _ in range(3):
            run(True)
            run(False)
        pers = float(np.median([run(True) for _ in range(7)]))
        seq = float(np.median([run(False) for _ in range(7)]))
        run(True, trace=True)
    finally:
        L.gpt2_tune_prefill_trace(None, 0, T)
        L.gpt2_tune_prefill_persistent(-1)
    tr = buf.numpy(np.uint64, (ntask, 8)).astype(np.int64)
    nrb, nqb = (T + 31) // 32, (T + 15) // 16
    types = [0] * nrb
    for _ in range(12):
        types += [1] * (nrb * 36) + [2] * (nqb * 12) + [3] * (nrb * 12) + [4] * (nrb * 48) + [5] * (nrb * 24)
    types = np.array(types)
    ready = np.where(tr[:, 2] > 0, tr[:, 2], tr[:, 1])
    kst = np.where(tr[:, 3] > 0, tr[:, 3], ready)
    ken = np.where(tr[:, 4] > 0, tr[:, 4], tr[:, 5])
    us = lambda x: x / 100.0   # s_memrealtime ticks at 100 MHz
    phases = {"wait": us(ready - tr[:, 1]), "pre": us(kst - ready), "kloop": us(ken - kst),
              "epilogue": us(tr[:, 5] - ken), "drain": us(tr[:, 6] - tr[:, 5]), "signal": us(tr[:, 7] - tr[:, 6])}
    per = {}
    for k, name in enumerate(["embed", "qkv", "attention", "attn_proj", "fc", "mlp_proj"]):
        m = types == k
        per[name] = {"tasks": int(m.sum()), **{p: round(float(v[m].mean()), 2) for p, v in phases.items()}}
    gaps = []
    for wg in np.unique(tr[:, 0]):
        r = tr[tr[:, 0] == wg]
        r = r[np.argsort(r[:, 1])]
        gaps += list(us(r[1:, 1] - r[:-1, 7]))
    span = us(tr[:, 7].max() - tr[:, 1].min())
    scr.free()
    kv.free()
    model.free()
    return {"T": T, "backend": backend, "tasks": ntask, "work_groups": int(len(np.unique(tr[:, 0]))),
            "persistent_ms": round(pers, 4), "launch_sequence_ms": round(seq, 4), "traced_span_us": round(float(span), 1),
            "gap_between_tasks_us": round(float(np.mean(gaps)), 2), "per_task_us": per}


# ------------------------------------------------------------------------------ measured ceilings
def measured_peaks(B, cus):
    """This box's ceilings, measured in the same run beside the datasheet peaks (the role of
    bench/microbench.cu:69-377 in the reference): the HBM read stream over 4 GiB (16x the 256 MB
    MALL, so every byte comes from HBM; the faster of two launch shapes) and the fp16 MFMA issue loop
    (v_mfma_f32_32x32x16_f16, four independent accumulators per wave, one work-group of four waves
    per CU)."""
    L = B.L
    nbytes = 4 << 30
    buf = B.pkg.Dev(nbytes)
    L.gpt2_memset(buf.ptr, 1, nbytes)
    ms = C.c_float()
    if B.H.gpt2_bench_read(buf.ptr, nbytes, 5, C.byref(ms)):
        B.pkg.check("gpt2_bench_read")
    read_gbs = nbytes / (ms.value * 1e-3) / 1e9
    buf.free()
    blocks, iters = cus, 20000
    if B.H.gpt2_bench_mfma(blocks, iters, C.byref(ms)):
        B.pkg.check("gpt2_bench_mfma")
    mfma_tflops = blocks * 4.0 * iters * 4 * (32 * 32 * 16 * 2) / (ms.value * 1e-3) / 1e12
    return {"hbm_read_GBs": round(read_gbs, 1), "hbm_read_bytes": nbytes,
            "mfma_fp16_tflops": round(mfma_tflops, 1), "mfma_loop": f"{blocks} work-groups x 4 waves x {iters} x 4 "
            "v_mfma_f32_32x32x16_f16 (one wave per SIMD; the clock drops to ~1.7 GHz under this load)",
            "datasheet": {"hbm_GBs": PEAK_HBM_GBS, "mfma_fp16_tflops": PEAK_FP16_TFLOPS}}


def guard_legs(out, read_gbs):
    """The reference's bug line (bench/correctness_cuda.cu:261-270): a bandwidth figure above the
    achieved read stream cannot be HBM.  Every leg this line calls cold (HBM) is checked against the
    measured read stream and listed under "suspicious" when it exceeds it; the warm legs (weights held
    in the 256 MB MALL) are listed with their ratio, labelled as MALL-resident, never as HBM."""
    cold, warm = [], []
    g = out.get("gemv_int8", {})
    for name, r in g.items():
        if "cold_GBs" in r:
            cold.append((f"gemv_int8.{name}.cold_GBs", r["cold_GBs"]))
        if "warm_GBs" in r:
            warm.append((f"gemv_int8.{name}.warm_GBs", r["warm_GBs"]))
    if "trunk_chain_48" in g:
        warm.append(("gemv_int8.trunk_chain_48.GBs", g["trunk_chain_48"]["GBs"]))
    h = out.get("head_gemv_fp16")
    if h:
        cold.append(("head_gemv_fp16.cold_GBs", h["cold_GBs"]))
        warm.append(("head_gemv_fp16.warm_GBs", h["warm_GBs"]))
    d = out.get("decode")
    if d:
        warm.append(("decode.step_GBs_at_512", d["step_GBs_at_512"]))
        if d.get("cold"):
            cold.append(("decode.cold.step_GBs_at_512", d["cold"]["step_GBs_at_512"]))
    sus = [{"leg": k, "GBs": v, "over_read_stream": round(v / read_gbs, 3)} for k, v in cold if v > read_gbs]
    return {"read_stream_GBs": read_gbs, "suspicious": sus,
            "cold_frac_of_read_stream": {k: round(v / read_gbs, 3) for k, v in cold},
            "warm_mall_frac_of_read_stream": {k: round(v / read_gbs, 3) for k, v in warm}}


# ------------------------------------------------------------------------------ CPU baseline
def host_cpu():
    """nproc, the CPUs this process may run on, and the CPU model name (lscpu, else /proc/cpuinfo)."""
    model = None
    try:
        import subprocess
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, ValueError, Exception):
        pass
    return {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)), "model": model or cpu_model()}


def omp_set_threads(n):
    try:
        C.CDLL("libgomp.so.1").omp_set_num_threads(int(n))
        return True
    except OSError:
        return False


def cpu_baseline(budget_s=12.0, one_thread_s=6.0):
    """The reference's CPU matmul on the four GEMM shapes at M=512 (`value`: on OMP_NUM_THREADS
    threads, the CPU share this GPU's box gives one process), then a shorter sample on one thread."""
    import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", "1"))
    rng = np.random.default_rng(99)
    use_ref = oracle.ref_available()
    mm = oracle.ref_matmul if use_ref else oracle.matmul
    X = rng.standard_normal((M_PREFILL, 768), dtype=np.float32)
    Xf = rng.standard_normal((M_PREFILL, 3072), dtype=np.float32)
    Ws = [(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02), rng.standard_normal(N, dtype=np.float32))
          for _, N, K in GEMM_SET]
    flops = 0.0
    t0 = time.perf_counter()
    sets = 0
    while True:
        for (name, N, K), (W, b) in zip(GEMM_SET, Ws):
            mm(Xf if K == 3072 else X, W, b)
            flops += 2.0 * M_PREFILL * N * K
        sets += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    # one thread: GEMMs of the same set, one after another, while the shorter budget lasts
    one = None
    if omp_set_threads(1):
        fl1, n1, t1 = 0.0, 0, time.perf_counter()
        while True:
            name, N, K = GEMM_SET[n1 % len(GEMM_SET)]
            W, b = Ws[n1 % len(GEMM_SET)]
            mm(Xf if K == 3072 else X, W, b)
            fl1 += 2.0 * M_PREFILL * N * K
            n1 += 1
            if time.perf_counter() - t1 > one_thread_s:
                break
        d1 = time.perf_counter() - t1
        omp_set_threads(threads)
        one = {"value": round(fl1 / d1 / 1e12, 6), "cores": 1,
               "sample": f"{n1} GEMMs of the set in order, {fl1 / 1e9:.2f} GFLOP, {d1:.1f} s"}
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "reference" if use_ref else "port",
            "sample": f"{sets} x the 4-GEMM set at M=512 (one layer of the workload, {flops / sets / 1e9:.3f} GFLOP"
                      f" per set), fp32 storage / double accumulation, {dt:.1f} s",
            "one_thread": one, "host": host_cpu(),
            "threads_note": "cores = OMP_NUM_THREADS, the CPU share of one GPU on this pool's boxes (16); nproc "
                            "counts the whole host"}


def cpu_decode_baseline(budget_s=8.0):
    """Decode tok/s @ctx=512 of the reference's CPU path (cpu/forward_cpu.c): it has no KV cache, so a
    token is a full forward over 513 positions with last-row logits (bench/correctness.c:252-263,
    92 GFLOP), on the same seeded body as the decode leg, fp32.  At least one token, more while the
    budget lasts."""
    import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", "1"))
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    body = seeded_body()
    ids = synth.token_ids(513, seed=1234)
    use_ref = oracle.ref_available()
    off = oracle.oracle_offsets() if use_ref else None
    n, t0 = 0, time.perf_counter()
    while True:
        if use_ref:
            oracle.ref_forward(body, off, ids, logits_all=False)
        else:
            oracle.forward(body, ids, logits_all=False)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 4), "unit": "tok/s", "cores": threads, "kind": "reference" if use_ref else "port",
            "sample": f"{n} token(s) at ctx=512, each a full fp32 forward over 513 positions (no KV cache on the "
                      f"reference CPU path), {dt:.1f} s"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-clock", action="store_true",
                    help="skip the amd-smi clock sampler; use it under rocprofv3, whose preload would make the "
                         "amd-smi child initialise the GPU before its launcher execs python")
    ap.add_argument("--no-extras", action="store_true", help="only the headline GEMM set")
    ap.add_argument("--no-decode", action="store_true", help="skip the graph-replayed decode leg")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the decode GEMV legs (INT8 trunk cold/warm, the 48-GEMV chain, INT8 and fp16 head) "
                         "with a few launches each, printed as one JSON line: the driver for their rocprofv3 "
                         "counter runs")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the config-5 decode leg (prefill, step at pos 512 warm and with its weights cold; "
                         "no greedy run), printed as one JSON line: the driver for the decode step's counter runs")
    ap.add_argument("--prefill-trace", type=int, default=0, metavar="T",
                    help="only the persistent prefill at T tokens (INT8 and fp16) beside the launch sequence, "
                         "with its per-task trace, printed as one JSON line")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the headline GEMM set (no peaks, extras or CPU legs): the driver of the "
                         "committed rocprofv3 trace that the roofline's kernel time is read from")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="also run one plain copy of BYTES (calibrates FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the matmul path "
              "would shard by output rows (each GPU a slice of N), but no multi-GPU run is part of it.", file=sys.stderr)
        sys.exit(2)
    # The GPU boxes give one GPU's process a 16-thread CPU share and export OMP_NUM_THREADS=16; where
    # it is not set, use every CPU this process may run on.
    os.environ.setdefault("OMP_NUM_THREADS", str(max(1, len(os.sched_getaffinity(0)))))

    import __graft_entry__
    pkg = __graft_entry__.load_package()
    L = pkg.lib()
    B = Bench(pkg)
    cus, clk = C.c_int(), C.c_int()
    name = C.create_string_buffer(256)
    if B.H.gpt2_device_info(C.byref(cus), C.byref(clk), name, 256):
        raise SystemExit("no HIP device visible")
    log(f"device {name.value.decode()} CUs={cus.value} clock={clk.value / 1e3:.0f} MHz")

    if args.copy_probe:
        src, dst = pkg.Dev(args.copy_probe), pkg.Dev(args.copy_probe)
        L.gpt2_memset(src.ptr, 1, args.copy_probe)
        ms = C.c_float()
        B.H.gpt2_bench_copy(dst.ptr, src.ptr, args.copy_probe, C.byref(ms))
        log(f"copy probe: {args.copy_probe} B in {ms.value * 1e3:.1f} us")
        src.free()
        dst.free()
    if args.gemv_only:
        gemv, head = bench_gemv(B, quick=True)
        print(json.dumps({"gemv_int8": gemv, "head_gemv_fp16": head}), flush=True)
        return
    if args.prefill_trace:
        print(json.dumps({"prefill_trace": [prefill_trace(B, args.prefill_trace, be) for be in ("int8", "flash")]}),
              flush=True)
        return
    if args.decode_only:
        print(json.dumps({"decode": bench_decode(B, steady_reps=32, greedy=False)}), flush=True)
        return
    flops_step, ms_step, shapes, roofline, ms_graph, step_stats, clock = bench_gemm_set(B, args.steps, args.warmup, not args.no_clock)
    value = flops_step / (ms_step * 1e-3) / 1e12
    log(f"prefill GEMM set: {ms_step * 1e3:.1f} us/step -> {value:.1f} TFLOP/s; steps {step_stats}; clock {clock}")
    log(f"per shape {shapes}")
    out = {"metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
           "config": {"workload": "prefill trunk GEMM set @P=512: 12 layers x {QKV 512x2304x768, attn-proj "
                                  "512x768x768, fc 512x3072x768, mlp-proj 512x768x3072} + bias, fp16 in, fp32 acc, "
                                  "fp16 out (BASELINE config 2, per layer)",
                      "M": M_PREFILL, "layers": N_LAYER, "gflop_per_step": round(flops_step / 1e9, 4),
                      "device": name.value.decode()},
           "step_stats": step_stats, "clock": clock, "launch_floor_us": launch_floor_us(B),
           "roofline": roofline, "gemm_shapes": shapes,
           "gemm_set_graph_replay": {"us_per_step": round(ms_graph * 1e3, 2),
                                     "tflops": round(flops_step / (ms_graph * 1e-3) / 1e12, 2)}}
    B.keep.clear()
    if args.headline_only:
        print(json.dumps(out), flush=True)
        return
    peaks = measured_peaks(B, cus.value)
    out["measured_peaks"] = peaks
    roofline["peak_measured"] = peaks["mfma_fp16_tflops"]
    roofline["frac_of_measured"] = round(roofline["achieved"] / peaks["mfma_fp16_tflops"], 4)
    log(f"measured peaks: {peaks}")
    if not args.no_extras:
        gemv, head = bench_gemv(B)
        B.keep.clear()
        log(f"gemv: {gemv}\nhead: {head}")
        out["gemv_int8"] = gemv
        out["head_gemv_fp16"] = head
        out["gemm_int8_set"], out["head_gemm_fp16"] = bench_gemm_extra(B, args.steps)
        log(f"int8 gemm set: {out['gemm_int8_set']}\nhead gemm: {out['head_gemm_fp16']}")
        out["gemm_m_sweep"] = bench_m_sweep(B)
        B.keep.clear()
        log(f"m sweep: {out['gemm_m_sweep']}")
        out["attention_prefill"] = bench_attention(B)
        B.keep.clear()
        log(f"attention: {out['attention_prefill']}")
        out["forward_t64"] = bench_forward_t64(B)
        B.keep.clear()
        log(f"forward T=64: {out['forward_t64']}")
        out["prefill"] = bench_prefill(B)
        B.keep.clear()
        log(f"prefill: {out['prefill']}")
        if not args.no_decode:
            out["decode"] = bench_decode(B)
            B.keep.clear()
            log(f"decode: {out['decode']}")
            out["decode_fp16_vs_int8"] = bench_decode_compare(B)
            B.keep.clear()
            log(f"decode fp16 vs int8: {out['decode_fp16_vs_int8']}")
    out["bandwidth_guard"] = guard_legs(out, peaks["hbm_read_GBs"])
    if out["bandwidth_guard"]["suspicious"]:
        log(f"SUSPICIOUS (above the measured read stream): {out['bandwidth_guard']['suspicious']}")
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
        log(f"cpu: {out['cpu_baseline']}")
        if not args.no_extras:
            out["cpu_forward_t64"] = cpu_forward_t64()
            log(f"cpu forward T=64: {out['cpu_forward_t64']}")
        if not args.no_extras and not args.no_decode:
            out["cpu_decode_baseline"] = cpu_decode_baseline()
            log(f"cpu decode: {out['cpu_decode_baseline']}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
