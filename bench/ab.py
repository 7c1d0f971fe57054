#!/usr/bin/env python
"""Interleaved A/B timing with a noise verdict (the reference's bench/ab_forward.cu:61-73 pattern).

Two variants of one workload are timed in alternating rounds (A B, B A, A B, ...), so drift of the
box (clock, temperature, other tenants) lands on both sides alike.  Each round yields one sample per
side; the report gives every side's median and [min, max] over the rounds, the ratio of the medians,
and the verdict: when the two [min, max] ranges overlap the difference is NOT above noise.

    python bench/ab.py WORKLOAD --a SPEC --b SPEC [--rounds 15] [--json]

WORKLOAD (one sample = the mean over a short burst, microseconds):
  gemm_set       the headline step: 12 layers x {QKV, attn-proj, fc, mlp-proj} fp16 GEMMs at M=512
  gemm_int8_set  the same set with INT8 weights
  gemm_shape     one trunk shape, 12 layers of distinct weights back to back (knob shape=qkv|...)
  head_gemm      the tied head as a GEMM, [512x768] . [768x50257]^T
  gemv_chain     the 48 trunk GEMVs of one decode step, distinct weights (knob dtype=int8|fp16)
  gemv           one GEMV per launch, us per launch (knobs shape (a trunk shape or head), dtype,
                 cold=1|0, gemv_cfg)
  decode_step    one persistent (or multi-kernel) decode step of GPT-2-124M, re-pinned at a position
  prefill        gpt2_prefill_fill_cache at T tokens, host-timed around a device sync
  empty          an empty kernel back to back (the launch floor)

SPEC: comma-separated key=value knobs; an empty SPEC ("") is the library's default.
  lib=DIR        a build of the library in DIR (libgpt2amd.so + libgpt2bench.so, see ab_build.sh);
                 a side with lib= runs in worker subprocesses, alternated with the other side's
  gemm_cfg=C     force GEMM tile config C for every call (gpt2_tune_gemm_force; -1 = the picks)
  prefill_persistent=0|1, lnfold=0|1 (the prefill's LayerNorm fold), backend=int8|gemv|flash, pos=P, T=T, mode=persistent|multi,
  gemv_cfg=C     force GEMV config C (gemv workload; -1 = the library's pick),
  dtype=int8|fp16, shape=qkv|attn_proj|fc|mlp_proj, cold=1|0, big_alloc=GiB (allocate, touch and free that
  much device memory before the workload's own buffers, as bench.py's measured peaks leg does)
  epi=gelu|resid  gemm_shape / gemm_set: the fused-epilogue GEMM the prefill runs (gelu after the
                 product, or the residual added in place) instead of the plain one
  m=M            gemm_shape / gemm_set: rows of A (default 512)
  skinny=N       the skinny GEMM takes M up to N (gpt2_tune_gemm_skinny; 0: never, -1: the default)
  holds=A/X/H    decode_step: the persistent step's poll hold-offs in 10 ns ticks (attention words, x,
                 gelu(fc); -1 keeps a default; gpt2_tune_decode_holds)

Examples:
  python bench/ab.py gemm_set --a "" --b gemm_cfg=12
  python bench/ab.py decode_step --a "backend=gemv" --b "backend=int8"
  bash bench/ab_build.sh 650516e /tmp/ab_r1 && python bench/ab.py gemv_chain --a lib=/tmp/ab_r1 --b ""
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib
import json
import os
import subprocess
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SHAPES = {"qkv": (2304, 768), "attn_proj": (768, 768), "fc": (3072, 768), "mlp_proj": (768, 3072)}
ORDER = ["qkv", "attn_proj", "fc", "mlp_proj"]


# ------------------------------------------------------------------------------ statistics
def stats(samples):
    v = sorted(float(x) for x in samples)
    return {"median": float(np.median(v)), "min": v[0], "max": v[-1], "n": len(v)}


def verdict(a, b):
    """a, b: stats() of the two sides (times: lower is better).  Ratio > 1 means B is faster."""
    ratio = a["median"] / b["median"]
    overlap = not (b["max"] < a["min"] or a["max"] < b["min"])
    if overlap:
        text = "[min,max] OVERLAP -> NOT above noise"
    else:
        text = "disjoint ranges -> above noise (" + ("B faster" if ratio > 1.0 else "B SLOWER") + ")"
    return {"speedup_b_vs_a": round(ratio, 4), "overlap": overlap, "verdict": text}


def parse_spec(spec):
    out = {}
    for item in filter(None, (s.strip() for s in spec.split(","))):
        k, _, v = item.partition("=")
        out[k] = v
    return out


# ------------------------------------------------------------------------------ workloads
class Env:
    """The product library and the timing harness, loaded from the tree or from a variant build."""

    def __init__(self, libdir=None):
        sys.path.insert(0, ROOT)
        sys.path.insert(0, HERE)
        import __graft_entry__
        self.pkg = __graft_entry__.load_package()
        self.harness = importlib.import_module("harness")
        if libdir:
            libdir = os.path.abspath(libdir)      # dlopen reads a bare relative name as a search name
            self.pkg.LIB_PATH = os.path.join(libdir, "libgpt2amd.so")
            self.harness.LIB_PATH = os.path.join(libdir, "libgpt2bench.so")
            raw = C.CDLL(self.pkg.LIB_PATH)
            for name in list(self.pkg.SIGNATURES):     # an older build may lack newer entry points
                if not hasattr(raw, name):
                    del self.pkg.SIGNATURES[name]
        self.L = self.pkg.lib()
        self.H = self.harness.lib(self.pkg)
        self.synth = importlib.import_module(self.pkg.__name__ + ".synth")
        self.keep = []

    def dev(self, a):
        d = self.pkg.Dev.from_numpy(np.ascontiguousarray(a))
        self.keep.append(d)
        return d

    def empty(self, n):
        d = self.pkg.Dev(n)
        self.keep.append(d)
        return d


def f16(rng, shape, std):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float16)


def big_alloc(env, gib):
    """Allocate, touch and free `gib` GiB of device memory (the order bench.py's peaks leg runs in)."""
    if gib <= 0:
        return
    n = int(gib * (1 << 30))
    d = env.pkg.Dev(n)
    env.L.gpt2_memset(d.ptr, 1, n)
    env.L.gpt2_sync()
    d.free()


def skinny_knob(env, knobs):
    """Applies the skinny knob for one sample (-1: the library's default); returns -1, the value to
    restore, or None when the build has no such hook."""
    L = env.L
    if not hasattr(L, "gpt2_tune_gemm_skinny"):
        return None
    L.gpt2_tune_gemm_skinny(int(knobs.get("skinny", -1)))
    return -1


class OpsWorkload:
    """A list of harness ops timed as one step; a sample is the mean step time over `burst` steps."""

    def __init__(self, env, ops, burst):
        self.env, self.burst = env, burst
        self.arr = (env.harness.GPT2BenchOp * len(ops))(*ops)
        self.n = len(ops)

    def sample(self, knobs):
        env = self.env
        cfg = int(knobs.get("gemm_cfg", -1))
        if hasattr(env.L, "gpt2_tune_gemm_force"):
            env.L.gpt2_tune_gemm_force(cfg)
        prev = skinny_knob(env, knobs)
        ms = C.c_float()
        rc = env.H.gpt2_bench_ops(self.arr, self.n, 2, self.burst, C.byref(ms), None)
        if hasattr(env.L, "gpt2_tune_gemm_force"):
            env.L.gpt2_tune_gemm_force(-1)
        if prev is not None:
            env.L.gpt2_tune_gemm_skinny(prev)
        if rc:
            env.pkg.check("gpt2_bench_ops")
            raise RuntimeError(f"gpt2_bench_ops rc={rc}")
        return ms.value * 1e3


def make_gemm_set(env, knobs, int8=False, only=None):
    rng = np.random.default_rng(1234)
    H = env.harness
    M = int(knobs.get("m", 512))
    X = env.dev(f16(rng, (M, 768), 1.0))
    Xf = env.dev(f16(rng, (M, 3072), 1.0))
    # plain GEMM (harness kind 0 fp16 / 1 INT8), or the fused epilogue: 8 gelu, 6 residual added into C
    # (C then starts as data, not as whatever the allocation held)
    epi = {"gelu": 8, "resid": 6}.get(knobs.get("epi", ""), None)
    if epi is None:
        outs = {k: env.empty(M * SHAPES[k][0] * 2) for k in ORDER}
    else:
        outs = {k: env.dev(f16(np.random.default_rng(99), (M, SHAPES[k][0]), 1.0)) for k in ORDER}
    ops = []
    for _ in range(12):
        for k in ORDER if only is None else [only]:
            N, K = SHAPES[k]
            A = Xf if K == 3072 else X
            b = env.dev(f16(rng, N, 0.01))
            if int8:
                W = env.dev(rng.integers(-127, 128, (N, K), dtype=np.int8))
                s = env.dev((rng.random(N, dtype=np.float32) * np.float32(2e-4) + np.float32(1e-4)))
                ops.append(H.GPT2BenchOp(epi or 1, outs[k].ptr, A.ptr, W.ptr, s.ptr, b.ptr, M, N, K))
            else:
                W = env.dev(f16(rng, (N, K), 0.02))
                ops.append(H.GPT2BenchOp(epi or 0, outs[k].ptr, A.ptr, W.ptr, None, b.ptr, M, N, K))
    return OpsWorkload(env, ops, burst=10)


def make_head_gemm(env, knobs):
    rng = np.random.default_rng(4242)
    A = env.dev(f16(rng, (512, 768), 1.0))
    W = env.dev(f16(rng, (50257, 768), 0.02))
    Cm = env.empty(512 * 50257 * 2)
    return OpsWorkload(env, [env.harness.GPT2BenchOp(0, Cm.ptr, A.ptr, W.ptr, None, None, 512, 50257, 768)], burst=10)


def make_gemv_chain(env, knobs):
    rng = np.random.default_rng(4321)
    fp16 = knobs.get("dtype", "int8") == "fp16"
    x768, x3072 = env.dev(f16(rng, 768, 1.0)), env.dev(f16(rng, 3072, 1.0))
    y = env.empty(3072 * 2)
    ops = []
    for _ in range(12):
        for k in ORDER:
            N, K = SHAPES[k]
            x = x3072 if K == 3072 else x768
            b = env.dev(f16(rng, N, 0.01))
            if fp16:
                W = env.dev(f16(rng, (N, K), 0.02))
                ops.append(env.harness.GPT2BenchOp(2, y.ptr, x.ptr, W.ptr, None, b.ptr, 1, N, K))
            else:
                W = env.dev(rng.integers(-127, 128, (N, K), dtype=np.int8))
                s = env.dev(np.full(N, 1e-3, np.float32))
                ops.append(env.harness.GPT2BenchOp(3, y.ptr, x.ptr, W.ptr, s.ptr, b.ptr, 1, N, K))
    return OpsWorkload(env, ops, burst=20)


def make_gemv(env, knobs):
    """One trunk GEMV (knob shape), INT8 or fp16 (knob dtype); cold (knob cold=1, the default): the
    launches rotate over >= 600 MB of weight copies, so each streams from HBM; gemv_cfg=C forces
    GEMV config C (the harness's kind 256 + C), -1 the library's pick."""
    rng = np.random.default_rng(4321)
    name = knobs.get("shape", "mlp_proj")
    N, K = (50257, 768) if name == "head" else SHAPES[name]
    fp16 = knobs.get("dtype", "int8") == "fp16"
    cold = int(knobs.get("cold", 1)) != 0
    cfg = int(knobs.get("gemv_cfg", -1))
    x = env.dev(f16(rng, K, 1.0))
    y = env.empty(N * 2)
    b = env.dev(f16(rng, N, 0.01))
    nb = N * K * (2 if fp16 else 1)
    copies = max(1, int(600e6 // nb) + 1) if cold else 1
    big = env.empty(copies * nb)
    w_host = f16(rng, (N, K), 0.02) if fp16 else rng.integers(-127, 128, (N, K), dtype=np.int8)
    env.L.gpt2_h2d(big.ptr, w_host.ctypes.data, nb)
    env.L.gpt2_sync()
    s = None if fp16 else env.dev(np.full(N, 1e-3, np.float32))
    for r in range(1, copies):
        env.L.gpt2_d2d(big.ptr + r * nb, big.ptr, nb)
    env.L.gpt2_sync()
    kind = 256 + cfg if cfg >= 0 else (2 if fp16 else 3)
    ops = [env.harness.GPT2BenchOp(kind, y.ptr, x.ptr, big.ptr + r * nb, s.ptr if s is not None else None, b.ptr, 1,
                                   N, K) for r in range(copies)]

    class GemvWorkload(OpsWorkload):
        def sample(self, knobs):
            return OpsWorkload.sample(self, knobs) / copies   # us per launch

    return GemvWorkload(env, ops, burst=3 if cold else 300)


class EmptyWorkload:
    def __init__(self, env, knobs):
        self.env = env

    def sample(self, knobs):
        ms = C.c_float()
        if self.env.H.gpt2_bench_empty(200, C.byref(ms)):
            raise RuntimeError("gpt2_bench_empty")
        return ms.value * 1e3


class DecodeWorkload:
    """One GPT-2-124M decode step (seeded body, base seed 1234) after a prefill of max(pos) tokens; a
    sample is the median of 8 single steps, each re-pinned at `pos`.  The model, cache and graph are
    built per (backend, mode) on first use, so both sides of an in-process A/B share nothing but the
    device."""

    def __init__(self, env, knobs):
        self.env, self.cache = env, {}
        self.body = env.synth.make_body(seed=1234, plain=True)

    def state(self, backend, mode, P, holds=(-1, -1, -1)):
        key = (backend, mode, P, holds)
        if key not in self.cache:
            env, pkg, L = self.env, self.env.pkg, self.env.L
            model = pkg.Model(self.body)
            if backend == "int8":
                model.quantize()
            kv, scr = pkg.KVCache(1024), pkg.Scratch(1024)
            d_ids = env.dev(env.synth.token_ids(P, seed=1234))
            logits, tokens = env.empty(50257 * 2), env.empty(1024 * 4)
            caps = pkg.GPT2CapsGPU()
            caps.logits, caps.logits_all = logits.ptr, 0
            be = pkg.backend(backend)
            L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, P, C.byref(scr.s), C.byref(caps))
            L.gpt2_sync()
            pkg.check("prefill")
            first = int(np.argmax(pkg.half_bits_to_f32(logits.numpy(np.uint16, (50257,)))))
            m = {"persistent": pkg.DECODE_PERSISTENT, "multi": pkg.DECODE_MULTI}[mode]
            def tune(name, *args):          # an older build (lib=) may lack these hooks
                if hasattr(L, name):
                    getattr(L, name)(*args)
            tune("gpt2_tune_decode_holds", *holds)
            g = L.gpt2_decode_graph_create_mode(be, C.byref(model.gpu), C.byref(kv.kv), C.byref(scr.s), logits.ptr,
                                                tokens.ptr, m)
            tune("gpt2_tune_decode_holds", -1, -1, -1)
            if not g:
                pkg.check("graph create")
                raise RuntimeError("graph create failed")
            self.cache[key] = (model, kv, scr, g, first)
        return self.cache[key]

    def sample(self, knobs):
        L = self.env.L
        pos = int(knobs.get("pos", 512))
        holds = tuple(int(v) for v in knobs.get("holds", "-1/-1/-1").split("/"))
        _, _, _, g, first = self.state(knobs.get("backend", "int8"), knobs.get("mode", "persistent"), max(pos, 1),
                                       holds)
        ms, out = C.c_float(), []
        for _ in range(10):
            L.gpt2_decode_graph_set(g, first, pos)
            L.gpt2_decode_graph_time(g, 1, C.byref(ms))
            out.append(ms.value)
        tok, p = C.c_int(), C.c_int()
        if L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(p)):
            self.env.pkg.check("decode")
            raise RuntimeError("decode step failed")
        return float(np.median(out[2:])) * 1e3


class PrefillWorkload:
    def __init__(self, env, knobs):
        self.env, self.cache = env, {}
        self.body = env.synth.make_body(seed=1234, plain=True)

    def state(self, backend, T):
        key = (backend, T)
        if key not in self.cache:
            env, pkg = self.env, self.env.pkg
            model = pkg.Model(self.body)
            if backend == "int8":
                model.quantize()
            kv, scr = pkg.KVCache(max(T, 1)), pkg.Scratch(max(T, 1))
            d_ids = env.dev(env.synth.token_ids(T, seed=1))
            logits = env.empty(50257 * 2)
            caps = pkg.GPT2CapsGPU()
            caps.logits, caps.logits_all = logits.ptr, 0
            self.cache[key] = (model, kv, scr, d_ids, caps)
        return self.cache[key]

    def sample(self, knobs):
        env, L = self.env, self.env.L
        backend, T = knobs.get("backend", "int8"), int(knobs.get("T", 512))
        model, kv, scr, d_ids, caps = self.state(backend, T)
        if hasattr(L, "gpt2_tune_prefill_persistent"):
            L.gpt2_tune_prefill_persistent(int(knobs.get("prefill_persistent", -1)))
        if hasattr(L, "gpt2_tune_prefill_lnfold"):
            L.gpt2_tune_prefill_lnfold(int(knobs.get("lnfold", -1)))
        prev = skinny_knob(env, knobs)
        be = env.pkg.backend(backend)
        out = []
        for _ in range(5):
            L.gpt2_sync()
            t = time.perf_counter()
            L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, T, C.byref(scr.s), C.byref(caps))
            L.gpt2_sync()
            out.append((time.perf_counter() - t) * 1e6)
        if hasattr(L, "gpt2_tune_prefill_persistent"):
            L.gpt2_tune_prefill_persistent(-1)
        if hasattr(L, "gpt2_tune_prefill_lnfold"):
            L.gpt2_tune_prefill_lnfold(-1)
        if prev is not None:
            L.gpt2_tune_gemm_skinny(prev)
        env.pkg.check("prefill")
        return float(np.median(out[1:]))


def make_workload(env, name, knobs):
    big_alloc(env, float(knobs.get("big_alloc", 0)))
    if name == "gemm_set":
        return make_gemm_set(env, knobs, int8=knobs.get("dtype") == "int8")
    if name == "gemm_int8_set":
        return make_gemm_set(env, knobs, int8=True)
    if name == "gemm_shape":
        return make_gemm_set(env, knobs, int8=knobs.get("dtype") == "int8", only=knobs.get("shape", "mlp_proj"))
    if name == "gemv":
        return make_gemv(env, knobs)
    if name == "head_gemm":
        return make_head_gemm(env, knobs)
    if name == "gemv_chain":
        return make_gemv_chain(env, knobs)
    if name == "decode_step":
        return DecodeWorkload(env, knobs)
    if name == "prefill":
        return PrefillWorkload(env, knobs)
    if name == "empty":
        return EmptyWorkload(env, knobs)
    raise SystemExit(f"unknown workload {name}")


# ------------------------------------------------------------------------------ drivers
def worker(args):
    """One side's samples in its own process (a variant build): prints a JSON list."""
    knobs = parse_spec(args.spec)
    env = Env(knobs.get("lib"))
    w = make_workload(env, args.workload, knobs)
    w.sample(knobs)                      # first sample untimed (setup, clocks)
    print(json.dumps([w.sample(knobs) for _ in range(args.samples)]), flush=True)


def run_subprocess(workload, spec, samples):
    cmd = [sys.executable, os.path.abspath(__file__), "--worker", workload, "--spec", spec, "--samples", str(samples)]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if out.returncode:
        raise SystemExit(f"worker failed ({spec}): {out.stderr[-2000:]}")
    return json.loads(out.stdout.strip().splitlines()[-1])


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("workload")
    ap.add_argument("--a", default="")
    ap.add_argument("--b", default="")
    ap.add_argument("--rounds", type=int, default=15)
    ap.add_argument("--json", action="store_true", help="print the result as one JSON line")
    ap.add_argument("--worker", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--spec", default="", help=argparse.SUPPRESS)
    ap.add_argument("--samples", type=int, default=3, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.worker:
        worker(args)
        return
    ka, kb = parse_spec(args.a), parse_spec(args.b)
    sa, sb = [], []
    if "lib" in ka or "lib" in kb:
        # variant builds: alternate worker processes, 3 samples per process, A B / B A order
        for r in range(args.rounds):
            for side in ((0, 1) if r % 2 == 0 else (1, 0)):
                spec = args.a if side == 0 else args.b
                got = run_subprocess(args.workload, spec, 3)
                (sa if side == 0 else sb).append(float(np.median(got)))
            print(f"round {r}: A {sa[-1]:.2f}  B {sb[-1]:.2f} us", file=sys.stderr, flush=True)
    else:
        env = Env()
        wa = make_workload(env, args.workload, ka)
        # the same workload object serves both sides unless their buffers would differ
        same = all(ka.get(k) == kb.get(k) for k in ("big_alloc", "dtype", "shape", "gemv_cfg", "cold", "epi", "m"))
        wb = wa if same else make_workload(env, args.workload, kb)
        wa.sample(ka)
        wb.sample(kb)
        for r in range(args.rounds):
            for side in ((0, 1) if r % 2 == 0 else (1, 0)):
                if side == 0:
                    sa.append(wa.sample(ka))
                else:
                    sb.append(wb.sample(kb))
            print(f"round {r}: A {sa[-1]:.2f}  B {sb[-1]:.2f} us", file=sys.stderr, flush=True)
    A, B = stats(sa), stats(sb)
    res = {"workload": args.workload, "a": args.a, "b": args.b, "rounds": args.rounds, "unit": "us",
           "A": {k: round(v, 3) if isinstance(v, float) else v for k, v in A.items()},
           "B": {k: round(v, 3) if isinstance(v, float) else v for k, v in B.items()}, **verdict(A, B)}
    if args.json:
        print(json.dumps(res), flush=True)
        return
    for tag, spec, s in (("A", args.a, A), ("B", args.b, B)):
        spread = 100.0 * (s["max"] - s["min"]) / s["median"]
        print(f"  {args.workload:<14} {tag} [{spec or 'default'}]  {s['median']:10.3f} us "
              f"[{s['min']:.3f}-{s['max']:.3f}] (+-{spread:.2f}%)  n={s['n']}")
    print(f"  speedup B vs A: {res['speedup_b_vs_a']:.3f}x   {res['verdict']}")


if __name__ == "__main__":
    main()
