"""Times the prefill forward of a seeded GPT-2-124M-shaped body (the config-5 prefill).

    python bench/prefill_bench.py [--tokens 512] [--reps 8] [--backend int8] [--unfused] [--ln-cfg C]

Each repetition is one `gpt2_prefill_fill_cache` call (embed, 12 layers, final LayerNorm, the last
row's logits, the K/V cache fill), host-timed around a device sync; the first call is reported
apart (it includes one-time work).  `--backend int8` quantizes the 48 trunk matrices on the GPU first
(head kept fp16), as bench.py's decode leg does.  `--unfused` runs the reference's unfused sequence
(`gpt2_tune_prefill_fused(0)`) for comparison.  `--ln-cfg C` runs LN1 -> QKV and LN2 -> fc as
LayerNorm-panel GEMMs with config C (`gpt2_tune_gemm_ln_force`; off by default).  Run it under `rocprofv3 --kernel-trace --stats` for
the per-kernel split.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib
import os
import sys
import time

import numpy as np


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=512)
    ap.add_argument("--reps", type=int, default=8)
    ap.add_argument("--backend", default="int8")
    ap.add_argument("--unfused", action="store_true")
    ap.add_argument("--ln-cfg", type=int, default=-1)
    args = ap.parse_args()

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, root)
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    L = pkg.lib()
    synth = importlib.import_module(pkg.__name__ + ".synth")

    model = pkg.Model(synth.make_body(seed=1234, plain=True))
    if args.backend == "int8":
        model.quantize()
    T = args.tokens
    kv, scr = pkg.KVCache(max(T, 1)), pkg.Scratch(max(T, 1))
    d_ids = pkg.Dev.from_numpy(synth.token_ids(T, seed=1234))
    logits = pkg.Dev(50257 * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits = logits.ptr
    caps.logits_all = 0
    be = pkg.backend(args.backend)
    L.gpt2_tune_prefill_fused(0 if args.unfused else 1)
    L.gpt2_tune_gemm_ln_force(args.ln_cfg)
    ms = []
    for _ in range(args.reps + 1):
        L.gpt2_sync()
        t = time.perf_counter()
        L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, T, C.byref(scr.s), C.byref(caps))
        L.gpt2_sync()
        ms.append((time.perf_counter() - t) * 1e3)
    L.gpt2_tune_prefill_fused(1)
    L.gpt2_tune_gemm_ln_force(-1)
    pkg.check("prefill")
    mode = "unfused" if args.unfused else "fused"
    if args.ln_cfg >= 0:
        mode += " ln-panel " + L.gpt2_tune_gemm_ln_name(args.ln_cfg).decode()
    print("prefill T=%d backend=%s %s: first %.3f ms, then median %.3f ms (min %.3f) over %d" % (
        T, args.backend, mode, ms[0], float(np.median(ms[1:])), min(ms[1:]), args.reps))


if __name__ == "__main__":
    main()
