"""Phase timeline of the persistent decode step (one kernel per token).

Runs a P=512 prefill of a seeded GPT-2-124M-shaped body (INT8 trunk, fp16 head, as bench.py's decode
leg), creates a persistent decode graph with the profiling hook `gpt2_tune_decode_trace` set, replays
it `--reps` times at position 512 and prints, per layer, when each phase's input arrived and when its
work-groups finished (s_memrealtime, 100 MHz), plus the layer-1 sub-phase marks.

    python bench/decode_trace.py [--reps 20] [--backend int8]

Phases per layer l: 4l attention work-groups (0..47: LN1, q/k/v, attention), 4l+1 proj, 4l+2 fc,
4l+3 mlp-proj (GEMV work-groups 48..239).  "wait" is the median arrival of a phase's input minus the
latest end of the phase before it; "compute" is the latest end minus the median arrival.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib
import os
import sys

import numpy as np

NA, NG = 48, 192          # attention work-groups; GEMV work-groups with rows


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--backend", default="int8")
    args = ap.parse_args()

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, root)
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    L = pkg.lib()
    synth = importlib.import_module(pkg.__name__ + ".synth")

    body = synth.make_body(seed=1234, plain=True)
    model = pkg.Model(body)
    model.quantize()                       # 48 trunk tensors INT8, head fp16
    kv, scr = pkg.KVCache(1024), pkg.Scratch(1024)
    P = 512
    d_ids = pkg.Dev.from_numpy(synth.token_ids(P, seed=1234))
    logits, tokens = pkg.Dev(50257 * 2), pkg.Dev(1024 * 4)
    be = pkg.backend(args.backend)
    caps = pkg.GPT2CapsGPU()
    caps.logits = logits.ptr
    caps.logits_all = 0
    L.gpt2_prefill_fill_cache(be, C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, P, C.byref(scr.s), C.byref(caps))
    L.gpt2_sync()
    pkg.check("prefill")

    tr = pkg.Dev(256 * 128 * 8)
    L.gpt2_memset(tr.ptr, 0, 256 * 128 * 8)
    L.gpt2_tune_decode_trace(tr.ptr)
    g = L.gpt2_decode_graph_create_mode(be, C.byref(model.gpu), C.byref(kv.kv), C.byref(scr.s), logits.ptr,
                                        tokens.ptr, pkg.DECODE_PERSISTENT)
    L.gpt2_tune_decode_trace(None)
    if not g or L.gpt2_decode_graph_mode(g) != pkg.DECODE_PERSISTENT:
        raise SystemExit("the persistent step is not available for this backend")
    ms = C.c_float()
    for _ in range(args.reps):
        L.gpt2_decode_graph_set(g, 1000, P)
        L.gpt2_decode_graph_time(g, 1, C.byref(ms))
    tok, pos = C.c_int(), C.c_int()
    rc = L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos))
    print("last replay: %.1f us (graph launch included), status %d" % (ms.value * 1000.0, rc))

    t = tr.numpy(np.uint64, (256, 128)).astype(np.int64)
    rel = (t - t[:, 63].min()) * 0.01                  # us since the first work-group started
    print("shader clock %.3f GHz" % ((t[0, 127] - t[0, 126]) / ((t[0, 62] - t[0, 63]) * 10.0)))
    st = rel[:, 63]
    print("work-group start: median %.2f, max %.2f us (attention work-groups max %.2f); layer 0 attention "
          "input %.2f us after its work-group started (median)" % (
              np.median(st), st.max(), st[:NA].max(), np.median(rel[:NA, 64] - st[:NA])))
    names = ["attention", "proj", "fc", "mlp-proj"]
    sets = [slice(0, NA), slice(NA, NA + NG), slice(NA, NA + NG), slice(NA, NA + NG)]
    prev = 0.0
    tot_wait = tot_comp = 0.0
    print("layer  phase      input arrived (med/max)   end (med/max)     +step   wait  compute")
    for l in range(12):
        for k in range(4):
            p = 4 * l + k
            end, arr = rel[sets[k], p], rel[sets[k], 64 + p]
            wait, comp = np.median(arr) - prev, end.max() - np.median(arr)
            tot_wait += wait
            tot_comp += comp
            print("%5d  %-9s %9.2f %9.2f   %9.2f %9.2f   %6.2f %6.2f %6.2f" % (
                l, names[k], np.median(arr), arr.max(), np.median(end), end.max(), end.max() - prev, wait, comp))
            prev = end.max()
    print("12 layers: %.1f us waiting for inputs, %.1f us computing" % (tot_wait, tot_comp))
    a = rel[0:NA]
    print("layer 1, attention work-groups (medians): input %.2f, weights landed %.2f, LN1 %.2f, q/k/v %.2f, "
          "attention %.2f, merged %.2f, stored %.2f" % tuple(np.median(a[:, c]) for c in (68, 113, 114, 115, 116, 117, 118)))
    rounds = t[0:NA, 123]
    print("layer 1 poll for x: %d-%d rounds, %.3f us per round" % (
        rounds.min(), rounds.max(), np.median((a[:, 68] - a[:, 122]) / (rounds + 1))))
    gw = rel[NA:NA + NG]
    print("layer 1, GEMV work-groups (medians): proj input %.2f, combined %.2f, proj end %.2f | fc input %.2f, "
          "LN2 %.2f, fc rows %.2f, fc end %.2f" % tuple(np.median(gw[:, c]) for c in (69, 118, 5, 70, 120, 121, 6)))
    print("head: start max %.2f, end max %.2f; step end %.2f us" % (rel[:, 60].max(), rel[:, 61].max(), rel[0, 62]))
    L.gpt2_decode_graph_destroy(g)


if __name__ == "__main__":
    main()
