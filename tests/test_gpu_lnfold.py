"""The prefill's LayerNorm fold: LN1 and LN2 folded into the QKV and fc GEMMs (the GEMM that produces
the residual stream -- the embedding, attn-proj, mlp-proj -- also writes x*gamma of the next
LayerNorm and 48 partial row sums; the consumer finishes the LayerNorm in its epilogue).

It is not bit-identical to LayerNorm-then-GEMM (the fp16 rounding moves from the normalized row to
x*gamma, the variance comes from the sums), so it is held to the fp16 gates:
  against the unfolded launch sequence at every captured stage: every layer's residual stream, the
  final LayerNorm, all logits rows, the K/V cache (rel_err <= 5e-3; logits KL < 2e-3);
  against the fp32 CPU oracle (rel_err <= 1e-2 per stage, KL < 0.02; INT8 on the dequantized body);
and to exactness where the fold decides alone: the same call twice gives the same bits; every one of
the 47 sites ran folded (12 QKV + 12 attn-proj + 12 fc + 11 mlp-proj: the last mlp-proj has no next
LN1); no site runs folded at T = 1 or with the fold switched off, and at its default only up to the
measured lengths; the cached per-weights constants follow the weights (new weights after
gpt2_free_gpu, INT8 codes after gpt2_quant_build).
"""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

V, E = 50257, 768
SITES = 47


def rel_err(got, ref):
    return float(np.abs(got.astype(np.float64) - ref).max() / (np.abs(ref).max() + 1e-9))


def kl_rows(ref, got):
    def logsm(x):
        x = x.astype(np.float64)
        m = x.max(axis=-1, keepdims=True)
        return x - m - np.log(np.exp(x - m).sum(axis=-1, keepdims=True))
    lr, lg = logsm(ref), logsm(got)
    return (np.exp(lr) * (lr - lg)).sum(axis=-1)


def f32(a):
    return oracle.f16_to_f32(a)


@pytest.fixture(scope="module")
def model(pkg, synth):
    m = pkg.Model(synth.make_body(seed=77, plain=False))
    yield m
    m.free()


def prefill(pkg, L, model, backend, ids, lnfold):
    """The launch-sequence prefill (persistent trunk off) with the fold on, off or at its default
    (lnfold None); returns every capture as fp16 bits and the number of sites that ran folded."""
    T = len(ids)
    d_ids = pkg.Dev.from_numpy(np.asarray(ids, np.int32))
    scr, kv = pkg.Scratch(T), pkg.KVCache(T)
    logits, blocks, fin = pkg.Dev(T * V * 2), pkg.Dev(12 * T * E * 2), pkg.Dev(T * E * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all, caps.final_ln, caps.blocks = logits.ptr, 1, fin.ptr, blocks.ptr
    L.gpt2_memset(kv.kv.data, 0, kv.kv.bytes)
    L.gpt2_tune_prefill_persistent(0)
    L.gpt2_tune_prefill_lnfold(-1 if lnfold is None else (1 if lnfold else 0))
    try:
        L.gpt2_prefill_fill_cache(pkg.backend(backend), C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, T,
                                  C.byref(scr.s), C.byref(caps))
        L.gpt2_sync()
        pkg.check(f"prefill lnfold={lnfold}")
        sites = L.gpt2_tune_prefill_lnfold_sites()
    finally:
        L.gpt2_tune_prefill_lnfold(-1)
        L.gpt2_tune_prefill_persistent(-1)
    cache = np.empty(kv.kv.bytes // 2, np.uint16)
    assert L.gpt2_d2h(cache.ctypes.data, kv.kv.data, cache.nbytes) == 0
    out = {"blocks": blocks.numpy(np.uint16, (12, T, E)), "final_ln": fin.numpy(np.uint16, (T, E)),
           "logits": logits.numpy(np.uint16, (T, V)), "kv": cache}
    scr.free()
    kv.free()
    return out, sites


def drop_int8(L, model):
    L.gpt2_quant_free(C.byref(model.q))
    model.q = None
    model.gpu.q = None


def assert_close(got, ref, tol=5e-3):
    for Lyr in range(12):
        assert rel_err(f32(got["blocks"][Lyr]), f32(ref["blocks"][Lyr])) <= tol, ("layer", Lyr)
    for k in ("final_ln", "logits", "kv"):
        assert rel_err(f32(got[k]), f32(ref[k])) <= tol, k
    assert kl_rows(f32(ref["logits"]), f32(got["logits"])).max() < 2e-3


@pytest.mark.parametrize("backend", ["flash", "int8"])
@pytest.mark.parametrize("T", [2, 17, 64, 200, 512, 1024])
def test_lnfold_matches_unfolded(pkg, L, synth, model, backend, T):
    ids = synth.token_ids(T, seed=T + 11)
    if backend == "int8":
        model.quantize()
    try:
        print(f"lnfold {backend} T={T}", flush=True)
        got, sites = prefill(pkg, L, model, backend, ids, True)
        again, _ = prefill(pkg, L, model, backend, ids, True)
        ref, sites_off = prefill(pkg, L, model, backend, ids, False)
    finally:
        if backend == "int8":
            drop_int8(L, model)
    assert sites == SITES
    assert sites_off == 0
    assert_close(got, ref)
    for k in got:
        assert np.array_equal(got[k], again[k]), f"{k}: not deterministic"


@pytest.mark.parametrize("backend,T", [("flash", 64), ("int8", 64), ("flash", 300), ("int8", 1024)])
def test_lnfold_vs_oracle(pkg, L, synth, model, backend, T):
    body = synth.make_body(seed=77, plain=False)
    ref_body = oracle.fp16_view(body)
    ids = synth.token_ids(T, seed=T + 5)
    if backend == "int8":
        off = synth.offsets()
        for Lyr in range(12):
            for name in ("qkv_w", "attn_proj_w", "fc_w", "proj_w"):
                o, shape = off[f"h{Lyr}.{name}"]
                n = int(np.prod(shape))
                q, s, _ = oracle.quantize_fp16_view(body[o:o + n].reshape(shape))
                ref_body[o:o + n] = oracle.dequantize(q, s).reshape(-1)
        model.quantize()
    try:
        print(f"lnfold vs oracle {backend} T={T}", flush=True)
        got, sites = prefill(pkg, L, model, backend, ids, True)
    finally:
        if backend == "int8":
            drop_int8(L, model)
    assert sites == SITES
    ref = oracle.forward(ref_body, ids, logits_all=True, want_blocks=True)
    for Lyr in range(12):
        assert rel_err(f32(got["blocks"][Lyr]), ref["blocks"][Lyr]) <= 1e-2, Lyr
    assert rel_err(f32(got["final_ln"]), ref["final_ln"]) <= 1e-2
    lg = f32(got["logits"])
    assert rel_err(lg, ref["logits"]) <= 1e-2
    assert kl_rows(ref["logits"], lg).max() < 0.02


@pytest.mark.parametrize("backend,T,sites", [("flash", 16, 0), ("flash", 32, 0), ("flash", 33, SITES), ("int8", 64, 0),
                                              ("int8", 65, SITES),
                                              ("flash", 128, SITES), ("flash", 129, 0), ("int8", 256, SITES),
                                              ("int8", 257, 0), ("flash", 512, 0)])
def test_lnfold_default_by_length(pkg, L, synth, model, backend, T, sites):
    """Left at its default, the fold runs where it measured faster: T <= 128, INT8 up to 256, above the
    skinny GEMM's rows (T <= 32 fp16, <= 64 INT8: its LayerNorm prologue takes LN1 and LN2)."""
    ids = synth.token_ids(T, seed=T)
    if backend == "int8":
        model.quantize()
    try:
        _, got = prefill(pkg, L, model, backend, ids, None)
    finally:
        if backend == "int8":
            drop_int8(L, model)
    assert got == sites


def test_lnfold_not_at_t1(pkg, L, synth, model):
    """One row: the matmuls are GEMVs, the fold does not apply (and the result is the unfolded one)."""
    ids = synth.token_ids(1, seed=9)
    got, sites = prefill(pkg, L, model, "flash", ids, True)
    ref, _ = prefill(pkg, L, model, "flash", ids, False)
    assert sites == 0
    for k in got:
        assert np.array_equal(got[k], ref[k]), k


def test_lnfold_constants_follow_weights(pkg, L, synth):
    """The fold's per-weights constants are cached by the weights' device address: freed weights
    drop them, so a second model (here often at the same address) gets its own; INT8 codes get their
    own table beside the fp16 one."""
    T = 96
    ids = synth.token_ids(T, seed=4)
    for seed in (5, 6):
        m = pkg.Model(synth.make_body(seed=seed, plain=False))
        try:
            print(f"lnfold constants seed={seed}", flush=True)
            got, sites = prefill(pkg, L, m, "flash", ids, True)
            ref, _ = prefill(pkg, L, m, "flash", ids, False)
            assert sites == SITES
            assert_close(got, ref)
            m.quantize()
            try:
                got, sites = prefill(pkg, L, m, "int8", ids, True)
                ref, _ = prefill(pkg, L, m, "int8", ids, False)
            finally:
                drop_int8(L, m)
            assert sites == SITES
            assert_close(got, ref)
            got, _ = prefill(pkg, L, m, "flash", ids, True)   # the fp16 table again
            ref, _ = prefill(pkg, L, m, "flash", ids, False)
            assert_close(got, ref)
        finally:
            m.free()


def hip_runtime():
    h = C.CDLL("libamdhip64.so")
    for name in ("hipStreamCreate", "hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate",
                 "hipGraphLaunch", "hipStreamSynchronize", "hipGraphExecDestroy", "hipGraphDestroy",
                 "hipStreamDestroy"):
        getattr(h, name).restype = C.c_int
    return h


@pytest.mark.parametrize("warm", [True, False])
def test_lnfold_under_graph_capture(pkg, L, synth, warm):
    """gpt2_forward_cuda at T = 96 (inside the fold's default range) captured into a HIP graph on a
    stream of its own.  warm: the weights' fold constants exist (an eager call built them), so the
    captured forward runs folded (47 sites) and every replay equals the eager folded call bit for bit.
    cold: fresh weights, so the constants would need an allocation, which is not made under capture;
    the captured forward runs unfolded (0 sites) and every replay equals the eager unfolded call.
    Between the replays the eager forward runs on other ids at the default (in the cold case that
    builds the constants; the instantiated graph is unaffected)."""
    hip = hip_runtime()
    m = pkg.Model(synth.make_body(seed=21 if warm else 22, plain=False))
    T = 96
    ids, other = synth.token_ids(T, seed=61), synth.token_ids(T, seed=62)
    d_ids, d_other = pkg.Dev.from_numpy(np.asarray(ids, np.int32)), pkg.Dev.from_numpy(np.asarray(other, np.int32))
    scr = pkg.Scratch(T)
    logits, fin = pkg.Dev(T * V * 2), pkg.Dev(T * E * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all, caps.final_ln = logits.ptr, 1, fin.ptr
    be = pkg.backend("flash")

    def eager(d, lnfold):
        L.gpt2_tune_prefill_lnfold(lnfold)
        try:
            L.gpt2_forward_cuda(be, C.byref(m.gpu), d.ptr, T, C.byref(scr.s), C.byref(caps))
            L.gpt2_sync()
            pkg.check("eager forward")
            sites = L.gpt2_tune_prefill_lnfold_sites()
        finally:
            L.gpt2_tune_prefill_lnfold(-1)
        return (logits.numpy(np.uint16, (T * V,)).copy(), fin.numpy(np.uint16, (T * E,)).copy()), sites

    stream, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    try:
        print(f"lnfold capture warm={warm}", flush=True)
        ref, sites = eager(d_ids, -1 if warm else 0)
        assert sites == (SITES if warm else 0)
        assert hip.hipStreamCreate(C.byref(stream)) == 0
        L.gpt2_set_stream(stream)
        assert hip.hipStreamBeginCapture(stream, 1) == 0          # hipStreamCaptureModeThreadLocal
        L.gpt2_forward_cuda(be, C.byref(m.gpu), d_ids.ptr, T, C.byref(scr.s), C.byref(caps))
        captured_sites = L.gpt2_tune_prefill_lnfold_sites()
        assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
        pkg.check("capture")
        assert captured_sites == (SITES if warm else 0)
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for r in range(3):
            eager(d_other, -1)
            L.gpt2_memset(logits.ptr, 0, T * V * 2)
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            pkg.check("replay")
            got = (logits.numpy(np.uint16, (T * V,)), fin.numpy(np.uint16, (T * E,)))
            for name, a, b in zip(("logits", "final_ln"), got, ref):
                assert np.array_equal(a, b), f"replay {r}: {name} differs in {np.count_nonzero(a != b)} elements"
    finally:
        L.gpt2_set_stream(None)
        if exe:
            hip.hipGraphExecDestroy(exe)
        if graph:
            hip.hipGraphDestroy(graph)
        if stream:
            hip.hipStreamDestroy(stream)
        scr.free()
        m.free()
