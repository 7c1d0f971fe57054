"""gpt2_forward_noalloc (the forward with its activations in a static device array, no allocation)
against gpt2_forward_cuda (the same forward on an allocated GPT2ScratchGPU).  The no-allocation entry
point runs the per-op launch sequence unfolded (the persistent trunk kernel allocates its arena, and
the LayerNorm fold its per-weights constants, on first use), so it matches gpt2_forward_cuda with
both switched off bit for bit -- all logits rows, the final LayerNorm, every layer's residual stream
and the K/V cache it fills -- and gpt2_forward_cuda with the fold on (the default), or with the
persistent kernel on, within the fp16 gates.  Two calls in a row, the second with fewer tokens
(the array keeps the first call's contents), for the fp16 and the INT8 backend; and a call past the
static limit is refused with an error and writes nothing.  The property itself: across a call, the
library's allocation count (every device allocation goes through gpt2_dmalloc) and the device's free
memory (hipMemGetInfo) do not change; and one call captured into a HIP graph, replayed three times
with eager work between the replays, matches the eager call bit for bit on every replay."""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

V, E = 50257, 768


def run(pkg, L, model, backend, ids, noalloc):
    T = len(ids)
    d_ids = pkg.Dev.from_numpy(np.asarray(ids, np.int32))
    logits, blocks, fin = pkg.Dev(T * V * 2), pkg.Dev(12 * T * E * 2), pkg.Dev(T * E * 2)
    kv = pkg.KVCache(T)
    L.gpt2_memset(kv.kv.data, 0, kv.kv.bytes)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all, caps.final_ln, caps.blocks = logits.ptr, 1, fin.ptr, blocks.ptr
    caps.kv = C.addressof(kv.kv)
    scr = None
    if noalloc:
        L.gpt2_forward_noalloc(pkg.backend(backend), C.byref(model.gpu), d_ids.ptr, T, C.byref(caps))
    else:
        scr = pkg.Scratch(T)
        L.gpt2_forward_cuda(pkg.backend(backend), C.byref(model.gpu), d_ids.ptr, T, C.byref(scr.s), C.byref(caps))
    L.gpt2_sync()
    pkg.check("forward noalloc=%d" % noalloc)
    cache = np.empty(kv.kv.bytes // 2, np.uint16)
    assert L.gpt2_d2h(cache.ctypes.data, kv.kv.data, cache.nbytes) == 0
    out = (logits.numpy(np.uint16, (T * V,)), fin.numpy(np.uint16, (T * E,)), blocks.numpy(np.uint16, (12 * T * E,)),
           cache)
    if scr is not None:
        scr.free()
    kv.free()
    return out


@pytest.fixture(scope="module")
def model(pkg, synth):
    m = pkg.Model(synth.make_body(seed=31, plain=False))
    yield m
    m.free()


@pytest.mark.parametrize("backend", ["flash", "int8"])
def test_forward_noalloc_matches_forward(pkg, L, synth, model, backend):
    if backend == "int8":
        model.quantize()
    try:
        for T in (128, 37):   # the limit, then a smaller call on the same static array
            ids = synth.token_ids(T, seed=T + 3)
            print(f"forward_noalloc backend={backend} T={T}", flush=True)
            got = run(pkg, L, model, backend, ids, noalloc=True)
            # the no-allocation entry point runs the unfolded launch sequence (the LayerNorm fold builds
            # per-weights constants on first use): bit for bit against gpt2_forward_cuda with the
            # fold off, to the fp16 bar against it with the fold on
            L.gpt2_tune_prefill_persistent(0)
            L.gpt2_tune_prefill_lnfold(0)
            try:
                ref = run(pkg, L, model, backend, ids, noalloc=False)
            finally:
                L.gpt2_tune_prefill_persistent(-1)
                L.gpt2_tune_prefill_lnfold(-1)
            for name, a, b in zip(("logits", "final_ln", "blocks", "kv"), got, ref):
                assert np.array_equal(a, b), f"{backend} T={T}: {name} differs in {np.count_nonzero(a != b)} elements"
            L.gpt2_tune_prefill_persistent(0)
            try:
                folded = run(pkg, L, model, backend, ids, noalloc=False)
            finally:
                L.gpt2_tune_prefill_persistent(-1)
            for name, a, b in zip(("logits", "final_ln", "blocks"), got, folded):
                fa, fb = oracle.f16_to_f32(a).astype(np.float64), oracle.f16_to_f32(b).astype(np.float64)
                assert np.abs(fa - fb).max() / (np.abs(fb).max() + 1e-9) <= 1e-2, (backend, T, name, "lnfold")
            L.gpt2_tune_prefill_persistent(1)
            try:
                pers = run(pkg, L, model, backend, ids, noalloc=False)
            finally:
                L.gpt2_tune_prefill_persistent(-1)
            for name, a, b in zip(("logits", "final_ln", "blocks"), got, pers):
                fa, fb = oracle.f16_to_f32(a).astype(np.float64), oracle.f16_to_f32(b).astype(np.float64)
                assert np.abs(fa - fb).max() / (np.abs(fb).max() + 1e-9) <= 1e-2, (backend, T, name)
    finally:
        if backend == "int8":
            L.gpt2_quant_free(C.byref(model.q))
            model.q = None
            model.gpu.q = None


def test_forward_noalloc_rejects_past_limit(pkg, L, synth, model):
    T = 129
    ids = synth.token_ids(T, seed=1)
    d_ids = pkg.Dev.from_numpy(np.asarray(ids, np.int32))
    sentinel = np.full(V, 0x7BFF, np.uint16)
    logits = pkg.Dev.from_numpy(sentinel)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all = logits.ptr, 0
    L.gpt2_last_error()
    L.gpt2_forward_noalloc(pkg.backend("flash"), C.byref(model.gpu), d_ids.ptr, T, C.byref(caps))
    L.gpt2_sync()
    assert L.gpt2_last_error() != 0
    assert np.array_equal(logits.numpy(np.uint16, (V,)), sentinel)


def test_forward_noalloc_allocates_nothing(pkg, L, synth, model):
    """The no-allocation property, measured: after one warm-up call (the first call on a device
    resolves the static array's address and loads the kernels), a second call changes neither the
    library's count of gpt2_dmalloc calls nor the device's free memory."""
    T = 64
    ids = synth.token_ids(T, seed=77)
    d_ids = pkg.Dev.from_numpy(np.asarray(ids, np.int32))
    logits = pkg.Dev(T * V * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all = logits.ptr, 1
    be = pkg.backend("flash")
    L.gpt2_forward_noalloc(be, C.byref(model.gpu), d_ids.ptr, T, C.byref(caps))
    L.gpt2_sync()
    pkg.check("warm-up call")
    n0, f0 = L.gpt2_test_dmalloc_calls(), L.gpt2_test_mem_free()
    L.gpt2_forward_noalloc(be, C.byref(model.gpu), d_ids.ptr, T, C.byref(caps))
    L.gpt2_sync()
    pkg.check("second call")
    n1, f1 = L.gpt2_test_dmalloc_calls(), L.gpt2_test_mem_free()
    assert f0 > 0
    assert n1 == n0, f"gpt2_dmalloc called {n1 - n0} times"
    assert f1 == f0, f"free device memory changed by {f0 - f1} bytes"


def hip_runtime():
    h = C.CDLL("libamdhip64.so")
    for name in ("hipStreamCreate", "hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate",
                 "hipGraphLaunch", "hipStreamSynchronize", "hipGraphExecDestroy", "hipGraphDestroy",
                 "hipStreamDestroy"):
        getattr(h, name).restype = C.c_int
    return h


def test_forward_noalloc_under_graph_capture(pkg, L, synth, model):
    """gpt2_forward_noalloc captured into a HIP graph on a stream of its own (gpt2_set_stream resolves
    the static array's address before the capture begins), the graph replayed three times; between
    the replays the eager call runs again on other ids, so each replay starts from the array holding
    another call's contents.  Every replay matches the eager call on the same ids bit for bit, and the
    whole sequence (capture, instantiation aside) makes no gpt2_dmalloc call."""
    hip = hip_runtime()
    T = 48
    ids, other = synth.token_ids(T, seed=91), synth.token_ids(T, seed=92)
    d_ids, d_other = pkg.Dev.from_numpy(np.asarray(ids, np.int32)), pkg.Dev.from_numpy(np.asarray(other, np.int32))
    logits, fin = pkg.Dev(T * V * 2), pkg.Dev(T * E * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all, caps.final_ln = logits.ptr, 1, fin.ptr
    be = pkg.backend("flash")

    def eager(d):
        L.gpt2_forward_noalloc(be, C.byref(model.gpu), d.ptr, T, C.byref(caps))
        L.gpt2_sync()
        pkg.check("eager noalloc")
        return logits.numpy(np.uint16, (T * V,)).copy(), fin.numpy(np.uint16, (T * E,)).copy()

    ref = eager(d_ids)
    stream, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.hipStreamCreate(C.byref(stream)) == 0
    try:
        L.gpt2_set_stream(stream)
        n0 = L.gpt2_test_dmalloc_calls()
        assert hip.hipStreamBeginCapture(stream, 1) == 0          # hipStreamCaptureModeThreadLocal
        L.gpt2_forward_noalloc(be, C.byref(model.gpu), d_ids.ptr, T, C.byref(caps))
        assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
        pkg.check("capture")
        assert L.gpt2_test_dmalloc_calls() == n0
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for r in range(3):
            eager(d_other)                                          # the array now holds another call
            L.gpt2_memset(logits.ptr, 0, T * V * 2)
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            pkg.check("replay")
            got = (logits.numpy(np.uint16, (T * V,)), fin.numpy(np.uint16, (T * E,)))
            for name, a, b in zip(("logits", "final_ln"), got, ref):
                assert np.array_equal(a, b), f"replay {r}: {name} differs in {np.count_nonzero(a != b)} elements"
        assert L.gpt2_test_dmalloc_calls() == n0
    finally:
        L.gpt2_set_stream(None)
        if exe:
            hip.hipGraphExecDestroy(exe)
        if graph:
            hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(stream)
