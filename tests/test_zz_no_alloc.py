"""gpt2_forward_noalloc (the forward with its activations in a static device array, no allocation)
against gpt2_forward_cuda (the same forward on an allocated GPT2ScratchGPU).  The no-allocation entry
point runs the per-op launch sequence (the persistent trunk kernel allocates its arena on first use),
so it matches gpt2_forward_cuda with that kernel switched off (the default) bit for bit -- all logits
rows, the final LayerNorm, every layer's residual stream and the K/V cache it fills -- and
gpt2_forward_cuda with the persistent kernel switched on within the fp16 gates.  Two calls in a row, the second with fewer tokens
(the array keeps the first call's contents), for the fp16 and the INT8 backend; and a call past the
static limit is refused with an error and writes nothing."""
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
            L.gpt2_tune_prefill_persistent(0)
            try:
                ref = run(pkg, L, model, backend, ids, noalloc=False)
            finally:
                L.gpt2_tune_prefill_persistent(-1)
            for name, a, b in zip(("logits", "final_ln", "blocks", "kv"), got, ref):
                assert np.array_equal(a, b), f"{backend} T={T}: {name} differs in {np.count_nonzero(a != b)} elements"
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
