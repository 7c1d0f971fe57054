"""Whole-model parity: the prefill forward, the M=1 decode step and the graph-replayed greedy loop.

Gates follow the reference's own (QUALITY_GATES.md, bench/correctness_cuda.cu:70-75,200-219,
bench/kv_gate.cu:114-138), applied to the fp16 engine against the fp32 CPU oracle:
  rel_err = max|got - ref| / max|ref| <= 1e-2 per captured stage (gate (a), fp16 bound),
  max KL(softmax(ref) || softmax(got)) < 0.02 over the logits rows (gate (c)),
  cached decode == no-KV recompute within fp16 noise (the [EQ] gate).
INT8 runs are compared with the oracle on the dequantized weights (tools/dequant_check.py).
The multi-kernel graph decode uses the same kernels in the same order as the eager step, so its
tokens and logits must match the eager loop bit for bit.  The persistent decode step (one kernel per
token) sums in a different order, so it is held to the same fp16 gates against the eager step, and
to exactness where its own logic decides (the greedy token is the first argmax of its own logits,
replays are deterministic).
"""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

V, E = 50257, 768


def rel_err(got, ref):
    return float(np.abs(got.astype(np.float64) - ref).max() / (np.abs(ref).max() + 1e-9))


def kl_rows(ref, got):
    def logsm(x):
        x = x.astype(np.float64)
        m = x.max(axis=-1, keepdims=True)
        return x - m - np.log(np.exp(x - m).sum(axis=-1, keepdims=True))
    lr, lg = logsm(ref), logsm(got)
    return (np.exp(lr) * (lr - lg)).sum(axis=-1)


@pytest.fixture(scope="module")
def body(synth):
    return synth.make_body(seed=555, plain=False)


@pytest.fixture(scope="module")
def model(pkg, body):
    m = pkg.Model(body)
    yield m
    m.free()


@pytest.fixture(scope="module")
def deq_body(synth, body):
    """The fp32 body with every trunk matrix replaced by fl32(q*s) of its fp16 view (head kept)."""
    out = body.copy()
    off = synth.offsets()
    for Lyr in range(12):
        for name in ("qkv_w", "attn_proj_w", "fc_w", "proj_w"):
            o, shape = off[f"h{Lyr}.{name}"]
            q, s, _ = oracle.quantize_fp16_view(body[o:o + int(np.prod(shape))].reshape(shape))
            out[o:o + int(np.prod(shape))] = oracle.dequantize(q, s).reshape(-1)
    return out


def gpu_forward(pkg, L, model, ids, backend="flash", logits_all=True, want_blocks=False):
    T = len(ids)
    scr = pkg.Scratch(T)
    d_ids = pkg.Dev.from_numpy(np.asarray(ids, np.int32))
    logits = pkg.Dev((T if logits_all else 1) * V * 2)
    blocks = pkg.Dev(12 * T * E * 2) if want_blocks else None
    fin = pkg.Dev(T * E * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all, caps.final_ln = logits.ptr, int(logits_all), fin.ptr
    if blocks is not None:
        caps.blocks = blocks.ptr
    L.gpt2_forward_cuda(pkg.backend(backend), C.byref(model.gpu), d_ids.ptr, T, C.byref(scr.s), C.byref(caps))
    L.gpt2_sync()
    pkg.check("forward")
    out = {"logits": oracle.f16_to_f32(logits.numpy(np.uint16, ((T if logits_all else 1), V))),
           "final_ln": oracle.f16_to_f32(fin.numpy(np.uint16, (T, E)))}
    if blocks is not None:
        out["blocks"] = oracle.f16_to_f32(blocks.numpy(np.uint16, (12, T, E)))
    scr.free()
    return out


def test_prefill_forward_fp16(pkg, L, synth, body, model):
    ids = synth.token_ids(24, seed=1)
    got = gpu_forward(pkg, L, model, ids, "flash", want_blocks=True)
    ref = oracle.forward(oracle.fp16_view(body), ids, logits_all=True, want_blocks=True)
    for Lyr in range(12):
        assert rel_err(got["blocks"][Lyr], ref["blocks"][Lyr]) <= 1e-2, Lyr
    assert rel_err(got["final_ln"], ref["final_ln"]) <= 1e-2
    assert rel_err(got["logits"], ref["logits"]) <= 1e-2
    assert kl_rows(ref["logits"], got["logits"]).max() < 0.02
    assert (got["logits"].argmax(-1) == ref["logits"].argmax(-1)).mean() >= 0.95


def test_config1_forward_t64(pkg, L, synth):
    """plain model (biases 0, LN 1/0), 64 random ids, logits [64 x 50257]."""
    b = synth.make_body(seed=1234, plain=True)
    m = pkg.Model(b)
    try:
        ids = synth.token_ids(64, seed=1234)
        got = gpu_forward(pkg, L, m, ids, "flash")
        ref = oracle.forward(oracle.fp16_view(b), ids, logits_all=True)
        assert rel_err(got["logits"], ref["logits"]) <= 1e-2
        assert kl_rows(ref["logits"], got["logits"]).max() < 0.02
    finally:
        m.free()


def test_prefill_forward_backends_agree(pkg, L, synth, model):
    ids = synth.token_ids(17, seed=2)
    outs = {be: gpu_forward(pkg, L, model, ids, be)["logits"] for be in ("naive", "tiled", "flash", "gemv")}
    for be in ("naive", "tiled", "gemv"):
        assert rel_err(outs[be], outs["flash"]) <= 5e-3, be


@pytest.mark.parametrize("backend,T,ln", [("flash", 200, -1), ("int8", 200, -1), ("tiled", 33, -1), ("int8", 512, -1),
                                          ("flash", 200, 1), ("int8", 512, 2), ("flash", 16, -1), ("int8", 40, -1),
                                          ("int8", 2, -1), ("flash", 32, -1), ("int8", 64, -1)])
def test_fused_prefill_bit_identical(pkg, L, synth, model, backend, T, ln):
    """The fused launch sequence of the prefill (gelu and the residual adds in GEMM epilogues, the K/V
    cache fill inside the attention launch; the persistent trunk kernel and the LayerNorm fold
    switched off) equals the unfused reference sequence bit for bit: every layer's residual stream,
    the final LayerNorm, all logits rows and the whole K/V cache.  ln >= 0 also runs LN1 -> QKV and
    LN2 -> fc as LayerNorm-panel GEMMs with that config (at T where the plain GEMMs have one k group).
    At T <= 32 (fp16) or 64 (INT8) the fused sequence runs LN1 -> QKV and LN2 -> fc as the skinny
    GEMM with its LayerNorm prologue (and the other GEMMs as skinny fused epilogues), the unfused one
    the LayerNorm launch and the plain skinny GEMM.  The fold moves rounding points; test_gpu_lnfold holds it to the fp16 gates."""
    ids = synth.token_ids(T, seed=T + 7)
    d_ids = pkg.Dev.from_numpy(np.asarray(ids, np.int32))
    if backend == "int8":
        model.quantize()
    runs = []
    L.gpt2_tune_prefill_persistent(0)
    L.gpt2_tune_prefill_lnfold(0)
    try:
        for fused in (1, 0):
            L.gpt2_tune_prefill_fused(fused)
            L.gpt2_tune_gemm_ln_force(ln if fused else -1)
            scr, kv = pkg.Scratch(T), pkg.KVCache(T)
            logits, blocks, fin = pkg.Dev(T * V * 2), pkg.Dev(12 * T * E * 2), pkg.Dev(T * E * 2)
            caps = pkg.GPT2CapsGPU()
            caps.logits, caps.logits_all, caps.final_ln, caps.blocks = logits.ptr, 1, fin.ptr, blocks.ptr
            L.gpt2_memset(kv.kv.data, 0, kv.kv.bytes)
            calls = L.gpt2_tune_gemm_skinny_calls()
            L.gpt2_prefill_fill_cache(pkg.backend(backend), C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, T,
                                      C.byref(scr.s), C.byref(caps))
            L.gpt2_sync()
            pkg.check("prefill fused=%d" % fused)
            # the 48 trunk GEMMs of a short prompt run as the skinny kernel in both sequences
            skinny = 48 if 2 <= T <= L.gpt2_tune_gemm_skinny_max(backend == "int8") else 0
            assert L.gpt2_tune_gemm_skinny_calls() - calls == skinny, (fused, T)
            assert kv.kv.len == T
            cache = np.empty(kv.kv.bytes // 2, np.uint16)
            assert L.gpt2_d2h(cache.ctypes.data, kv.kv.data, cache.nbytes) == 0
            runs.append((blocks.numpy(np.uint16, (12 * T * E,)), fin.numpy(np.uint16, (T * E,)),
                         logits.numpy(np.uint16, (T * V,)), cache))
            scr.free()
            kv.free()
    finally:
        L.gpt2_tune_prefill_fused(1)
        L.gpt2_tune_gemm_ln_force(-1)
        L.gpt2_tune_prefill_persistent(-1)
        L.gpt2_tune_prefill_lnfold(-1)
        if backend == "int8":
            L.gpt2_quant_free(C.byref(model.q))
            model.q = None
            model.gpu.q = None
    for name, a, b in zip(("blocks", "final_ln", "logits", "kv"), runs[0], runs[1]):
        bad = np.flatnonzero(a != b)
        where = ""
        if bad.size and name == "blocks":
            lyr, rem = np.divmod(bad[0], T * E)
            where = f"first at layer {lyr}, row {rem // E}, column {rem % E}"
        assert bad.size == 0, f"{name}: {bad.size} elements differ; {where}"


def test_prefill_forward_int8(pkg, L, synth, body, model, deq_body):
    ids = synth.token_ids(20, seed=3)
    model.quantize()
    try:
        got = gpu_forward(pkg, L, model, ids, "int8")
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None
    ref = oracle.forward(oracle.fp16_view(deq_body), ids, logits_all=True)
    assert rel_err(got["final_ln"], ref["final_ln"]) <= 1e-2
    assert rel_err(got["logits"], ref["logits"]) <= 1e-2
    assert kl_rows(ref["logits"], got["logits"]).max() < 0.02


def test_last_row_logits(pkg, L, synth, model):
    ids = synth.token_ids(33, seed=4)
    full = gpu_forward(pkg, L, model, ids, "flash", logits_all=True)["logits"]
    last = gpu_forward(pkg, L, model, ids, "flash", logits_all=False)["logits"]
    assert rel_err(last[0], full[-1]) <= 2e-3


def decode_setup(pkg, L, model, ids, backend):
    P = len(ids)
    kv = pkg.KVCache(1024)
    scr = pkg.Scratch(1024)
    d_ids = pkg.Dev.from_numpy(np.asarray(ids, np.int32))
    logits = pkg.Dev(V * 2)
    caps = pkg.GPT2CapsGPU()
    caps.logits, caps.logits_all = logits.ptr, 0
    L.gpt2_prefill_fill_cache(pkg.backend(backend), C.byref(model.gpu), C.byref(kv.kv), d_ids.ptr, P,
                              C.byref(scr.s), C.byref(caps))
    L.gpt2_sync()
    pkg.check("prefill_fill_cache")
    assert kv.kv.len == P
    return kv, scr, logits


@pytest.mark.parametrize("backend", ["gemv", "int8", "flash"])
def test_decode_matches_recompute(pkg, L, synth, model, backend):
    """[EQ]: logits of cached M=1 steps == last-row logits of a full forward over the sequence."""
    if backend == "int8":
        model.quantize()
    try:
        ids = list(synth.token_ids(40, seed=5))
        P = 32
        kv, scr, logits = decode_setup(pkg, L, model, ids[:P], backend)
        be = pkg.backend(backend)
        caps = pkg.Dev(14 * E * 2)
        for pos in range(P, len(ids)):
            L.gpt2_decode_step_cuda(be, C.byref(model.gpu), C.byref(kv.kv), int(ids[pos]), pos, C.byref(scr.s),
                                    logits.ptr, caps.ptr)
            L.gpt2_sync()
            pkg.check("decode step")
            assert kv.kv.len == pos + 1
            got = oracle.f16_to_f32(logits.numpy(np.uint16, (1, V)))
            ref = gpu_forward(pkg, L, model, ids[:pos + 1], backend, logits_all=False)["logits"]
            assert kl_rows(ref, got).max() < 0.02
            assert rel_err(got, ref) <= 1e-2
            assert got.argmax() == ref.argmax()
        scr.free()
        kv.free()
    finally:
        if backend == "int8":
            L.gpt2_quant_free(C.byref(model.q))
            model.q = None
            model.gpu.q = None


def test_decode_vs_oracle(pkg, L, synth, body, model):
    """Decode-only run from position 0 (cache filled entirely by M=1 steps) against the oracle."""
    ids = synth.token_ids(12, seed=6)
    kv = pkg.KVCache(64)
    scr = pkg.Scratch(64)
    logits = pkg.Dev(V * 2)
    be = pkg.backend("gemv")
    try:
        for pos, tok in enumerate(ids):
            L.gpt2_decode_step_cuda(be, C.byref(model.gpu), C.byref(kv.kv), int(tok), pos, C.byref(scr.s),
                                    logits.ptr, None)
        L.gpt2_sync()
        pkg.check("decode")
        got = oracle.f16_to_f32(logits.numpy(np.uint16, (1, V)))
        ref = oracle.forward(oracle.fp16_view(body), ids, logits_all=False)["logits"]
        assert rel_err(got, ref) <= 1e-2
        assert kl_rows(ref, got).max() < 0.02
    finally:
        scr.free()
        kv.free()


def test_decode_rejects_bad_position(pkg, L, model):
    kv = pkg.KVCache(8)
    scr = pkg.Scratch(8)
    logits = pkg.Dev(V * 2)
    L.gpt2_last_error()
    try:
        L.gpt2_decode_step_cuda(pkg.backend("gemv"), C.byref(model.gpu), C.byref(kv.kv), 5, 3, C.byref(scr.s),
                                logits.ptr, None)   # pos 3 > kv.len 0
        assert L.gpt2_last_error() != 0
        assert kv.kv.len == 0
    finally:
        scr.free()
        kv.free()


def eager_greedy(pkg, L, model, kv, scr, logits, backend, first, P, n):
    be = pkg.backend(backend)
    toks, tok = [], first
    rows = []
    for i in range(n):
        L.gpt2_decode_step_cuda(be, C.byref(model.gpu), C.byref(kv.kv), int(tok), P + i, C.byref(scr.s),
                                logits.ptr, None)
        lg = logits.numpy(np.uint16, (V,))
        rows.append(lg)
        tok = int(np.argmax(oracle.f16_to_f32(lg)))   # numpy argmax keeps the first maximum
        toks.append(tok)
    pkg.check("eager greedy")
    return toks, rows


@pytest.mark.parametrize("backend", ["int8", "gemv"])
def test_graph_decode_matches_eager(pkg, L, synth, model, backend):
    if backend == "int8":
        model.quantize()
    try:
        ids = synth.token_ids(48, seed=8)
        P, n = len(ids), 24
        kv, scr, logits = decode_setup(pkg, L, model, ids, backend)
        first = int(np.argmax(oracle.f16_to_f32(logits.numpy(np.uint16, (V,)))))
        eager_toks, eager_rows = eager_greedy(pkg, L, model, kv, scr, logits, backend, first, P, n)
        # graph: same cache prefix (positions >= P are rewritten by the replays)
        kv.kv.len = P
        tokens = pkg.Dev(1024 * 4)
        g = L.gpt2_decode_graph_create_mode(pkg.backend(backend), C.byref(model.gpu), C.byref(kv.kv),
                                            C.byref(scr.s), logits.ptr, tokens.ptr, pkg.DECODE_MULTI)
        assert g, pkg.check("graph create")
        try:
            assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_MULTI
            assert L.gpt2_decode_graph_set(g, first, P) == 0
            # replay one step at a time, with unrelated eager work and syncs between replays
            junk_a, junk_c = pkg.Dev(64 * 768 * 2), pkg.Dev(64 * 2304 * 2)
            for i in range(n):
                assert L.gpt2_decode_graph_run(g, 1) == 0
                L.gpt2_matmul_tiled(junk_c.ptr, junk_a.ptr, model.gpu.layers[0].qkv_w, None, 64, 2304, 768)
                tok, pos = C.c_int(), C.c_int()
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0
                assert pos.value == P + i + 1
                assert tok.value == eager_toks[i], i
                assert np.array_equal(logits.numpy(np.uint16, (V,)), eager_rows[i]), i
            toks = tokens.numpy(np.int32, (1024,))
            assert list(toks[P + 1:P + 1 + n]) == eager_toks
            # back-to-back replays from the same start reproduce the run
            assert L.gpt2_decode_graph_set(g, first, P) == 0
            assert L.gpt2_decode_graph_run(g, n) == 0
            assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0
            assert pos.value == P + n and tok.value == eager_toks[-1]
            assert kv.kv.len == P + n
            # replays past the cache are refused
            assert L.gpt2_decode_graph_run(g, 1024) != 0
            L.gpt2_last_error()
        finally:
            L.gpt2_decode_graph_destroy(g)
        pkg.check("graph")
        scr.free()
        kv.free()
    finally:
        if backend == "int8":
            L.gpt2_quant_free(C.byref(model.q))
            model.q = None
            model.gpu.q = None


def first_argmax(lg16):
    """Greedy token as the step defines it: the lowest index among the maxima of the fp16 logits."""
    return int(np.argmax(oracle.f16_to_f32(lg16)))


@pytest.mark.parametrize("backend", ["int8", "gemv"])
def test_persistent_decode_matches_eager(pkg, L, synth, model, backend):
    """One-kernel-per-token decode against the eager multi-kernel step, teacher-forced: before every
    replay the graph state is set to the eager run's (token, pos), so each step starts from the same
    cache prefix and input token.  Gates: rel_err <= 1e-2 and KL < 2e-3 per step against the eager
    logits; the step's own greedy token equals the first argmax of its own logits exactly."""
    if backend == "int8":
        model.quantize()
    try:
        ids = synth.token_ids(40, seed=18)
        P, n = len(ids), 20
        kv, scr, logits = decode_setup(pkg, L, model, ids, backend)
        first = first_argmax(logits.numpy(np.uint16, (V,)))
        eager_toks, eager_rows = eager_greedy(pkg, L, model, kv, scr, logits, backend, first, P, n)
        feed = [first] + eager_toks[:-1]
        kv.kv.len = P
        tokens = pkg.Dev(1024 * 4)
        g = L.gpt2_decode_graph_create_mode(pkg.backend(backend), C.byref(model.gpu), C.byref(kv.kv),
                                            C.byref(scr.s), logits.ptr, tokens.ptr, pkg.DECODE_PERSISTENT)
        assert g, pkg.check("graph create")
        try:
            assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_PERSISTENT
            tok, pos = C.c_int(), C.c_int()
            for i in range(n):
                assert L.gpt2_decode_graph_set(g, feed[i], P + i) == 0
                assert L.gpt2_decode_graph_run(g, 1) == 0
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check("persistent step")
                assert pos.value == P + i + 1
                lg = logits.numpy(np.uint16, (V,))
                got, ref = oracle.f16_to_f32(lg)[None], oracle.f16_to_f32(eager_rows[i])[None]
                assert rel_err(got, ref) <= 1e-2, (i, rel_err(got, ref))
                assert kl_rows(ref, got).max() < 2e-3, i
                assert tok.value == first_argmax(lg), i
                assert tokens.numpy(np.int32, (1024,))[P + i + 1] == tok.value
            assert kv.kv.len == P + n
        finally:
            L.gpt2_decode_graph_destroy(g)
        pkg.check("persistent graph")
        scr.free()
        kv.free()
    finally:
        if backend == "int8":
            L.gpt2_quant_free(C.byref(model.q))
            model.q = None
            model.gpu.q = None


def test_persistent_decode_deterministic_free_run(pkg, L, synth, model):
    """Two free-running greedy replays of the persistent step from the same state produce the same
    tokens and the same final logits bit for bit (fixed reduction orders, no atomics in the math),
    and a replay re-pinned to an already used position is not confused by the previous epoch."""
    model.quantize()
    try:
        ids = synth.token_ids(32, seed=19)
        P, n = len(ids), 16
        kv, scr, logits = decode_setup(pkg, L, model, ids, "int8")
        first = first_argmax(logits.numpy(np.uint16, (V,)))
        tokens = pkg.Dev(1024 * 4)
        g = L.gpt2_decode_graph_create_mode(pkg.backend("int8"), C.byref(model.gpu), C.byref(kv.kv),
                                            C.byref(scr.s), logits.ptr, tokens.ptr, pkg.DECODE_PERSISTENT)
        assert g, pkg.check("graph create")
        try:
            runs = []
            for _ in range(2):
                tok, pos = C.c_int(), C.c_int()
                assert L.gpt2_decode_graph_set(g, first, P) == 0
                assert L.gpt2_decode_graph_run(g, n) == 0
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check("free run")
                assert pos.value == P + n
                runs.append((list(tokens.numpy(np.int32, (1024,))[P + 1:P + n + 1]), logits.numpy(np.uint16, (V,))))
            assert runs[0][0] == runs[1][0]
            assert np.array_equal(runs[0][1], runs[1][1])
            assert runs[0][0][-1] == first_argmax(runs[0][1])
        finally:
            L.gpt2_decode_graph_destroy(g)
        scr.free()
        kv.free()
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None


def test_persistent_decode_holds_change_timing_not_bits(pkg, L, synth, model):
    """The poll hold-offs (gpt2_tune_decode_holds) only delay polls: graphs built with none (0 / 0 / 0),
    the defaults and long ones (10 us each) give the same greedy tokens and the same final logits bit
    for bit over a 12-step free run."""
    model.quantize()
    try:
        ids = synth.token_ids(24, seed=23)
        P, n = len(ids), 12
        kv, scr, logits = decode_setup(pkg, L, model, ids, "int8")
        first = first_argmax(logits.numpy(np.uint16, (V,)))
        tokens = pkg.Dev(1024 * 4)
        runs = []
        for holds in ((-1, -1, -1), (0, 0, 0), (1000, 1000, 1000)):
            L.gpt2_tune_decode_holds(*holds)
            try:
                g = L.gpt2_decode_graph_create_mode(pkg.backend("int8"), C.byref(model.gpu), C.byref(kv.kv),
                                                    C.byref(scr.s), logits.ptr, tokens.ptr, pkg.DECODE_PERSISTENT)
            finally:
                L.gpt2_tune_decode_holds(-1, -1, -1)
            assert g, pkg.check("graph create")
            try:
                tok, pos = C.c_int(), C.c_int()
                assert L.gpt2_decode_graph_set(g, first, P) == 0
                assert L.gpt2_decode_graph_run(g, n) == 0
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check(f"holds {holds}")
                assert pos.value == P + n
                runs.append((list(tokens.numpy(np.int32, (1024,))[P + 1:P + n + 1]), logits.numpy(np.uint16, (V,))))
            finally:
                L.gpt2_decode_graph_destroy(g)
        for r in runs[1:]:
            assert r[0] == runs[0][0]
            assert np.array_equal(r[1], runs[0][1])
        scr.free()
        kv.free()
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None


def test_persistent_decode_positions(pkg, L, synth, model):
    """Key-split edge cases of the persistent step: position 0 (no earlier keys, every split empty),
    small contexts where some splits or waves get no keys, splits that do not divide evenly, and the
    last slots of a full 1024-row cache (each attention wave then holds 64 keys, its register
    capacity).  Each position is teacher-forced against the eager step on the same cache prefix (a
    1023-token prefill); gates as in test_persistent_decode_matches_eager."""
    model.quantize()
    try:
        ids = synth.token_ids(1023, seed=23)
        kv, scr, logits = decode_setup(pkg, L, model, ids, "int8")
        be = pkg.backend("int8")
        tokens = pkg.Dev(1024 * 4)
        g = L.gpt2_decode_graph_create_mode(be, C.byref(model.gpu), C.byref(kv.kv), C.byref(scr.s), logits.ptr,
                                            tokens.ptr, pkg.DECODE_PERSISTENT)
        assert g, pkg.check("graph create")
        try:
            assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_PERSISTENT
            tok, pos = C.c_int(), C.c_int()
            for p in (0, 1, 2, 3, 4, 5, 7, 8, 9, 13, 63, 64, 65, 255, 256, 257, 511, 777, 1000, 1021, 1022, 1023):
                tok_in = int(ids[p]) if p < len(ids) else 17
                kv.kv.len = len(ids)
                L.gpt2_decode_step_cuda(be, C.byref(model.gpu), C.byref(kv.kv), tok_in, p, C.byref(scr.s),
                                        logits.ptr, None)
                pkg.check("eager step")
                ref16 = logits.numpy(np.uint16, (V,)).copy()
                assert L.gpt2_decode_graph_set(g, tok_in, p) == 0
                assert L.gpt2_decode_graph_run(g, 1) == 0
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check("persistent step")
                assert pos.value == p + 1
                lg = logits.numpy(np.uint16, (V,))
                got, ref = oracle.f16_to_f32(lg)[None], oracle.f16_to_f32(ref16)[None]
                assert rel_err(got, ref) <= 1e-2, (p, rel_err(got, ref))
                assert kl_rows(ref, got).max() < 2e-3, p
                assert tok.value == first_argmax(lg), p
        finally:
            L.gpt2_decode_graph_destroy(g)
        scr.free()
        kv.free()
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None


def test_persistent_decode_falls_back_without_gemv(pkg, L, synth, model):
    """Backends without this library's GEMV slots (flash: M=1 matmul fallback) get the multi-kernel
    step even when the persistent one is requested."""
    ids = synth.token_ids(8, seed=20)
    kv, scr, logits = decode_setup(pkg, L, model, ids, "flash")
    tokens = pkg.Dev(1024 * 4)
    g = L.gpt2_decode_graph_create_mode(pkg.backend("flash"), C.byref(model.gpu), C.byref(kv.kv), C.byref(scr.s),
                                        logits.ptr, tokens.ptr, pkg.DECODE_PERSISTENT)
    assert g, pkg.check("graph create")
    try:
        assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_MULTI
    finally:
        L.gpt2_decode_graph_destroy(g)
    scr.free()
    kv.free()


def test_persistent_decode_timeout_is_reported(pkg, L, synth, model):
    """Error path forced from the host: with a zero-round poll limit a work-group gives up at the
    first exchange word that has not arrived yet, every work-group still exits, and the sync call
    reports the failure instead of returning a token.  The same graph then recovers: with the default
    limit restored, gpt2_decode_graph_set clears the error word and moves to a new epoch, so the words
    the aborted step left behind cannot satisfy a poll, and the next step matches the eager step."""
    ids = synth.token_ids(8, seed=21)
    kv, scr, logits = decode_setup(pkg, L, model, ids, "gemv")
    be = pkg.backend("gemv")
    tokens = pkg.Dev(1024 * 4)
    L.gpt2_tune_decode_spin(0)
    try:
        g = L.gpt2_decode_graph_create_mode(be, C.byref(model.gpu), C.byref(kv.kv),
                                            C.byref(scr.s), logits.ptr, tokens.ptr, pkg.DECODE_PERSISTENT)
        assert g, pkg.check("graph create")
        try:
            assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_PERSISTENT
            tok, pos = C.c_int(), C.c_int()
            assert L.gpt2_decode_graph_set(g, 5, len(ids)) == 0
            assert L.gpt2_decode_graph_run(g, 1) == 0
            assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) != 0
            assert L.gpt2_last_error() != 0
            L.gpt2_tune_decode_spin(-1)
            # the eager step at the same position, then the recovered persistent step
            kv.kv.len = len(ids)
            L.gpt2_decode_step_cuda(be, C.byref(model.gpu), C.byref(kv.kv), 5, len(ids), C.byref(scr.s),
                                    logits.ptr, None)
            pkg.check("eager step")
            ref16 = logits.numpy(np.uint16, (V,)).copy()
            assert L.gpt2_decode_graph_set(g, 5, len(ids)) == 0
            assert L.gpt2_decode_graph_run(g, 1) == 0
            assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check("recovered step")
            assert pos.value == len(ids) + 1
            lg = logits.numpy(np.uint16, (V,))
            got, ref = oracle.f16_to_f32(lg)[None], oracle.f16_to_f32(ref16)[None]
            assert rel_err(got, ref) <= 1e-2
            assert kl_rows(ref, got).max() < 2e-3
            assert tok.value == first_argmax(lg)
        finally:
            L.gpt2_decode_graph_destroy(g)
    finally:
        L.gpt2_tune_decode_spin(-1)
    L.gpt2_last_error()
    scr.free()
    kv.free()


# ------------------------------------------------------------------ config 5 at full scale
@pytest.fixture(scope="module")
def int8_ref_body(synth, body):
    """The oracle's view of the INT8 model: every tensor as the fp16 engine holds it, and each trunk
    matrix replaced by its dequantized weights fl32(q*s) (tools/dequant_check.py:61-65), not rounded
    again; the tied head stays fp16 (the reference's default INT8 build)."""
    out = oracle.fp16_view(body)
    off = synth.offsets()
    for Lyr in range(12):
        for name in ("qkv_w", "attn_proj_w", "fc_w", "proj_w"):
            o, shape = off[f"h{Lyr}.{name}"]
            n = int(np.prod(shape))
            q, s, _ = oracle.quantize_fp16_view(body[o:o + n].reshape(shape))
            out[o:o + n] = oracle.dequantize(q, s).reshape(-1)
    return out


def test_config5_prefill_p512_vs_oracle(pkg, L, synth, model, int8_ref_body):
    """BASELINE config 5's prefill at full size against the fp32 oracle, the reference's gate (a)/(c)
    (bench/correctness_cuda.cu:200-219): P=512 random ids through the INT8 trunk (48 matrices, the
    fused prefill) and the fp16 tied head, every layer's residual stream rel_err <= 1e-2, the final
    LayerNorm and all 512 logits rows rel_err <= 1e-2, max KL < 0.02 over the rows."""
    ids = synth.token_ids(512, seed=512)
    model.quantize()
    try:
        got = gpu_forward(pkg, L, model, ids, "int8", logits_all=True, want_blocks=True)
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None
    ref = oracle.forward(int8_ref_body, ids, logits_all=True, want_blocks=True)
    for Lyr in range(12):
        assert rel_err(got["blocks"][Lyr], ref["blocks"][Lyr]) <= 1e-2, Lyr
    assert rel_err(got["final_ln"], ref["final_ln"]) <= 1e-2
    assert rel_err(got["logits"], ref["logits"]) <= 1e-2
    assert kl_rows(ref["logits"], got["logits"]).max() < 0.02


def test_config5_decode_512_steps_vs_oracle(pkg, L, synth, model, int8_ref_body):
    """BASELINE config 5's decode at full depth, the reference's deepest cache gate
    (bench/kv_gate.cu:15,190-219): from a 512-token INT8 prefill, 512 consecutive greedy steps of the
    graph-replayed persistent step (positions 512..1023, the device state carrying token and
    position from step to step), each step's logits against the matching row of ONE oracle forward
    over the 1024 tokens the GPU consumed (prompt + its own greedy tokens).  Per position: rel_err
    <= 1e-2 and KL < 0.02; the token each step picks is the first argmax of its own logits."""
    P, n = 512, 512
    ids = synth.token_ids(P, seed=5120)
    model.quantize()
    try:
        kv, scr, logits = decode_setup(pkg, L, model, ids, "int8")
        first_row = logits.numpy(np.uint16, (V,)).copy()
        first = first_argmax(first_row)
        tokens = pkg.Dev(1024 * 4)
        g = L.gpt2_decode_graph_create_mode(pkg.backend("int8"), C.byref(model.gpu), C.byref(kv.kv),
                                            C.byref(scr.s), logits.ptr, tokens.ptr, pkg.DECODE_PERSISTENT)
        assert g, pkg.check("graph create")
        rows, toks = [], []
        try:
            assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_PERSISTENT
            assert L.gpt2_decode_graph_set(g, first, P) == 0
            tok, pos = C.c_int(), C.c_int()
            for i in range(n):
                assert L.gpt2_decode_graph_run(g, 1) == 0
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check(f"step {i}")
                assert pos.value == P + i + 1
                lg = logits.numpy(np.uint16, (V,))
                rows.append(lg)
                assert tok.value == first_argmax(lg), i
                toks.append(tok.value)
        finally:
            L.gpt2_decode_graph_destroy(g)
        scr.free()
        kv.free()
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None
    seq = np.concatenate([ids, [first], toks[:-1]]).astype(np.int32)
    assert seq.size == P + n == 1024
    ref = oracle.forward(int8_ref_body, seq, logits_all=True)["logits"]
    got = oracle.f16_to_f32(np.stack(rows))
    # step i ran at position P + i and predicts the token after seq[P + i]: oracle row P + i
    refr = ref[P:P + n]
    per_rel = [rel_err(got[i], refr[i]) for i in range(n)]
    kl = kl_rows(refr, got)
    worst = int(np.argmax(per_rel))
    assert max(per_rel) <= 1e-2, (worst, per_rel[worst])
    assert kl.max() < 0.02, (int(np.argmax(kl)), float(kl.max()))
    # the prefill's last row against the oracle's row P-1
    assert rel_err(oracle.f16_to_f32(first_row)[None], ref[P - 1:P]) <= 1e-2


# ------------------------------------------------------------------ every tensor INT8, the head included
ALL_INT8 = [0] * 49     # tools/quantize.py:92 default --fp16-keep none: wte is quantized too


@pytest.fixture(scope="module")
def deq_head(synth, body):
    """fl32(q*s) of the fp16 view of wte: the tied head as the INT8 build streams it
    (tools/dequant_check.py:61-65); the embedding lookup keeps reading the fp16 wte."""
    o, shape = synth.offsets()["wte"]
    q, s, _ = oracle.quantize_fp16_view(body[o:o + int(np.prod(shape))].reshape(shape))
    return oracle.dequantize(q, s).astype(np.float64)


def oracle_int8_head_logits(int8_ref_body, deq_head, seq):
    """Oracle logits of the all-INT8 model over seq: the oracle forward on the body with every trunk
    matrix dequantized gives the final LayerNorm of every row; the head is that LayerNorm times the
    dequantized wte (no bias, cuda/forward_cuda.cu:111-115), summed in float64."""
    fin = oracle.forward(int8_ref_body, np.asarray(seq, np.int32), logits_all=False)["final_ln"]
    return fin.astype(np.float64) @ deq_head.T


def test_int8_head_persistent_step_vs_eager(pkg, L, synth, model):
    """The persistent step's INT8-head branch (the head rows dequantized in registers) against the
    eager step with the same all-INT8 weights, teacher-forced at positions 0, 1, 63, 511, 1022 and
    1023 of a 1023-token prefill: rel_err <= 1e-2 and KL < 2e-3 per position, and the step's token is
    the first argmax of its own logits."""
    model.quantize(keep=ALL_INT8)
    try:
        assert model.q.wte.q, "head not quantized"
        ids = synth.token_ids(1023, seed=31)
        kv, scr, logits = decode_setup(pkg, L, model, ids, "int8")
        be = pkg.backend("int8")
        tokens = pkg.Dev(1024 * 4)
        g = L.gpt2_decode_graph_create_mode(be, C.byref(model.gpu), C.byref(kv.kv), C.byref(scr.s), logits.ptr,
                                            tokens.ptr, pkg.DECODE_PERSISTENT)
        assert g, pkg.check("graph create")
        try:
            assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_PERSISTENT
            tok, pos = C.c_int(), C.c_int()
            for p in (0, 1, 63, 511, 1022, 1023):
                tok_in = int(ids[p]) if p < len(ids) else 17
                kv.kv.len = len(ids)
                L.gpt2_decode_step_cuda(be, C.byref(model.gpu), C.byref(kv.kv), tok_in, p, C.byref(scr.s),
                                        logits.ptr, None)
                pkg.check("eager step")
                ref16 = logits.numpy(np.uint16, (V,)).copy()
                assert L.gpt2_decode_graph_set(g, tok_in, p) == 0
                assert L.gpt2_decode_graph_run(g, 1) == 0
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check("persistent step")
                assert pos.value == p + 1
                lg = logits.numpy(np.uint16, (V,))
                got, ref = oracle.f16_to_f32(lg)[None], oracle.f16_to_f32(ref16)[None]
                assert rel_err(got, ref) <= 1e-2, (p, rel_err(got, ref))
                assert kl_rows(ref, got).max() < 2e-3, p
                assert tok.value == first_argmax(lg), p
        finally:
            L.gpt2_decode_graph_destroy(g)
        scr.free()
        kv.free()
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None


def test_int8_head_multi_kernel_graph_matches_eager(pkg, L, synth, model):
    """The multi-kernel graph step with the head quantized uses the eager step's kernels in the same
    order: 12 replays match 12 eager steps bit for bit (tokens and logits)."""
    model.quantize(keep=ALL_INT8)
    try:
        ids = synth.token_ids(40, seed=32)
        P, n = len(ids), 12
        kv, scr, logits = decode_setup(pkg, L, model, ids, "int8")
        first = first_argmax(logits.numpy(np.uint16, (V,)))
        eager_toks, eager_rows = eager_greedy(pkg, L, model, kv, scr, logits, "int8", first, P, n)
        kv.kv.len = P
        tokens = pkg.Dev(1024 * 4)
        g = L.gpt2_decode_graph_create_mode(pkg.backend("int8"), C.byref(model.gpu), C.byref(kv.kv),
                                            C.byref(scr.s), logits.ptr, tokens.ptr, pkg.DECODE_MULTI)
        assert g, pkg.check("graph create")
        try:
            assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_MULTI
            assert L.gpt2_decode_graph_set(g, first, P) == 0
            tok, pos = C.c_int(), C.c_int()
            for i in range(n):
                assert L.gpt2_decode_graph_run(g, 1) == 0
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check("graph step")
                assert tok.value == eager_toks[i], i
                assert np.array_equal(logits.numpy(np.uint16, (V,)), eager_rows[i]), i
        finally:
            L.gpt2_decode_graph_destroy(g)
        scr.free()
        kv.free()
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None


def test_int8_head_prefill_and_decode_vs_oracle(pkg, L, synth, model, int8_ref_body, deq_head):
    """All 49 tensors INT8 (the reference quantizer's default): a P=64 prefill with logits for every
    row, then 16 free-running greedy replays of the persistent step, against the oracle on the body
    with every tensor dequantized, the head included.  Gates: rel_err <= 1e-2 per row and per step,
    KL < 0.02; each step's token is the first argmax of its own logits."""
    P, n = 64, 16
    ids = synth.token_ids(P, seed=640)
    model.quantize(keep=ALL_INT8)
    try:
        got_pre = gpu_forward(pkg, L, model, ids, "int8", logits_all=True)["logits"]
        kv, scr, logits = decode_setup(pkg, L, model, ids, "int8")
        first = first_argmax(logits.numpy(np.uint16, (V,)))
        tokens = pkg.Dev(1024 * 4)
        g = L.gpt2_decode_graph_create_mode(pkg.backend("int8"), C.byref(model.gpu), C.byref(kv.kv),
                                            C.byref(scr.s), logits.ptr, tokens.ptr, pkg.DECODE_AUTO)
        assert g, pkg.check("graph create")
        rows, toks = [], []
        try:
            assert L.gpt2_decode_graph_mode(g) == pkg.DECODE_PERSISTENT
            assert L.gpt2_decode_graph_set(g, first, P) == 0
            tok, pos = C.c_int(), C.c_int()
            for i in range(n):
                assert L.gpt2_decode_graph_run(g, 1) == 0
                assert L.gpt2_decode_graph_sync(g, C.byref(tok), C.byref(pos)) == 0, pkg.check(f"step {i}")
                lg = logits.numpy(np.uint16, (V,))
                rows.append(lg)
                assert tok.value == first_argmax(lg), i
                toks.append(tok.value)
        finally:
            L.gpt2_decode_graph_destroy(g)
        scr.free()
        kv.free()
    finally:
        L.gpt2_quant_free(C.byref(model.q))
        model.q = None
        model.gpu.q = None
    seq = np.concatenate([ids, [first], toks[:-1]]).astype(np.int32)
    ref = oracle_int8_head_logits(int8_ref_body, deq_head, seq)
    assert rel_err(got_pre, ref[:P]) <= 1e-2
    assert kl_rows(ref[:P], got_pre).max() < 0.02
    assert first == int(np.argmax(got_pre[-1]))
    got = oracle.f16_to_f32(np.stack(rows))
    refr = ref[P:P + n]
    per_rel = [rel_err(got[i], refr[i]) for i in range(n)]
    assert max(per_rel) <= 1e-2, per_rel
    assert kl_rows(refr, got).max() < 0.02
