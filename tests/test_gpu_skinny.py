"""The skinny GEMM (csrc/gemm_skinny.hip): gpt2_matmul_tiled / gpt2_matmul_int8 with a few rows of A
(M in [2, gpt2_tune_gemm_skinny_max(qw)], the GPT-2 trunk shapes K = 768 / 3072) take it instead of the
tile pipeline (the same contract, cuda/kernels_tiled.cu:24-53, cuda/kernels_quant.cu:38-67).  The
tests below set the limit to 64 for both weight formats (the default is 64 for INT8, 32 for fp16).

Bars: against the CPU oracle on the same fp16-valued inputs (INT8: on the dequantized weights), the
GEMM bar (max abs <= 2e-2, rel-L2 <= 1e-3); rows of C past M are left as they were; the fused gelu
and residual epilogues bit for bit against the skinny product followed by gpt2_gelu / gpt2_add (the
prefill's fused == unfused identity); the launch counter shows which calls took it (M = 1 is the
GEMV, larger M, forced tile configs, other K or N % 16 != 0 keep their paths).  Its LayerNorm
prologue is covered through the whole prefill in tests/test_gpu_model.py
(test_fused_prefill_bit_identical at T <= 32 fp16, <= 64 INT8)."""
import numpy as np
import pytest

import oracle
from conftest import tol_check

pytestmark = pytest.mark.gpu

SHAPES = {"qkv": (2304, 768), "attn_proj": (768, 768), "fc": (3072, 768), "mlp_proj": (768, 3072)}
NAN16 = 0x7E00


@pytest.fixture(autouse=True)
def limit64(L):
    L.gpt2_tune_gemm_skinny(64)
    yield
    L.gpt2_tune_gemm_skinny(-1)


def f16v(rng, shape, std):
    return oracle.fp16_view(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def dev16(pkg, x):
    return pkg.Dev.from_numpy(oracle.f32_to_f16(x))


def weights(pkg, rng, kind, N, K):
    """Device weights and their dequantized fp32 values (INT8: the reference quantizer's scheme)."""
    if kind == "int8":
        q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        return (pkg.Dev.from_numpy(q), pkg.Dev.from_numpy(s)), oracle.dequantize(q, s)
    W = f16v(rng, (N, K), 0.02)
    return (dev16(pkg, W), None), W


def matmul(L, kind, dC, dA, dW, b, M, N, K):
    W, s = dW
    if kind == "int8":
        L.gpt2_matmul_int8(dC.ptr, dA.ptr, W.ptr, s.ptr, b.ptr if b is not None else None, M, N, K)
    else:
        L.gpt2_matmul_tiled(dC.ptr, dA.ptr, W.ptr, b.ptr if b is not None else None, M, N, K)


@pytest.mark.parametrize("kind", ["fp16", "int8"])
@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("M", [2, 5, 16, 17, 40, 64])
def test_skinny_vs_oracle(pkg, L, kind, shape, M):
    """Every trunk shape at M from 2 to the limit (one partial 16-row block, several; odd M without a
    bias): the oracle's result within the GEMM bar, the skinny kernel launched once, and the 16 rows
    of C past M untouched."""
    N, K = SHAPES[shape]
    rng = np.random.default_rng(M * 31 + N + K)
    A, b = f16v(rng, (M, K), 1.0), (f16v(rng, N, 0.01) if M % 2 == 0 else None)
    dW, Wd = weights(pkg, rng, kind, N, K)
    dA, db = dev16(pkg, A), (dev16(pkg, b) if b is not None else None)
    dC = pkg.Dev.from_numpy(np.full((M + 16) * N, NAN16, np.uint16))
    before = L.gpt2_tune_gemm_skinny_calls()
    matmul(L, kind, dC, dA, dW, db, M, N, K)
    L.gpt2_sync()
    pkg.check("skinny gemm")
    assert L.gpt2_tune_gemm_skinny_calls() == before + 1
    out = dC.numpy(np.uint16, (M + 16, N))
    assert np.all(out[M:] == NAN16), "rows past M were written"
    tol_check(oracle.f16_to_f32(out[:M]), oracle.matmul(A, Wd, b))


@pytest.mark.parametrize("kind", ["fp16", "int8"])
@pytest.mark.parametrize("shape,M", [("fc", 16), ("qkv", 33), ("attn_proj", 7), ("mlp_proj", 64), ("mlp_proj", 2)])
def test_skinny_epilogues_bit_exact(pkg, L, kind, shape, M):
    """gelu and the residual add fused into the skinny GEMM (gpt2_tune_gemm_fused, as the prefill
    calls it) equal the plain skinny GEMM followed by gpt2_gelu / gpt2_add bit for bit; the residual
    both in place (C += product) and from another buffer; and both sides within the oracle's bar."""
    N, K = SHAPES[shape]
    rng = np.random.default_rng(M * 17 + N)
    A, b, R = f16v(rng, (M, K), 1.0), f16v(rng, N, 0.01), f16v(rng, (M, N), 1.0)
    dW, Wd = weights(pkg, rng, kind, N, K)
    W, s = dW
    dA, db = dev16(pkg, A), dev16(pkg, b)
    plain = pkg.Dev(M * N * 2)
    matmul(L, kind, plain, dA, dW, db, M, N, K)
    L.gpt2_sync()
    base = plain.numpy(np.uint16, (M, N))
    # unfused references on the device: gelu in place on a copy, and R + product
    ref_gelu = dev16(pkg, oracle.f16_to_f32(base))
    L.gpt2_gelu(ref_gelu.ptr, M * N)
    ref_add = dev16(pkg, R)
    L.gpt2_add(ref_add.ptr, plain.ptr, M * N)
    L.gpt2_sync()
    pkg.check("unfused")
    want = {1: ref_gelu.numpy(np.uint16, (M, N)), 2: ref_add.numpy(np.uint16, (M, N))}
    for epi in (1, 2):
        for in_place in ((False, True) if epi == 2 else (False,)):
            dC = dev16(pkg, R) if in_place else pkg.Dev(M * N * 2)
            dR = dC if in_place else dev16(pkg, R)
            before = L.gpt2_tune_gemm_skinny_calls()
            ran = L.gpt2_tune_gemm_fused(dC.ptr, dA.ptr, W.ptr, s.ptr if s is not None else None, db.ptr, M, N, K,
                                         epi, dR.ptr if epi == 2 else None)
            L.gpt2_sync()
            pkg.check("fused skinny")
            assert ran == 1 and L.gpt2_tune_gemm_skinny_calls() == before + 1, (epi, in_place)
            got = dC.numpy(np.uint16, (M, N))
            assert np.array_equal(got, want[epi]), (kind, shape, M, epi, in_place)
    ref = oracle.fp16_view(oracle.matmul(A, Wd, b))
    tol_check(oracle.f16_to_f32(want[1]), oracle.fp16_view(oracle.gelu(ref)))
    tol_check(oracle.f16_to_f32(want[2]), oracle.fp16_view(R + ref))


def test_skinny_domain(pkg, L):
    """Which calls take it: M in [2, limit] at the trunk shapes; not M = 1 (the GEMV), M above the
    limit, K outside {768, 3072}, N % 16 != 0, a forced tile config, or the limit set to 0; and the
    results of the calls it declines still meet the oracle's bar."""
    rng = np.random.default_rng(99)
    lim = L.gpt2_tune_gemm_skinny_max(0)
    assert lim == 64

    def run(M, N, K, expect):
        A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.02), f16v(rng, N, 0.01)
        dA, dW, db, dC = dev16(pkg, A), dev16(pkg, W), dev16(pkg, b), pkg.Dev(M * N * 2)
        before = L.gpt2_tune_gemm_skinny_calls()
        L.gpt2_matmul_tiled(dC.ptr, dA.ptr, dW.ptr, db.ptr, M, N, K)
        L.gpt2_sync()
        pkg.check("domain")
        assert L.gpt2_tune_gemm_skinny_calls() - before == expect, (M, N, K)
        tol_check(oracle.f16_to_f32(dC.numpy(np.uint16, (M, N))), oracle.matmul(A, W, b))

    run(8, 768, 768, 1)
    run(1, 768, 768, 0)
    run(lim + 1, 768, 768, 0)
    run(8, 768, 1536, 0)
    run(8, 760, 768, 0)
    L.gpt2_tune_gemm_force(8)
    try:
        run(8, 768, 768, 0)
    finally:
        L.gpt2_tune_gemm_force(-1)
    L.gpt2_tune_gemm_skinny(0)
    try:
        run(8, 768, 768, 0)
    finally:
        L.gpt2_tune_gemm_skinny(lim)
    run(8, 768, 768, 1)
    # the defaults: INT8 up to 64 rows, fp16 up to 32
    L.gpt2_tune_gemm_skinny(-1)
    assert (L.gpt2_tune_gemm_skinny_max(0), L.gpt2_tune_gemm_skinny_max(1)) == (32, 64)
    run(32, 768, 768, 1)
    run(33, 768, 768, 0)


def test_skinny_repeatable(pkg, L):
    """Deterministic: the same call twice gives the same bits (fixed wave order in the k-split sum)."""
    rng = np.random.default_rng(7)
    M, N, K = 24, 768, 3072
    A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.02), f16v(rng, N, 0.01)
    dA, dW, db = dev16(pkg, A), dev16(pkg, W), dev16(pkg, b)
    outs = []
    for _ in range(2):
        dC = pkg.Dev(M * N * 2)
        L.gpt2_matmul_tiled(dC.ptr, dA.ptr, dW.ptr, db.ptr, M, N, K)
        L.gpt2_sync()
        outs.append(dC.numpy(np.uint16, (M, N)))
    pkg.check("repeat")
    assert np.array_equal(outs[0], outs[1])
