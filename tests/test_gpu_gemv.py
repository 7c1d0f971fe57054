"""M=1 GEMV parity: gpt2_gemv_fp16 / gpt2_gemv_int8 / gpt2_gemv_dispatch against the CPU oracle.

Bar: max abs <= 2e-2 and rel-L2 <= 1e-3 against the double-accumulated matmul of the same inputs
(INT8: of the dequantized weights fl32(q*s)).  Shapes: BASELINE configs 3 and 4 (K x N in
{768x2304, 768x768, 768x3072, 3072x768}, and the tied head 768x50257 with its odd-N tail).
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from conftest import tol_check

pytestmark = pytest.mark.gpu

TRUNK = [(2304, 768), (768, 768), (3072, 768), (768, 3072)]   # (N, K)


def f16v(rng, shape, std):
    return oracle.fp16_view(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def dev16(pkg, x):
    return pkg.Dev.from_numpy(oracle.f32_to_f16(x))


def run(pkg, L, x, W=None, q=None, s=None, b=None, cfg=None):
    K = x.shape[-1]
    N = W.shape[0] if W is not None else q.shape[0]
    dx = dev16(pkg, x.reshape(1, K))
    db = dev16(pkg, b) if b is not None else None
    dy = pkg.Dev(max(1, N) * 2)
    bp = db.ptr if db is not None else None
    if q is not None:
        dq, ds = pkg.Dev.from_numpy(q), pkg.Dev.from_numpy(s)
        if cfg is None:
            L.gpt2_gemv_int8(dy.ptr, dx.ptr, dq.ptr, ds.ptr, bp, N, K)
        else:
            L.gpt2_tune_gemv_run(cfg, dy.ptr, dx.ptr, dq.ptr, ds.ptr, bp, N, K)
    else:
        dW = dev16(pkg, W)
        if cfg is None:
            L.gpt2_gemv_fp16(dy.ptr, dx.ptr, dW.ptr, bp, N, K)
        else:
            L.gpt2_tune_gemv_run(cfg, dy.ptr, dx.ptr, dW.ptr, None, bp, N, K)
    L.gpt2_sync()
    pkg.check("gemv")
    return oracle.f16_to_f32(dy.numpy(np.uint16, (1, N)))


@pytest.mark.parametrize("N,K", TRUNK)
def test_int8_trunk_shapes(pkg, L, N, K):
    rng = np.random.default_rng(N + 3 * K)
    x, b = f16v(rng, (1, K), 1.0), f16v(rng, N, 0.01)
    q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    ref = oracle.matmul(x, oracle.dequantize(q, s), b)
    tol_check(run(pkg, L, x, q=q, s=s, b=b), ref)
    tol_check(run(pkg, L, x, q=q, s=s), oracle.matmul(x, oracle.dequantize(q, s)))


@pytest.mark.parametrize("N,K", TRUNK)
def test_fp16_trunk_shapes(pkg, L, N, K):
    rng = np.random.default_rng(N * 5 + K)
    x, W, b = f16v(rng, (1, K), 1.0), f16v(rng, (N, K), 0.02), f16v(rng, N, 0.01)
    tol_check(run(pkg, L, x, W=W, b=b), oracle.matmul(x, W, b))


def test_fp16_head_gemv_tail(pkg, L):
    """Tied head: N = 50257, K = 768, no bias; the last 81 rows are the 128-row tail."""
    rng = np.random.default_rng(21)
    K, N = 768, 50257
    x = oracle.fp16_view(oracle.layernorm(rng.standard_normal((1, K), dtype=np.float32),
                                          np.ones(K, np.float32), np.zeros(K, np.float32)))
    W = f16v(rng, (N, K), 0.02)
    got = run(pkg, L, x, W=W)
    ref = oracle.matmul(x, W)
    tol_check(got, ref)
    tol_check(got[:, 50176:], ref[:, 50176:])


def test_int8_head_gemv(pkg, L):
    rng = np.random.default_rng(22)
    K, N = 768, 50257
    x = f16v(rng, (1, K), 1.0)
    q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    tol_check(run(pkg, L, x, q=q, s=s), oracle.matmul(x, oracle.dequantize(q, s)))


@pytest.mark.parametrize("N", [1, 2, 3, 5, 17, 63, 64, 65, 81, 255, 257])
def test_ragged_n(pkg, L, N):
    rng = np.random.default_rng(N)
    K = 768
    x, W, b = f16v(rng, (1, K), 1.0), f16v(rng, (N, K), 0.05), f16v(rng, N, 0.01)
    tol_check(run(pkg, L, x, W=W, b=b), oracle.matmul(x, W, b))
    q, s, _ = oracle.quantize_fp16_view(W)
    tol_check(run(pkg, L, x, q=q, s=s, b=b), oracle.matmul(x, oracle.dequantize(q, s), b))


@pytest.mark.parametrize("K", [2, 4, 6, 12, 100, 764, 1000])
def test_generic_k(pkg, L, K):
    """K that no vector kernel covers runs the generic kernel (the reference needs K even / K%4)."""
    rng = np.random.default_rng(K + 1)
    N = 130
    x, W, b = f16v(rng, (1, K), 1.0), f16v(rng, (N, K), 0.05), f16v(rng, N, 0.01)
    tol_check(run(pkg, L, x, W=W, b=b), oracle.matmul(x, W, b))
    q, s, _ = oracle.quantize_fp16_view(W)
    tol_check(run(pkg, L, x, q=q, s=s, b=b), oracle.matmul(x, oracle.dequantize(q, s), b))


def test_every_gemv_config(pkg, L):
    rng = np.random.default_rng(31)
    x768, x3072 = f16v(rng, (1, 768), 1.0), f16v(rng, (1, 3072), 1.0)
    for cfg in range(L.gpt2_tune_gemv_count()):
        name = L.gpt2_tune_gemv_name(cfg).decode()
        for K, x in ((768, x768), (3072, x3072)):
            for qw in (0, 1):
                if not L.gpt2_tune_gemv_fits(cfg, K, qw):
                    continue
                for N in (2304, 77):
                    W = f16v(rng, (N, K), 0.02)
                    b = f16v(rng, N, 0.01)
                    try:
                        if qw:
                            q, s, _ = oracle.quantize_fp16_view(W)
                            tol_check(run(pkg, L, x, q=q, s=s, b=b, cfg=cfg),
                                      oracle.matmul(x, oracle.dequantize(q, s), b))
                        else:
                            tol_check(run(pkg, L, x, W=W, b=b, cfg=cfg), oracle.matmul(x, W, b))
                    except AssertionError as e:
                        raise AssertionError(f"cfg {cfg} {name} N={N} K={K} qw={qw}: {e}")


def test_int8_exact_small_values(pkg, L):
    """x in {-1,0,1}, q small, s a power of two: every sum is exact, so y is bit-exact."""
    rng = np.random.default_rng(33)
    for N, K in TRUNK:
        x = rng.integers(-1, 2, (1, K)).astype(np.float32)
        q = rng.integers(-3, 4, (N, K)).astype(np.int8)
        s = np.full(N, 0.25, np.float32)
        b = rng.integers(-2, 3, N).astype(np.float32)
        got = run(pkg, L, x, q=q, s=s, b=b)
        assert np.array_equal(got, oracle.matmul(x, oracle.dequantize(q, s), b)), (N, K)


def test_gemv_matches_gemm_row(pkg, L):
    """The decode GEMV and the prefill GEMM agree on the same row (M=1 vs row m)."""
    rng = np.random.default_rng(34)
    K, N = 768, 3072
    A, W, b = f16v(rng, (8, K), 1.0), f16v(rng, (N, K), 0.02), f16v(rng, N, 0.01)
    dA, dW, db = dev16(pkg, A), dev16(pkg, W), dev16(pkg, b)
    dC = pkg.Dev(8 * N * 2)
    L.gpt2_matmul_tiled(dC.ptr, dA.ptr, dW.ptr, db.ptr, 8, N, K)
    L.gpt2_sync()
    gemm_rows = oracle.f16_to_f32(dC.numpy(np.uint16, (8, N)))
    got = run(pkg, L, A[5:6], W=W, b=b)
    tol_check(got, gemm_rows[5:6], max_abs=2e-3)


def test_gemv_dispatch(pkg, L):
    """gemv_q if quantized, else gemv, else the backend's M=1 matmul (cuda/kvcache.cu:225-230)."""
    rng = np.random.default_rng(35)
    N, K = 768, 768
    x, b = f16v(rng, (1, K), 1.0), f16v(rng, N, 0.01)
    w32 = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    W = oracle.fp16_view(w32)
    q, s, _ = oracle.quantize_fp16_view(w32)
    dx, dW, db = dev16(pkg, x), dev16(pkg, W), dev16(pkg, b)
    dq, ds = pkg.Dev.from_numpy(q), pkg.Dev.from_numpy(s)
    dy = pkg.Dev(N * 2)
    qw = pkg.GPT2QW(dq.ptr, ds.ptr)
    res = {}
    for be in ("int8", "gemv", "tiled", "naive"):
        L.gpt2_gemv_dispatch(pkg.backend(be), dy.ptr, dx.ptr, dW.ptr, C.byref(qw), db.ptr, N, K)
        L.gpt2_sync()
        res[be] = oracle.f16_to_f32(dy.numpy(np.uint16, (1, N)))
    pkg.check("gemv_dispatch")
    tol_check(res["int8"], oracle.matmul(x, oracle.dequantize(q, s), b))
    for be in ("gemv", "tiled", "naive"):
        tol_check(res[be], oracle.matmul(x, W, b))
