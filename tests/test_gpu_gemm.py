"""Prefill GEMM parity: gpt2_matmul_tiled / gpt2_matmul_int8 / gpt2_matmul_naive against the CPU
oracle (cpu/forward_cpu.c:35-50 restated: double accumulation of the same fp16-valued inputs).

Bar: max |C - C_ref| <= 2e-2 and rel-L2 <= 1e-3; INT8 compared against the
oracle run on the dequantized weights fl32(q*s) (tools/dequant_check.py:65).  Exact cases (one-hot
rows, small integers) must match bit for bit.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from conftest import tol_check

pytestmark = pytest.mark.gpu

CONFIG_SHAPES = [(512, 2304, 768), (512, 768, 768), (512, 3072, 768), (512, 768, 3072)]
RAGGED = [(1, 1, 8), (1, 17, 8), (2, 81, 24), (17, 33, 40), (63, 65, 72), (65, 127, 136), (127, 129, 200),
          (129, 257, 64), (100, 200, 136), (512, 50, 16)]


def f16v(rng, shape, std):
    return oracle.fp16_view(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def dev16(pkg, x):
    return pkg.Dev.from_numpy(oracle.f32_to_f16(x))


def gemm(pkg, L, A, W, b, cfg=None, kind="fp16", q=None, s=None, a_offset=0):
    M, K = A.shape
    N = W.shape[0] if W is not None else q.shape[0]
    if a_offset:
        buf = np.zeros(M * K + a_offset, np.uint16)
        buf[a_offset:] = oracle.f32_to_f16(A).reshape(-1)
        dAbuf = pkg.Dev.from_numpy(buf)
        a_ptr = dAbuf.at(2 * a_offset)
    else:
        dAbuf = dev16(pkg, A)
        a_ptr = dAbuf.ptr
    db = dev16(pkg, b) if b is not None else None
    dC = pkg.Dev(max(1, M * N) * 2)
    bptr = db.ptr if db is not None else None
    if kind == "int8":
        dq, ds = pkg.Dev.from_numpy(q), pkg.Dev.from_numpy(s)
        if cfg is None:
            L.gpt2_matmul_int8(dC.ptr, a_ptr, dq.ptr, ds.ptr, bptr, M, N, K)
        else:
            L.gpt2_tune_gemm_run(cfg, dC.ptr, a_ptr, dq.ptr, ds.ptr, bptr, M, N, K)
    else:
        dW = dev16(pkg, W)
        if kind == "naive":
            L.gpt2_matmul_naive(dC.ptr, a_ptr, dW.ptr, bptr, M, N, K)
        elif cfg is None:
            L.gpt2_matmul_tiled(dC.ptr, a_ptr, dW.ptr, bptr, M, N, K)
        else:
            L.gpt2_tune_gemm_run(cfg, dC.ptr, a_ptr, dW.ptr, None, bptr, M, N, K)
    L.gpt2_sync()
    pkg.check("gemm")
    return oracle.f16_to_f32(dC.numpy(np.uint16, (M, N)))


@pytest.mark.parametrize("M,N,K", CONFIG_SHAPES)
def test_fp16_config_shapes(pkg, L, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.02), f16v(rng, N, 0.01)
    tol_check(gemm(pkg, L, A, W, b), oracle.matmul(A, W, b))


@pytest.mark.parametrize("M,N,K", CONFIG_SHAPES)
def test_int8_config_shapes(pkg, L, M, N, K):
    rng = np.random.default_rng(M + N + K)
    A, b = f16v(rng, (M, K), 1.0), f16v(rng, N, 0.01)
    q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    got = gemm(pkg, L, A, None, b, kind="int8", q=q, s=s)
    tol_check(got, oracle.matmul(A, oracle.dequantize(q, s), b))


TRUNK_NK = [(2304, 768), (768, 768), (3072, 768), (768, 3072)]


@pytest.mark.parametrize("kind", ["fp16", "int8"])
@pytest.mark.parametrize("M", [2, 64, 100, 128, 200, 256, 700, 1024])
def test_trunk_shapes_every_m_bucket(pkg, L, kind, M):
    """The four trunk shapes at prompt lengths in every bucket of the tile table (M <= 64, 128, 256,
    512, 1024), including the longest prefill (M = 1024) and ragged M, against the oracle."""
    for N, K in TRUNK_NK:
        rng = np.random.default_rng(M * 5 + N + K)
        A, b = f16v(rng, (M, K), 1.0), f16v(rng, N, 0.01)
        if kind == "int8":
            q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
            got = gemm(pkg, L, A, None, b, kind="int8", q=q, s=s)
            tol_check(got, oracle.matmul(A, oracle.dequantize(q, s), b))
        else:
            W = f16v(rng, (N, K), 0.02)
            tol_check(gemm(pkg, L, A, W, b), oracle.matmul(A, W, b))


@pytest.mark.parametrize("kind", ["fp16", "int8"])
@pytest.mark.parametrize("M,N,K", [(300, 777, 768), (129, 257, 256), (64, 1001, 192), (512, 2305, 768)])
def test_unaligned_c_rows(pkg, L, kind, M, N, K):
    """Odd N (rows of C not 8-byte aligned) with C itself offset by 0, 1 or 3 elements: the tile is
    staged through LDS and written as dword column pairs plus lone end columns; the elements right
    before and after C must stay untouched."""
    rng = np.random.default_rng(M + N + K)
    A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.02), f16v(rng, N, 0.01)
    q, s, _ = oracle.quantize_fp16_view(W)
    ref = oracle.matmul(A, oracle.dequantize(q, s), b) if kind == "int8" else oracle.matmul(A, W, b)
    dA, db = dev16(pkg, A), dev16(pkg, b)
    dW = pkg.Dev.from_numpy(q) if kind == "int8" else dev16(pkg, W)
    ds = pkg.Dev.from_numpy(s)
    for off in (0, 1, 3):
        sentinel = np.full(M * N + off + 4, 0x7BFF, np.uint16)          # fp16 65504
        dC = pkg.Dev.from_numpy(sentinel)
        cptr = dC.at(2 * off)
        if kind == "int8":
            L.gpt2_matmul_int8(cptr, dA.ptr, dW.ptr, ds.ptr, db.ptr, M, N, K)
        else:
            L.gpt2_matmul_tiled(cptr, dA.ptr, dW.ptr, db.ptr, M, N, K)
        L.gpt2_sync()
        pkg.check("gemm unaligned C")
        out = dC.numpy(np.uint16, (M * N + off + 4,))
        assert (out[:off] == 0x7BFF).all() and (out[off + M * N:] == 0x7BFF).all(), off
        tol_check(oracle.f16_to_f32(out[off:off + M * N].reshape(M, N)), ref)


def test_head_gemm_tail_columns(pkg, L):
    """Tied head at M=512: N = 50257 is odd (rows of C are 100514 B, not 16-B aligned)."""
    rng = np.random.default_rng(4)
    M, N, K = 512, 50257, 768
    x = rng.standard_normal((M, K), dtype=np.float32)
    A = oracle.fp16_view(oracle.layernorm(x, np.ones(K, np.float32), np.zeros(K, np.float32)))
    W = f16v(rng, (N, K), 0.02)
    got = gemm(pkg, L, A, W, None)
    tol_check(got, oracle.matmul(A, W))                      # every row and column
    tail = slice(50176, 50257)
    tol_check(got[:, tail], oracle.matmul(A, W[tail]))       # the 81 tail columns on their own


@pytest.mark.parametrize("M,N,K", RAGGED)
def test_fp16_ragged(pkg, L, M, N, K):
    rng = np.random.default_rng(M * 131 + N * 17 + K)
    A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.05), f16v(rng, N, 0.01)
    tol_check(gemm(pkg, L, A, W, b), oracle.matmul(A, W, b))
    tol_check(gemm(pkg, L, A, W, None), oracle.matmul(A, W))


@pytest.mark.parametrize("M,N,K", [(3, 5, 7), (33, 17, 33), (64, 100, 100), (5, 9, 1)])
def test_generic_path_odd_k(pkg, L, M, N, K):
    rng = np.random.default_rng(K)
    A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.05), f16v(rng, N, 0.01)
    tol_check(gemm(pkg, L, A, W, b), oracle.matmul(A, W, b))


def test_generic_path_unaligned_a(pkg, L):
    rng = np.random.default_rng(9)
    M, N, K = 40, 72, 64
    A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.05), f16v(rng, N, 0.01)
    tol_check(gemm(pkg, L, A, W, b, a_offset=1), oracle.matmul(A, W, b))


def test_every_tile_config(pkg, L):
    """Every tile config on shapes whose K it accepts (K % (64*depth) == 0), ragged M and N, odd N
    (C rows not 8-byte aligned: the staged epilogue), plus shapes no config accepts (the guarded
    kernel)."""
    rng = np.random.default_rng(11)
    for M, N, K in [(100, 200, 136), (512, 768, 768), (7, 300, 768), (77, 130, 3072), (33, 96, 64),
                    (130, 1001, 768)]:
        A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.05), f16v(rng, N, 0.01)
        ref = oracle.matmul(A, W, b)
        q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.05))
        refq = oracle.matmul(A, oracle.dequantize(q, s), b)
        for cfg in range(L.gpt2_tune_gemm_count()):
            name = L.gpt2_tune_gemm_name(cfg).decode()
            if K != 136 and not L.gpt2_tune_gemm_fits(cfg, K):
                continue
            try:
                tol_check(gemm(pkg, L, A, W, b, cfg=cfg), ref)
                tol_check(gemm(pkg, L, A, None, b, cfg=cfg, kind="int8", q=q, s=s), refq)
            except AssertionError as e:
                raise AssertionError(f"cfg {cfg} {name} {M}x{N}x{K}: {e}")


def test_one_hot_rows_exact(pkg, L):
    """A row e_k selects W[:, k]: C[m, n] = fp16(W[n, k] + b[n]) exactly."""
    rng = np.random.default_rng(5)
    M, N, K = 64, 2304, 768
    ks = rng.integers(0, K, M)
    A = np.zeros((M, K), np.float32)
    A[np.arange(M), ks] = 1.0
    W, b = f16v(rng, (N, K), 0.02), f16v(rng, N, 0.01)
    got = gemm(pkg, L, A, W, b)
    ref = oracle.fp16_view(oracle.matmul(A, W, b))
    assert np.array_equal(got, ref)


def test_small_integers_exact(pkg, L):
    """Entries in {-1, 0, 1}: every partial sum is an integer below 2^11, so C is exact."""
    rng = np.random.default_rng(6)
    for M, N, K in [(512, 768, 768), (128, 3072, 768), (64, 768, 3072)]:
        A = rng.integers(-1, 2, (M, K)).astype(np.float32)
        W = rng.integers(-1, 2, (N, K)).astype(np.float32)
        if K > 2048:
            W[:, 2048:] = 0.0   # keep |sum| < 2048 so fp16 C is exact
        got = gemm(pkg, L, A, W, None)
        assert np.array_equal(got, oracle.matmul(A, W)), (M, N, K)


def test_int8_small_integers_exact(pkg, L):
    """q in [-127,127], s = 1, A in {-1,0,1}: exact sums up to 768*127 exceed fp16 range checks, so
    use K = 16 and check bit-exactness of the scale-then-bias epilogue."""
    rng = np.random.default_rng(8)
    M, N, K = 96, 200, 16
    A = rng.integers(-1, 2, (M, K)).astype(np.float32)
    q = rng.integers(-8, 9, (N, K)).astype(np.int8)
    s = np.full(N, 0.5, np.float32)
    b = rng.integers(-4, 5, N).astype(np.float32)
    got = gemm(pkg, L, A, None, b, kind="int8", q=q, s=s)
    assert np.array_equal(got, oracle.matmul(A, oracle.dequantize(q, s), b))


def test_naive_matmul(pkg, L):
    rng = np.random.default_rng(12)
    M, N, K = 33, 300, 96
    A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.05), f16v(rng, N, 0.01)
    tol_check(gemm(pkg, L, A, W, b, kind="naive"), oracle.matmul(A, W, b))


def test_m1_row_matches_m512(pkg, L):
    rng = np.random.default_rng(13)
    A, W, b = f16v(rng, (512, 768), 1.0), f16v(rng, (2304, 768), 0.02), f16v(rng, 2304, 0.01)
    full = gemm(pkg, L, A, W, b)
    one = gemm(pkg, L, A[300:301], W, b)
    tol_check(one, full[300:301], max_abs=2e-3)


def test_k_zero_gives_bias(pkg, L):
    b = oracle.fp16_view(np.linspace(-1, 1, 40).astype(np.float32))
    dC = pkg.Dev(3 * 40 * 2)
    db = dev16(pkg, b)
    dA, dW = pkg.Dev(16), pkg.Dev(16)
    L.gpt2_matmul_tiled(dC.ptr, dA.ptr, dW.ptr, db.ptr, 3, 40, 0)
    L.gpt2_sync()
    pkg.check("K=0")
    got = oracle.f16_to_f32(dC.numpy(np.uint16, (3, 40)))
    assert np.array_equal(got, np.tile(b, (3, 1)))


def test_bad_arguments_record_error(pkg, L):
    L.gpt2_last_error()
    dC = pkg.Dev(64)
    L.gpt2_matmul_tiled(dC.ptr, None, None, None, 4, 4, 8)
    assert L.gpt2_last_error() != 0
    L.gpt2_matmul_tiled(dC.ptr, dC.ptr, dC.ptr, None, -1, 4, 8)
    assert L.gpt2_last_error() != 0
    assert L.gpt2_last_error() == 0


def test_dispatch_rule(pkg, L):
    """INT8 iff the backend has matmul_q and the GPT2QW carries codes (cuda/forward_cuda.cu:27-31)."""
    rng = np.random.default_rng(14)
    M, N, K = 64, 256, 128
    A, b = f16v(rng, (M, K), 1.0), f16v(rng, N, 0.01)
    w32 = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.05)
    W = oracle.fp16_view(w32)
    q, s, _ = oracle.quantize_fp16_view(w32)
    dA, dW, db = dev16(pkg, A), dev16(pkg, W), dev16(pkg, b)
    dq, ds = pkg.Dev.from_numpy(q), pkg.Dev.from_numpy(s)
    qw = pkg.GPT2QW(dq.ptr, ds.ptr)
    qnull = pkg.GPT2QW(None, None)
    dC = pkg.Dev(M * N * 2)
    out = {}
    for be in ("int8", "flash"):
        for tag, w in (("q", qw), ("null", qnull)):
            L.gpt2_matmul_dispatch(pkg.backend(be), dC.ptr, dA.ptr, dW.ptr, C.byref(w), db.ptr, M, N, K)
            L.gpt2_sync()
            out[(be, tag)] = oracle.f16_to_f32(dC.numpy(np.uint16, (M, N)))
    pkg.check("dispatch")
    ref16, refq = oracle.matmul(A, W, b), oracle.matmul(A, oracle.dequantize(q, s), b)
    tol_check(out[("int8", "q")], refq)
    assert not np.array_equal(out[("int8", "q")], out[("int8", "null")])
    for key in (("int8", "null"), ("flash", "q"), ("flash", "null")):
        tol_check(out[key], ref16)


@pytest.mark.parametrize("kind", ["fp16", "int8"])
@pytest.mark.parametrize("M,N,K", [(512, 768, 768), (512, 3072, 768), (200, 768, 3072), (33, 772, 768), (65, 770, 768),
                                   (64, 768, 3072), (20, 770, 3072), (128, 3072, 768), (128, 768, 3072),
                                   (1024, 768, 768), (1024, 3072, 768), (1000, 768, 3072), (256, 3072, 768)])
def test_fused_epilogues(pkg, L, kind, M, N, K):
    """The prefill's fused-epilogue GEMMs (forward_cuda.cu:99-105 folded into the GEMM: gelu_new of
    fp16(A.W^T + b), and fp16(resid + fp16(A.W^T + b)) with resid == C in place and in a separate
    buffer) against the oracle's matmul, gelu and add on the same fp16 values, at the trunk shapes,
    ragged M, and N with and without 8-byte C rows (the staged epilogue).  Bar as above.  The residual
    form needs 8-byte C rows (it reads the residual 4 columns at a time): elsewhere it declines and
    launches nothing, and the prefill runs the unfused sequence."""
    rng = np.random.default_rng(M * 7 + N + K)
    A = f16v(rng, (M, K), 1.0)
    b = f16v(rng, N, 0.01)
    R = f16v(rng, (M, N), 1.0)
    if kind == "int8":
        q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        Wd = oracle.dequantize(q, s)
        dW, ds = pkg.Dev.from_numpy(q), pkg.Dev.from_numpy(s)
    else:
        Wd = f16v(rng, (N, K), 0.02)
        dW, ds = dev16(pkg, Wd), None
    base = oracle.fp16_view(oracle.matmul(A, Wd, b))          # fp16(A.W^T + b)
    dA, db = dev16(pkg, A), dev16(pkg, b)
    for epi, want in ((1, oracle.fp16_view(oracle.gelu(base))), (2, oracle.fp16_view(R + base))):
        for in_place in ((False, True) if epi == 2 else (False,)):
            dC = dev16(pkg, R) if in_place else pkg.Dev(M * N * 2)
            dR = dC if in_place else dev16(pkg, R)
            ran = L.gpt2_tune_gemm_fused(dC.ptr, dA.ptr, dW.ptr, ds.ptr if ds is not None else None, db.ptr,
                                         M, N, K, epi, dR.ptr if epi == 2 else None)
            L.gpt2_sync()
            pkg.check("fused gemm")
            if epi == 2 and N % 4:
                assert ran == 0, (kind, M, N, K, epi)
                continue
            assert ran == 1, (kind, M, N, K, epi)
            got = oracle.f16_to_f32(dC.numpy(np.uint16, (M, N)))
            tol_check(got, want)


@pytest.mark.parametrize("kind", ["fp16", "int8"])
@pytest.mark.parametrize("M,N", [(512, 2304), (512, 3072), (200, 2304), (33, 3072), (1024, 2304), (2, 3072)])
def test_ln_panel_gemm(pkg, L, kind, M, N):
    """The LayerNorm-panel GEMMs (the prefill's LN1 -> QKV and LN2 -> fc in one launch, K = 768), every
    config, no epilogue and gelu: (a) bit for bit against gpt2_layernorm followed by the same GEMM on a
    one-k-group tile config (35) and gpt2_gelu -- the identity the fused prefill relies on; (b) against
    the oracle's layernorm, matmul and gelu (cpu/forward_cpu.c:35-50,52-69) on the same fp16 values, bar
    as above.  M = 200, 33 and 2 leave a partial 32-row block (rows past M normalize row M-1, unstored)."""
    K = 768
    rng = np.random.default_rng(M * 13 + N)
    X = oracle.fp16_view(rng.standard_normal((M, K), dtype=np.float32) +
                         rng.standard_normal((M, 1), dtype=np.float32) * np.float32(2.0))
    g = oracle.fp16_view(1.0 + rng.standard_normal(K, dtype=np.float32) * np.float32(0.2))
    bl = f16v(rng, K, 0.1)
    b = f16v(rng, N, 0.01)
    if kind == "int8":
        q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        Wd = oracle.dequantize(q, s)
        dW, ds = pkg.Dev.from_numpy(q), pkg.Dev.from_numpy(s)
    else:
        Wd = f16v(rng, (N, K), 0.02)
        dW, ds = dev16(pkg, Wd), None
    sp = ds.ptr if ds is not None else None
    dX, dg, dbl, db = dev16(pkg, X), dev16(pkg, g), dev16(pkg, bl), dev16(pkg, b)
    dLN, dRef = pkg.Dev(M * K * 2), pkg.Dev(M * N * 2)
    L.gpt2_layernorm(dLN.ptr, dX.ptr, dg.ptr, dbl.ptr, M, K)
    assert L.gpt2_tune_gemm_fits(35, K)
    L.gpt2_tune_gemm_run(35, dRef.ptr, dLN.ptr, dW.ptr, sp, db.ptr, M, N, K)
    L.gpt2_sync()
    pkg.check("layernorm + gemm")
    plain = dRef.numpy(np.uint16, (M, N))
    L.gpt2_gelu(dRef.ptr, M * N)
    L.gpt2_sync()
    gelu = dRef.numpy(np.uint16, (M, N))

    ln = oracle.fp16_view(oracle.layernorm(X, g, bl))
    base = oracle.fp16_view(oracle.matmul(ln, Wd, b))
    want = {0: base, 1: oracle.fp16_view(oracle.gelu(base))}
    exact = {0: plain, 1: gelu}
    dC = pkg.Dev(M * N * 2)
    for cfg in range(L.gpt2_tune_gemm_ln_count()):
        name = L.gpt2_tune_gemm_ln_name(cfg).decode()
        for epi in (0, 1):
            L.gpt2_memset(dC.ptr, 0xFF, M * N * 2)
            ran = L.gpt2_tune_gemm_ln(cfg, dC.ptr, dX.ptr, dg.ptr, dbl.ptr, dW.ptr, sp, db.ptr, M, N, K, epi)
            L.gpt2_sync()
            pkg.check("ln gemm " + name)
            assert ran == 1, (name, epi)
            got = dC.numpy(np.uint16, (M, N))
            bad = np.flatnonzero(got != exact[epi])
            assert bad.size == 0, f"{name} epi={epi}: {bad.size} elements differ from layernorm + gemm, first at {bad[0]}"
            tol_check(oracle.f16_to_f32(got), want[epi])
    # shapes the LayerNorm panel does not take: the caller falls back to the two launches
    assert L.gpt2_tune_gemm_ln(0, dC.ptr, dX.ptr, dg.ptr, dbl.ptr, dW.ptr, sp, db.ptr, M, N // 2, K // 2, 0) == 0
    assert L.gpt2_tune_gemm_ln(0, dC.ptr, dX.ptr, dg.ptr, dbl.ptr, dW.ptr, sp, db.ptr, 1, N, K, 0) == 0


def test_split_k_repeatable(pkg, L):
    """The split-K configs (K split over several work-groups per tile, the fp32 partials summed in
    split order by the last work-group to arrive, which also resets the tile's counter): a call
    repeated after a call with another tile count gives the same bits, and agrees with the oracle;
    fp16 and INT8."""
    rng = np.random.default_rng(21)
    sk = [c for c in range(L.gpt2_tune_gemm_count()) if L.gpt2_tune_gemm_name(c).decode().startswith("sk_")]
    assert sk
    big = (512, 768, 3072)
    small = (65, 200, 3072)
    data = {}
    for M, N, K in (big, small):
        A, W, b = f16v(rng, (M, K), 1.0), f16v(rng, (N, K), 0.05), f16v(rng, N, 0.01)
        q, s, _ = oracle.quantize_fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.05))
        data[(M, N, K)] = (A, W, b, q, s)
    for cfg in sk:
        name = L.gpt2_tune_gemm_name(cfg).decode()
        for kind in ("fp16", "int8"):
            runs = []
            for shape in (big, small, big):
                A, W, b, q, s = data[shape]
                runs.append(gemm(pkg, L, A, W if kind == "fp16" else None, b, cfg=cfg, kind=kind, q=q, s=s))
            assert np.array_equal(runs[0], runs[2]), f"{name} {kind}: repeated call differs"
            A, W, b, q, s = data[big]
            ref = oracle.matmul(A, W if kind == "fp16" else oracle.dequantize(q, s), b)
            tol_check(runs[0], ref)
