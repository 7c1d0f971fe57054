"""Support kernels around the matmul path, against the CPU oracle (cpu/forward_cpu.c restated).

fp16 storage on the GPU vs fp32 storage in the oracle: LayerNorm, gelu and attention are compared
with the fp16 parity bar (max abs 2e-2, rel-L2 1e-3) on identical fp16-valued inputs; embed and the
KV-cache writes are exact.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from conftest import tol_check

pytestmark = pytest.mark.gpu


def f16v(rng, shape, std, mean=0.0):
    return oracle.fp16_view(rng.standard_normal(shape, dtype=np.float32) * np.float32(std) + np.float32(mean))


def dev16(pkg, x):
    return pkg.Dev.from_numpy(oracle.f32_to_f16(x))


def back(d, shape):
    return oracle.f16_to_f32(d.numpy(np.uint16, shape))


@pytest.mark.parametrize("M,E", [(1, 768), (5, 768), (512, 768), (3, 100), (2, 1000)])
def test_layernorm(pkg, L, M, E):
    rng = np.random.default_rng(M * E)
    x, g, b = f16v(rng, (M, E), 2.0, 0.3), f16v(rng, E, 0.1, 1.0), f16v(rng, E, 0.1)
    dx, dg, db, dy = dev16(pkg, x), dev16(pkg, g), dev16(pkg, b), pkg.Dev(M * E * 2)
    L.gpt2_layernorm(dy.ptr, dx.ptr, dg.ptr, db.ptr, M, E)
    L.gpt2_sync()
    pkg.check("layernorm")
    tol_check(back(dy, (M, E)), oracle.layernorm(x, g, b))


@pytest.mark.parametrize("n", [1, 7, 8, 3072, 512 * 3072 + 3])
def test_gelu(pkg, L, n):
    rng = np.random.default_rng(n)
    x = f16v(rng, n, 2.0)
    dx = dev16(pkg, x)
    L.gpt2_gelu(dx.ptr, n)
    L.gpt2_sync()
    pkg.check("gelu")
    tol_check(back(dx, (n,)), oracle.gelu(x))


@pytest.mark.parametrize("n", [1, 8, 768, 512 * 768 + 5])
def test_add_exact(pkg, L, n):
    rng = np.random.default_rng(n + 1)
    x, y = f16v(rng, n, 1.0), f16v(rng, n, 1.0)
    dx, dy = dev16(pkg, x), dev16(pkg, y)
    L.gpt2_add(dx.ptr, dy.ptr, n)
    L.gpt2_sync()
    pkg.check("add")
    assert np.array_equal(back(dx, (n,)), oracle.fp16_view(x + y))


def test_embed_exact(pkg, L):
    rng = np.random.default_rng(2)
    T, E, V = 37, 768, 50257
    wte, wpe = f16v(rng, (V, E), 0.02), f16v(rng, (1024, E), 0.02)
    ids = rng.integers(0, V, T).astype(np.int32)
    ids[0], ids[-1] = 0, V - 1
    dwte, dwpe, dids, dx = dev16(pkg, wte), dev16(pkg, wpe), pkg.Dev.from_numpy(ids), pkg.Dev(T * E * 2)
    L.gpt2_embed(dx.ptr, dwte.ptr, dwpe.ptr, dids.ptr, T, E)
    L.gpt2_sync()
    pkg.check("embed")
    assert np.array_equal(back(dx, (T, E)), oracle.fp16_view(wte[ids] + wpe[:T]))
    # embed_one at position 300
    L.gpt2_embed_one(dx.ptr, dwte.ptr, dwpe.ptr, int(ids[3]), 300)
    L.gpt2_sync()
    assert np.array_equal(back(dx, (1, E))[0], oracle.fp16_view(wte[ids[3]] + wpe[300]))


# 16-query blocks and 32-key chunks: sizes on, just past and just short of those edges, and the
# largest cache (1024 rows).
@pytest.mark.parametrize("T", [1, 2, 15, 16, 17, 31, 32, 33, 48, 63, 64, 65, 127, 200, 512, 777, 1024])
def test_prefill_attention(pkg, L, T):
    rng = np.random.default_rng(T)
    qkv = f16v(rng, (T, 2304), 1.0)
    dq, da = dev16(pkg, qkv), pkg.Dev(T * 768 * 2)
    L.gpt2_attention_flash(da.ptr, dq.ptr, T, 768, 12, 64)
    L.gpt2_sync()
    pkg.check("attention")
    tol_check(back(da, (T, 768)), oracle.attention(qkv))


def test_prefill_attention_peaked_scores(pkg, L):
    """q, k ~ N(0, 16): scores q.k/8 of std 16, softmax near one-hot per row (online rescaling)."""
    rng = np.random.default_rng(77)
    T = 300
    qkv = f16v(rng, (T, 2304), 1.0)
    qkv[:, :1536] = oracle.fp16_view(qkv[:, :1536] * np.float32(4.0))
    dq, da = dev16(pkg, qkv), pkg.Dev(T * 768 * 2)
    L.gpt2_attention_flash(da.ptr, dq.ptr, T, 768, 12, 64)
    L.gpt2_sync()
    pkg.check("attention")
    got = back(da, (T, 768))
    assert np.isfinite(got).all()
    tol_check(got, oracle.attention(qkv))


def test_prefill_attention_equal_keys_is_mean(pkg, L):
    """All keys equal: every row is the running mean of the values (exact weights 1/(i+1))."""
    rng = np.random.default_rng(78)
    T = 129
    qkv = f16v(rng, (T, 2304), 1.0)
    qkv[:, 768:1536] = qkv[0, 768:1536]
    dq, da = dev16(pkg, qkv), pkg.Dev(T * 768 * 2)
    L.gpt2_attention_flash(da.ptr, dq.ptr, T, 768, 12, 64)
    L.gpt2_sync()
    pkg.check("attention")
    mean = np.cumsum(qkv[:, 1536:].astype(np.float64), 0) / np.arange(1, T + 1)[:, None]
    tol_check(back(da, (T, 768)), mean)


def test_attention_is_causal(pkg, L):
    rng = np.random.default_rng(3)
    T = 96
    a = f16v(rng, (T, 2304), 1.0)
    b = a.copy()
    b[50:] = f16v(rng, (T - 50, 2304), 1.0)
    outs = []
    for x in (a, b):
        dq, da = dev16(pkg, x), pkg.Dev(T * 768 * 2)
        L.gpt2_attention_flash(da.ptr, dq.ptr, T, 768, 12, 64)
        L.gpt2_sync()
        outs.append(back(da, (T, 768)))
    assert np.array_equal(outs[0][:50], outs[1][:50])
    assert not np.array_equal(outs[0][50:], outs[1][50:])


def make_kv(pkg, L, maxT):
    kv = pkg.KVCache(maxT)
    return kv


def test_kv_scatter_append_layout(pkg, L):
    """K[h][t][d] = qkv[t][768 + 64h + d], V likewise (cuda/kvcache.cu:57-76)."""
    rng = np.random.default_rng(4)
    maxT, T, Lyr = 256, 100, 7
    kv = make_kv(pkg, L, maxT)
    try:
        qkv = f16v(rng, (T, 2304), 1.0)
        dq = dev16(pkg, qkv)
        L.gpt2_kv_scatter_prefill(C.byref(kv.kv), Lyr, dq.ptr, T)
        one = f16v(rng, (1, 2304), 1.0)
        d1 = dev16(pkg, one)
        L.gpt2_kv_append_one(C.byref(kv.kv), Lyr, d1.ptr, T)
        L.gpt2_sync()
        pkg.check("kv writes")
        H, D = 12, 64
        raw = np.empty(kv.kv.bytes // 2, np.uint16)
        L.gpt2_d2h(raw.ctypes.data, kv.kv.data, kv.kv.bytes)
        arr = oracle.f16_to_f32(raw).reshape(12, 2, H, maxT, D)
        full = np.concatenate([qkv, one])
        for t in (0, 1, 57, T - 1, T):
            for h in (0, 5, 11):
                assert np.array_equal(arr[Lyr, 0, h, t], full[t, 768 + 64 * h:768 + 64 * h + 64])
                assert np.array_equal(arr[Lyr, 1, h, t], full[t, 1536 + 64 * h:1536 + 64 * h + 64])
    finally:
        kv.free()


@pytest.mark.parametrize("length", [1, 2, 63, 64, 65, 300, 513, 1024])
def test_decode_attention(pkg, L, length):
    """Decode attention of one query over cache rows [0, len) == prefill attention's last row."""
    rng = np.random.default_rng(length)
    maxT = 1024
    kv = make_kv(pkg, L, maxT)
    try:
        qkv = f16v(rng, (length, 2304), 1.0)
        dq = dev16(pkg, qkv)
        L.gpt2_kv_scatter_prefill(C.byref(kv.kv), 3, dq.ptr, length)
        last = dev16(pkg, qkv[-1:])
        da = pkg.Dev(768 * 2)
        L.gpt2_attn_decode(da.ptr, last.ptr, C.byref(kv.kv), 3, length)
        L.gpt2_sync()
        pkg.check("attn_decode")
        tol_check(back(da, (1, 768)), oracle.attention(qkv)[-1:])
    finally:
        kv.free()


def test_bad_launch_arguments(pkg, L):
    L.gpt2_last_error()
    d = pkg.Dev(1 << 16)
    L.gpt2_attention_flash(d.ptr, d.ptr, 4, 512, 8, 64)    # only E=768/H=12/D=64
    assert L.gpt2_last_error() != 0
    L.gpt2_embed_one(d.ptr, d.ptr, d.ptr, 50257, 0)       # token out of range
    assert L.gpt2_last_error() != 0
    kv = pkg.KVCache(16)
    try:
        L.gpt2_kv_append_one(C.byref(kv.kv), 0, d.ptr, 16)   # pos == maxT
        assert L.gpt2_last_error() != 0
        L.gpt2_attn_decode(d.ptr, d.ptr, C.byref(kv.kv), 12, 1)   # layer out of range
        assert L.gpt2_last_error() != 0
    finally:
        kv.free()
    assert L.gpt2_last_error() == 0
