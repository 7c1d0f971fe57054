"""The algebra behind the prefill's LayerNorm fold, checked on the CPU against the oracle's LayerNorm and
matmul (oracle/oracle.c, following the reference's cpu/ layernorm and matmul):

    LayerNorm(x; g, b) . W^T + bias  ==  rstd * ((x*g) . W^T - mu * G) + H + bias,
    G_n = sum_k g_k W_nk,  H_n = sum_k b_k W_nk,  mu = mean(x),  rstd = 1/sqrt(var(x) + 1e-5),

exactly in float64, and within the fp16 bar when x*g is rounded to fp16 and the variance comes from
sum x and sum x^2 over 16-column slices (as the GPU kernels do).  A dropped term (the mu*G
correction, H, the rstd scaling) or a transposed W fails the float64 check by orders of magnitude.
"""
import numpy as np

import oracle

E, N, EPS = 768, 320, 1e-5


def fold(x, g, b, W, bias, round_xg):
    x = x.astype(np.float64)
    parts = x.reshape(x.shape[0], E // 16, 16)
    s1, s2 = parts.sum(-1).sum(-1), (parts * parts).sum(-1).sum(-1)
    mu = s1 / E
    var = np.maximum(s2 / E - mu * mu, 0.0)
    rstd = 1.0 / np.sqrt(var + EPS)
    xg = x * g
    if round_xg:
        xg = xg.astype(np.float16).astype(np.float64)
    G, H = W.astype(np.float64) @ g, W.astype(np.float64) @ b
    return rstd[:, None] * (xg @ W.T.astype(np.float64) - mu[:, None] * G[None, :]) + H[None, :] + bias


def case(seed, shift=0.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((40, E)) * 0.5 + shift).astype(np.float16).astype(np.float64)
    g = 1.0 + 0.1 * rng.standard_normal(E)
    b = 0.1 * rng.standard_normal(E)
    W = 0.02 * rng.standard_normal((N, E))
    bias = 0.01 * rng.standard_normal(N)
    return x, g, b, W, bias


def reference(x, g, b, W, bias):
    y = oracle.layernorm(x.astype(np.float32), g.astype(np.float32), b.astype(np.float32))
    return oracle.matmul(y, W.astype(np.float32), bias.astype(np.float32)).astype(np.float64)


def rel(a, r):
    return float(np.abs(a - r).max() / np.abs(r).max())


def test_fold_identity_exact():
    x, g, b, W, bias = case(1)
    assert rel(fold(x, g, b, W, bias, False), reference(x, g, b, W, bias)) < 1e-5   # fp32 oracle vs f64


def test_fold_identity_fp16_xg():
    for seed, shift in ((2, 0.0), (3, 0.5)):
        x, g, b, W, bias = case(seed, shift)
        assert rel(fold(x, g, b, W, bias, True), reference(x, g, b, W, bias)) < 2e-3


def test_fold_catches_dropped_terms():
    x, g, b, W, bias = case(4, 0.5)
    ref = reference(x, g, b, W, bias)
    assert rel(fold(x, g, b, W, bias, False), ref) < 1e-5
    assert rel(fold(x, g, np.zeros(E), W, bias, False), ref) > 1e-2          # H dropped
    assert rel(fold(x, g, b, W[::-1].copy(), bias, False), ref) > 1e-2       # rows of W mixed up
    # a per-row shift of x leaves LayerNorm unchanged; the folded form keeps that only through mu * G
    assert rel(fold(x + 1.0, g, b, W, bias, False), ref) < 1e-5
    x64 = x.astype(np.float64)
    rstd = 1.0 / np.sqrt(x64.var(1) + EPS)
    no_mu = rstd[:, None] * ((x64 * g) @ W.T) + W @ b + bias                 # mu * G dropped
    assert rel(no_mu, ref) > 1e-2
