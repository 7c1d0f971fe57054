"""Seeded synthetic GPT-2-124M weights and inputs (there is no network for real checkpoints).

Distributions follow the benchmark configs: weight matrices and embeddings N(0, 0.02); LayerNorm
gain 1 and shift 0; biases 0 ("plain", the config-1 model).  With plain=False the biases are
N(0, 0.01) and the LayerNorm gains/shifts are perturbed too, so that parity tests exercise every
term.  numpy's PCG64 generator makes every run, here and on the GPU box, see identical values.
"""
from __future__ import annotations

import numpy as np

N_LAYER, N_EMBD, VOCAB, N_CTX, FFN, QKV = 12, 768, 50257, 1024, 3072, 2304
TOTAL_PARAMS = 124439808


def layout():
    """(name, shape, kind) for every tensor of the body, in file order (model/weights.c:44-55)."""
    E, V, CX, Q, F = N_EMBD, VOCAB, N_CTX, QKV, FFN
    out = [("wte", (V, E), "w"), ("wpe", (CX, E), "w")]
    for L in range(N_LAYER):
        out += [(f"h{L}.ln1_g", (E,), "g"), (f"h{L}.ln1_b", (E,), "b"),
                (f"h{L}.qkv_w", (Q, E), "w"), (f"h{L}.qkv_b", (Q,), "b"),
                (f"h{L}.attn_proj_w", (E, E), "w"), (f"h{L}.attn_proj_b", (E,), "b"),
                (f"h{L}.ln2_g", (E,), "g"), (f"h{L}.ln2_b", (E,), "b"),
                (f"h{L}.fc_w", (F, E), "w"), (f"h{L}.fc_b", (F,), "b"),
                (f"h{L}.proj_w", (E, F), "w"), (f"h{L}.proj_b", (E,), "b")]
    out += [("lnf_g", (E,), "g"), ("lnf_b", (E,), "b")]
    return out


def offsets():
    off, o = {}, 0
    for name, shape, _ in layout():
        off[name] = (o, shape)
        o += int(np.prod(shape))
    assert o == TOTAL_PARAMS
    return off


def make_body(seed: int = 1234, plain: bool = True) -> np.ndarray:
    rng = np.random.default_rng(seed)
    body = np.empty(TOTAL_PARAMS, np.float32)
    o = 0
    for _, shape, kind in layout():
        n = int(np.prod(shape))
        seg = body[o:o + n]
        if kind == "w":
            seg[:] = rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)
        elif kind == "g":
            seg[:] = 1.0 if plain else 1.0 + rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)
        else:
            seg[:] = 0.0 if plain else rng.standard_normal(n, dtype=np.float32) * np.float32(0.01)
        o += n
    return body


def tensor(body: np.ndarray, name: str) -> np.ndarray:
    o, shape = offsets()[name]
    return body[o:o + int(np.prod(shape))].reshape(shape)


def token_ids(n: int, seed: int = 1234) -> np.ndarray:
    return np.random.default_rng(seed + 7).integers(0, VOCAB, size=n, dtype=np.int32)


def normal(shape, std=1.0, seed=0) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std))
