"""ctypes bindings for the CPU oracle (liboracle.so) and the reference's own CPU code (_ref/libref.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker.  The shipped library (bare-metal-gpt2_amd/) never does.

Every array argument is a C-contiguous numpy array of the documented dtype; the wrappers check
that and pass raw pointers, mirroring the C signatures in oracle/oracle.h.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

N_LAYER, N_HEAD, N_EMBD, VOCAB, N_CTX = 12, 12, 768, 50257, 1024
HEAD_DIM, FFN, QKV = 64, 3072, 2304
TOTAL_PARAMS = 124439808

_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int)
_i8p = C.POINTER(C.c_int8)
_u16p = C.POINTER(C.c_uint16)


def build(force: bool = False) -> None:
    """Compile liboracle.so and, if /root/reference is present, _ref/libref.so."""
    args = ["make", "-s", "-C", HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True)


def _ptr(a, ctype, dtype):
    if a is None:
        return None
    if not isinstance(a, np.ndarray) or a.dtype != dtype or not a.flags.c_contiguous:
        raise TypeError(f"expected C-contiguous {np.dtype(dtype).name} array")
    return a.ctypes.data_as(ctype)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = C.CDLL(ORACLE_SO)
        L.or_matmul.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.or_layernorm.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int]
        L.or_gelu_new.argtypes = [C.c_float]
        L.or_gelu_new.restype = C.c_float
        L.or_gelu_inplace.argtypes = [_f32p, C.c_size_t]
        L.or_attention.argtypes = [_f32p, _f32p, C.c_int]
        L.or_bind_weights.argtypes = [C.c_void_p, _f32p]
        L.or_bind_weights.restype = C.c_size_t
        L.or_forward.argtypes = [C.c_void_p, _i32p, C.c_int, _f32p, _f32p, _f32p, _f32p, C.c_int]
        L.or_f32_to_f16.argtypes = [C.c_float]
        L.or_f32_to_f16.restype = C.c_uint16
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f16_to_f32.restype = C.c_float
        L.or_f32_to_f16_array.argtypes = [_u16p, _f32p, C.c_size_t]
        L.or_f16_to_f32_array.argtypes = [_f32p, _u16p, C.c_size_t]
        L.or_quantize_rows.argtypes = [_i8p, _f32p, _f32p, C.c_int, C.c_int]
        L.or_quantize_rows.restype = C.c_int
        L.or_quantize_rows_ld.argtypes = [_i8p, _f32p, _f32p, C.c_int, C.c_int]
        L.or_quantize_rows_ld.restype = C.c_int
        L.or_quantize_fp16_view.argtypes = [_i8p, _f32p, _f32p, C.c_int, C.c_int]
        L.or_quantize_fp16_view.restype = C.c_int
        L.or_dequantize.argtypes = [_f32p, _i8p, _f32p, C.c_int, C.c_int]
        L.or_check_f16c_range.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint32)]
        L.or_check_f16c_range.restype = C.c_uint64
        L.or_check_f16c_back.restype = C.c_uint64
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref():
    """The reference's own cpu/forward_cpu.c + model/weights.c, built by oracle/Makefile."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise FileNotFoundError(REF_SO)
        R = C.CDLL(REF_SO)
        R.ref_matmul.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        R.ref_layernorm.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int]
        R.ref_gelu_new.argtypes = [C.c_float]
        R.ref_gelu_new.restype = C.c_float
        R.ref_attention.argtypes = [_f32p, _f32p, C.c_int]
        R.ref_load_weights.argtypes = [C.c_char_p, C.POINTER(C.c_void_p)]
        R.ref_load_weights.restype = C.c_int
        R.ref_free_weights.argtypes = [C.c_void_p]
        R.ref_weight_offsets.argtypes = [C.c_void_p, C.POINTER(C.c_long)]
        R.ref_forward_flat.argtypes = [_f32p, C.POINTER(C.c_long), _i32p, C.c_int,
                                       _f32p, _f32p, _f32p, _f32p, C.c_int]
        _ref = R
    return _ref


# ---------------------------------------------------------------- numpy-level wrappers (oracle)

def matmul(A, W, bias=None):
    """C[M,N] = A[M,K] . W[N,K]^T + bias  (float32 in/out, double accumulation)."""
    A = np.ascontiguousarray(A, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    M, K = A.shape
    N, K2 = W.shape
    assert K == K2
    out = np.empty((M, N), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().or_matmul(_ptr(out, _f32p, np.float32), _ptr(A, _f32p, np.float32),
                    _ptr(W, _f32p, np.float32), _ptr(b, _f32p, np.float32), M, N, K)
    return out


def layernorm(x, g, b):
    x = np.ascontiguousarray(x, np.float32)
    M, E = x.shape
    out = np.empty_like(x)
    lib().or_layernorm(_ptr(out, _f32p, np.float32), _ptr(x, _f32p, np.float32),
                       _ptr(np.ascontiguousarray(g, np.float32), _f32p, np.float32),
                       _ptr(np.ascontiguousarray(b, np.float32), _f32p, np.float32), M, E)
    return out


def gelu(x):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().or_gelu_inplace(_ptr(x.reshape(-1), _f32p, np.float32), x.size)
    return x


def attention(qkv):
    qkv = np.ascontiguousarray(qkv, np.float32)
    T = qkv.shape[0]
    assert qkv.shape[1] == QKV
    out = np.empty((T, N_EMBD), np.float32)
    lib().or_attention(_ptr(out, _f32p, np.float32), _ptr(qkv, _f32p, np.float32), T)
    return out


class _OrLayer(C.Structure):
    _fields_ = [(n, _f32p) for n in ("ln1_g", "ln1_b", "qkv_w", "qkv_b", "attn_proj_w", "attn_proj_b",
                                     "ln2_g", "ln2_b", "fc_w", "fc_b", "proj_w", "proj_b")]


class _OrWeights(C.Structure):
    _fields_ = [("wte", _f32p), ("wpe", _f32p), ("layers", _OrLayer * N_LAYER),
                ("lnf_g", _f32p), ("lnf_b", _f32p)]


def forward(flat, ids, logits_all=True, want_blocks=False):
    """Whole-model forward on a flat fp32 body (file order). Returns dict of captures."""
    flat = np.ascontiguousarray(flat, np.float32)
    assert flat.size == TOTAL_PARAMS
    ids = np.ascontiguousarray(ids, np.int32)
    T = ids.size
    w = _OrWeights()
    used = lib().or_bind_weights(C.byref(w), _ptr(flat, _f32p, np.float32))
    assert used == TOTAL_PARAMS
    embed = np.empty((T, N_EMBD), np.float32)
    blocks = np.empty((N_LAYER, T, N_EMBD), np.float32) if want_blocks else None
    final_ln = np.empty((T, N_EMBD), np.float32)
    logits = np.empty((T if logits_all else 1, VOCAB), np.float32)
    lib().or_forward(C.byref(w), _ptr(ids, _i32p, np.int32), T, _ptr(embed, _f32p, np.float32),
                     _ptr(blocks, _f32p, np.float32), _ptr(final_ln, _f32p, np.float32),
                     _ptr(logits, _f32p, np.float32), 1 if logits_all else 0)
    return {"embed": embed, "blocks": blocks, "final_ln": final_ln, "logits": logits}


def f32_to_f16(x):
    """fp32 -> fp16 bit patterns (uint16), IEEE round-to-nearest-even."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_array(_ptr(out.reshape(-1), _u16p, np.uint16),
                              _ptr(x.reshape(-1), _f32p, np.float32), x.size)
    return out


def f16_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_array(_ptr(out.reshape(-1), _f32p, np.float32),
                              _ptr(h.reshape(-1), _u16p, np.uint16), h.size)
    return out


def fp16_view(x):
    return f16_to_f32(f32_to_f16(x))


def quantize_rows(w16, longdouble=False):
    """Per-output-row symmetric INT8 of an fp16-valued fp32 [N,K] matrix -> (q int8, s f32, dead)."""
    w16 = np.ascontiguousarray(w16, np.float32)
    N, K = w16.shape
    q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float32)
    fn = lib().or_quantize_rows_ld if longdouble else lib().or_quantize_rows
    dead = fn(_ptr(q, _i8p, np.int8), _ptr(s, _f32p, np.float32), _ptr(w16, _f32p, np.float32), N, K)
    return q, s, dead


def quantize_fp16_view(w32):
    w32 = np.ascontiguousarray(w32, np.float32)
    N, K = w32.shape
    q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float32)
    dead = lib().or_quantize_fp16_view(_ptr(q, _i8p, np.int8), _ptr(s, _f32p, np.float32),
                                       _ptr(w32, _f32p, np.float32), N, K)
    return q, s, dead


def dequantize(q, s):
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(s, np.float32)
    N, K = q.shape
    out = np.empty((N, K), np.float32)
    lib().or_dequantize(_ptr(out, _f32p, np.float32), _ptr(q, _i8p, np.int8),
                        _ptr(s, _f32p, np.float32), N, K)
    return out


# ---------------------------------------------------------------- reference wrappers (_ref)

def ref_matmul(A, W, bias=None):
    A = np.ascontiguousarray(A, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    M, K = A.shape
    N = W.shape[0]
    out = np.empty((M, N), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    ref().ref_matmul(_ptr(out, _f32p, np.float32), _ptr(A, _f32p, np.float32),
                     _ptr(W, _f32p, np.float32), _ptr(b, _f32p, np.float32), M, N, K)
    return out


def ref_layernorm(x, g, b):
    x = np.ascontiguousarray(x, np.float32)
    assert x.shape[1] == N_EMBD
    out = np.empty_like(x)
    ref().ref_layernorm(_ptr(out, _f32p, np.float32), _ptr(x, _f32p, np.float32),
                        _ptr(np.ascontiguousarray(g, np.float32), _f32p, np.float32),
                        _ptr(np.ascontiguousarray(b, np.float32), _f32p, np.float32), x.shape[0])
    return out


def ref_gelu(x):
    x = np.asarray(x, np.float32)
    return np.array([ref().ref_gelu_new(float(v)) for v in x.reshape(-1)], np.float32).reshape(x.shape)


def ref_attention(qkv):
    qkv = np.ascontiguousarray(qkv, np.float32)
    out = np.empty((qkv.shape[0], N_EMBD), np.float32)
    ref().ref_attention(_ptr(out, _f32p, np.float32), _ptr(qkv, _f32p, np.float32), qkv.shape[0])
    return out


def write_gpt2_file(path, flat):
    """Write a 'GPT2' v1 fp32 weight file (model/weights.c:18-29 header, then the body)."""
    hdr = np.zeros(16, np.int32)
    hdr[:10] = [0x47505432, 1, N_LAYER, N_HEAD, N_EMBD, VOCAB, N_CTX, FFN, QKV, 0]
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.ascontiguousarray(flat, np.float32).tobytes())


def ref_offsets_from_file(path):
    """Load a weight file with the reference loader; return (rc, offsets[148] or None)."""
    h = C.c_void_p()
    rc = ref().ref_load_weights(path.encode(), C.byref(h))
    if rc != 0:
        return rc, None
    off = (C.c_long * 148)()
    ref().ref_weight_offsets(h, off)
    ref().ref_free_weights(h)
    return 0, np.array(list(off), np.int64)


def ref_forward(flat, offsets, ids, logits_all=True, want_blocks=False):
    flat = np.ascontiguousarray(flat, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    T = ids.size
    off = (C.c_long * 148)(*[int(v) for v in offsets])
    embed = np.empty((T, N_EMBD), np.float32)
    blocks = np.empty((N_LAYER, T, N_EMBD), np.float32) if want_blocks else None
    final_ln = np.empty((T, N_EMBD), np.float32)
    logits = np.empty((T if logits_all else 1, VOCAB), np.float32)
    ref().ref_forward_flat(_ptr(flat, _f32p, np.float32), off, _ptr(ids, _i32p, np.int32), T,
                           _ptr(embed, _f32p, np.float32), _ptr(blocks, _f32p, np.float32),
                           _ptr(final_ln, _f32p, np.float32), _ptr(logits, _f32p, np.float32),
                           1 if logits_all else 0)
    return {"embed": embed, "blocks": blocks, "final_ln": final_ln, "logits": logits}


def oracle_offsets():
    """Tensor offsets of or_bind_weights, in the same 148-entry order as ref_weight_offsets."""
    flat = np.zeros(1, np.float32)
    w = _OrWeights()
    base = C.addressof(flat.ctypes.data_as(_f32p).contents)
    lib().or_bind_weights(C.byref(w), flat.ctypes.data_as(_f32p))
    def off(p):
        return (C.cast(p, C.c_void_p).value - base) // 4
    out = [off(w.wte), off(w.wpe)]
    for L in range(N_LAYER):
        ly = w.layers[L]
        out += [off(getattr(ly, n)) for n, _ in _OrLayer._fields_]
    out += [off(w.lnf_g), off(w.lnf_b)]
    return np.array(out, np.int64)
