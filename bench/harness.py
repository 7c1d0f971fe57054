"""ctypes binding of bench/libgpt2bench.so: the native timing loops and microbenchmarks that bench.py
and the drivers in this directory use (bench/bench.hip), kept out of the product library.

    import harness                 # with bench/ on sys.path
    H = harness.lib(pkg)           # loads bare-metal-gpt2_amd/libgpt2amd.so first, then this library
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgpt2bench.so")

_vp = C.c_void_p
_fp = C.POINTER(C.c_float)
_i, _sz = C.c_int, C.c_size_t


class GPT2BenchOp(C.Structure):
    """One timed operation (bench.hip): kind 0 fp16 GEMM, 1 INT8 GEMM, 2 fp16 GEMV, 3 INT8 GEMV,
    4 causal prefill attention (C = att, A = qkv, M = T), 5 LayerNorm (C = out, A = x, W = gamma,
    bias = beta, M rows of K), 6 GEMM + residual in place (C += A.W^T + b), 7 residual add (C += A,
    M*N elements), 8 GEMM + gelu, 9 gelu in place (M*N elements), 16 + c the GEMM on tile config c
    (INT8 when Ws is set), 256 + c the GEMV on config c (INT8 when Ws is set)."""
    _fields_ = [("kind", C.c_int), ("C", _vp), ("A", _vp), ("W", _vp), ("Ws", _vp), ("bias", _vp),
                ("M", C.c_int), ("N", C.c_int), ("K", C.c_int)]


SIGNATURES = {
    "gpt2_bench_ops": (_i, [C.POINTER(GPT2BenchOp), _i, _i, _i, _fp, _fp]),
    "gpt2_bench_ops_graph": (_i, [C.POINTER(GPT2BenchOp), _i, _i, _i, _fp]),
    "gpt2_bench_time": (_i, [_vp, _vp, _fp]),
    "gpt2_device_info": (_i, [C.POINTER(_i), C.POINTER(_i), C.c_char_p, _i]),
    "gpt2_bench_empty": (_i, [_i, _fp]),
    "gpt2_bench_read": (_i, [_vp, _sz, _i, _fp]),
    "gpt2_bench_mfma": (_i, [_i, _i, _fp]),
    "gpt2_bench_copy": (_i, [_vp, _vp, _sz, _fp]),
    "gpt2_bench_ops_steps": (_i, [C.POINTER(GPT2BenchOp), _i, _i, _i, _fp, _fp]),
}

_lib = None


def lib(pkg):
    """Load libgpt2bench.so after the product library (it links against it; both share one copy of
    the product's state).  Raises FileNotFoundError when it has not been built (make -C bench)."""
    global _lib
    if _lib is None:
        pkg.lib()
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        H = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(H, name)
            fn.restype = res
            fn.argtypes = args
        _lib = H
    return _lib
