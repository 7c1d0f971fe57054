"""Python binding of libgpt2amd.so, the MI355X (gfx950) matmul path of bare-metal-gpt2.

The library is C/HIP (csrc/); this module only loads it and mirrors its C structs with ctypes so
tests and bench.py can drive the C-ABI exactly as C host code would (include/gpt2_kernels.h,
include/gpt2_kvcache.h).  There is no fallback: if the library is missing, `lib()` raises.

Import it with `load_package()` from __graft_entry__ (the directory name is not an identifier), or
add the repository root to sys.path and use importlib.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgpt2amd.so")

N_LAYER, N_HEAD, N_EMBD, VOCAB, N_CTX = 12, 12, 768, 50257, 1024
HEAD_DIM, FFN, QKV = 64, 3072, 2304
TOTAL_PARAMS = 124439808
DECODE_AUTO, DECODE_MULTI, DECODE_PERSISTENT = -1, 0, 1   # gpt2_decode_graph_create_mode modes
N_QTENSORS = 1 + 4 * N_LAYER

_vp = C.c_void_p
_fp = C.POINTER(C.c_float)


def build(force: bool = True) -> None:
    """Compile libgpt2amd.so with hipcc for gfx950 (make -C csrc)."""
    args = ["make", "-s", "-C", os.path.join(HERE, "csrc"), "-j8"]
    if force:
        args.append("-B")
    subprocess.run(args, check=True)


# ----------------------------------------------------------------------------- C structs
class GPT2Layer(C.Structure):
    _fields_ = [(n, _fp) for n in ("ln1_g", "ln1_b", "qkv_w", "qkv_b", "attn_proj_w", "attn_proj_b",
                                   "ln2_g", "ln2_b", "fc_w", "fc_b", "proj_w", "proj_b")]


class GPT2Weights(C.Structure):
    _fields_ = [("data", _fp), ("n_floats", C.c_size_t), ("wte", _fp), ("wpe", _fp),
                ("layers", GPT2Layer * N_LAYER), ("lnf_g", _fp), ("lnf_b", _fp)]


class GPT2LayerGPU(C.Structure):
    _fields_ = [(n, _vp) for n in ("ln1_g", "ln1_b", "qkv_w", "qkv_b", "attn_proj_w", "attn_proj_b",
                                   "ln2_g", "ln2_b", "fc_w", "fc_b", "proj_w", "proj_b")]


class GPT2QW(C.Structure):
    _fields_ = [("q", _vp), ("s", _vp)]


class GPT2QLayerGPU(C.Structure):
    _fields_ = [("qkv_w", GPT2QW), ("attn_proj_w", GPT2QW), ("fc_w", GPT2QW), ("proj_w", GPT2QW)]


class GPT2QWeightsGPU(C.Structure):
    _fields_ = [("qdata", _vp), ("sdata", _vp), ("nq", C.c_size_t), ("ns", C.c_size_t),
                ("streamed_bytes", C.c_size_t), ("wte", GPT2QW), ("layers", GPT2QLayerGPU * N_LAYER)]


class GPT2WeightsGPU(C.Structure):
    _fields_ = [("data", _vp), ("n", C.c_size_t), ("wte", _vp), ("wpe", _vp),
                ("layers", GPT2LayerGPU * N_LAYER), ("lnf_g", _vp), ("lnf_b", _vp), ("q", _vp)]


class GPT2ScratchGPU(C.Structure):
    _fields_ = [(n, _vp) for n in ("x", "ln", "qkv", "att", "ao", "fc", "ff")] + [("maxT", C.c_int)]


class GPT2CapsGPU(C.Structure):
    _fields_ = [("embed", _vp), ("blocks", _vp), ("final_ln", _vp), ("logits", _vp),
                ("logits_all", C.c_int), ("kv", _vp)]


class GPT2KVCache(C.Structure):
    _fields_ = [("data", _vp), ("bytes", C.c_size_t), ("maxT", C.c_int), ("nLayer", C.c_int),
                ("nHead", C.c_int), ("headDim", C.c_int), ("len", C.c_int)]


class GPT2Backend(C.Structure):
    _fields_ = [("name", C.c_char_p)] + [(n, _vp) for n in (
        "embed", "layernorm", "matmul", "attention", "gelu", "add", "matmul_q", "gemv", "gemv_q")]


# (name, restype, argtypes) for every symbol declared in include/*.h plus the test/tuning hooks.
_i, _u, _sz, _d = C.c_int, C.c_uint, C.c_size_t, C.c_double
_BE = C.POINTER(GPT2Backend)
SIGNATURES = {
    # include/gpt2_kernels.h
    "gpt2_load_weights": (_i, [C.c_char_p, C.POINTER(GPT2Weights)]),
    "gpt2_free_weights": (None, [C.POINTER(GPT2Weights)]),
    "gpt2_bind_weights": (_sz, [C.POINTER(GPT2Weights), _vp]),
    "gpt2_upload_fp16": (None, [C.POINTER(GPT2Weights), C.POINTER(GPT2WeightsGPU)]),
    "gpt2_free_gpu": (None, [C.POINTER(GPT2WeightsGPU)]),
    "gpt2_scratch_alloc": (None, [C.POINTER(GPT2ScratchGPU), _i]),
    "gpt2_scratch_free": (None, [C.POINTER(GPT2ScratchGPU)]),
    "gpt2_matmul_tiled": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "gpt2_matmul_int8": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "gpt2_matmul_naive": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "gpt2_attention_flash": (None, [_vp, _vp, _i, _i, _i, _i]),
    "gpt2_embed": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "gpt2_layernorm": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "gpt2_gelu": (None, [_vp, _sz]),
    "gpt2_add": (None, [_vp, _vp, _sz]),
    "gpt2_backend_by_name": (_BE, [C.c_char_p]),
    "gpt2_matmul_dispatch": (None, [_BE, _vp, _vp, _vp, C.POINTER(GPT2QW), _vp, _i, _i, _i]),
    "gpt2_quant_load_upload": (_i, [C.c_char_p, C.POINTER(GPT2WeightsGPU), C.POINTER(GPT2QWeightsGPU)]),
    "gpt2_quant_free": (None, [C.POINTER(GPT2QWeightsGPU)]),
    "gpt2_quant_attach_if_needed": (_i, [_BE, C.POINTER(GPT2WeightsGPU), C.POINTER(GPT2QWeightsGPU)]),
    "gpt2_quant_build": (_i, [C.POINTER(GPT2WeightsGPU), C.POINTER(GPT2QWeightsGPU), _vp]),
    "gpt2_quantize_rows": (None, [_vp, _vp, _vp, _i, _i]),
    "gpt2_quant_write_file": (_i, [C.c_char_p, C.POINTER(GPT2QWeightsGPU), _vp]),
    "gpt2_forward_cuda": (None, [_BE, C.POINTER(GPT2WeightsGPU), _vp, _i, C.POINTER(GPT2ScratchGPU),
                                 C.POINTER(GPT2CapsGPU)]),
    "gpt2_forward_noalloc": (None, [_BE, C.POINTER(GPT2WeightsGPU), _vp, _i, C.POINTER(GPT2CapsGPU)]),
    "gpt2_set_stream": (None, [_vp]),
    "gpt2_get_stream": (_vp, []),
    "gpt2_last_error": (_i, []),
    "gpt2_error_string": (C.c_char_p, [_i]),
    "gpt2_dmalloc": (_vp, [_sz]),
    "gpt2_dfree": (None, [_vp]),
    "gpt2_h2d": (_i, [_vp, _vp, _sz]),
    "gpt2_d2h": (_i, [_vp, _vp, _sz]),
    "gpt2_d2d": (_i, [_vp, _vp, _sz]),
    "gpt2_memset": (_i, [_vp, _i, _sz]),
    "gpt2_sync": (_i, []),
    "gpt2_f32_to_f16": (None, [_vp, _vp, _sz]),
    # include/gpt2_kvcache.h
    "gpt2_kv_alloc": (_i, [C.POINTER(GPT2KVCache), _i]),
    "gpt2_kv_scatter_prefill": (None, [C.POINTER(GPT2KVCache), _i, _vp, _i]),
    "gpt2_embed_one": (None, [_vp, _vp, _vp, _i, _i]),
    "gpt2_kv_append_one": (None, [C.POINTER(GPT2KVCache), _i, _vp, _i]),
    "gpt2_attn_decode": (None, [_vp, _vp, C.POINTER(GPT2KVCache), _i, _i]),
    "gpt2_kv_free": (None, [C.POINTER(GPT2KVCache)]),
    "gpt2_kv_reset": (None, [C.POINTER(GPT2KVCache)]),
    "gpt2_kv_step_bytes": (_d, [C.POINTER(GPT2KVCache), _i]),
    "gpt2_decode_step_cuda": (None, [_BE, C.POINTER(GPT2WeightsGPU), C.POINTER(GPT2KVCache), _i, _i,
                                     C.POINTER(GPT2ScratchGPU), _vp, _vp]),
    "gpt2_prefill_fill_cache": (None, [_BE, C.POINTER(GPT2WeightsGPU), C.POINTER(GPT2KVCache), _vp, _i,
                                       C.POINTER(GPT2ScratchGPU), C.POINTER(GPT2CapsGPU)]),
    "gpt2_gemv_fp16": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "gpt2_gemv_int8": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "gpt2_gemv_dispatch": (None, [_BE, _vp, _vp, _vp, C.POINTER(GPT2QW), _vp, _i, _i]),
    "gpt2_decode_graph_create": (_vp, [_BE, C.POINTER(GPT2WeightsGPU), C.POINTER(GPT2KVCache),
                                       C.POINTER(GPT2ScratchGPU), _vp, _vp]),
    "gpt2_decode_graph_create_mode": (_vp, [_BE, C.POINTER(GPT2WeightsGPU), C.POINTER(GPT2KVCache),
                                            C.POINTER(GPT2ScratchGPU), _vp, _vp, _i]),
    "gpt2_decode_graph_mode": (_i, [_vp]),
    "gpt2_tune_decode_spin": (None, [_i]),
    "gpt2_tune_decode_holds": (None, [_i, _i, _i]),
    "gpt2_tune_decode_trace": (None, [_vp]),
    "gpt2_tune_prefill_fused": (None, [_i]),
    "gpt2_tune_prefill_lnfold": (None, [_i]),
    "gpt2_tune_prefill_lnfold_sites": (_i, []),
    "gpt2_decode_graph_set": (_i, [_vp, _i, _i]),
    "gpt2_decode_graph_run": (_i, [_vp, _i]),
    "gpt2_decode_graph_sync": (_i, [_vp, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "gpt2_decode_graph_destroy": (None, [_vp]),
    "gpt2_decode_graph_time": (_i, [_vp, _i, _fp]),
    # bench / tuning hooks (not part of the reference interface)
    "gpt2_tune_gemm_count": (_i, []),
    "gpt2_tune_gemm_name": (C.c_char_p, [_i]),
    "gpt2_tune_gemm_pick": (_i, [_i, _i, _i]),
    "gpt2_tune_prefill_persistent": (None, [_i]),
    "gpt2_tune_prefill_spin": (None, [_i]),
    "gpt2_prefill_status": (_i, []),
    "gpt2_test_dmalloc_calls": (C.c_long, []),
    "gpt2_test_mem_free": (C.c_longlong, []),
    "gpt2_tune_prefill_trace": (_i, [_vp, _i, _i]),
    "gpt2_tune_gemm_pick_q": (_i, [_i, _i, _i, _i]),
    "gpt2_tune_gemm_fits": (_i, [_i, _i]),
    "gpt2_tune_gemm_force": (None, [_i]),
    "gpt2_tune_gemm_run": (None, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "gpt2_tune_gemm_fused": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "gpt2_tune_gemm_ln_count": (_i, []),
    "gpt2_tune_gemm_ln_name": (C.c_char_p, [_i]),
    "gpt2_tune_gemm_ln_force": (None, [_i]),
    "gpt2_tune_gemm_skinny": (None, [_i]),
    "gpt2_tune_gemm_skinny_max": (_i, [_i]),
    "gpt2_tune_gemm_skinny_calls": (_i, []),
    "gpt2_tune_gemm_ln": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "gpt2_tune_gemv_count": (_i, []),
    "gpt2_tune_gemv_name": (C.c_char_p, [_i]),
    "gpt2_tune_gemv_fits": (_i, [_i, _i, _i]),
    "gpt2_tune_gemv_run": (None, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i]),
}

DATA_SYMBOLS = ["GPT2_BACKEND_NAIVE", "GPT2_BACKEND_TILED", "GPT2_BACKEND_FLASH", "GPT2_BACKEND_INT8",
                "GPT2_BACKEND_GEMV"]

_lib = None


def lib():
    """Load libgpt2amd.so (raises FileNotFoundError when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class GPUError(RuntimeError):
    pass


def check(what: str = "") -> None:
    """Raise GPUError if the library recorded an error since the last check."""
    code = lib().gpt2_last_error()
    if code:
        raise GPUError(f"{what}: {lib().gpt2_error_string(code).decode()}")


def backend(name: str):
    return lib().gpt2_backend_by_name(name.encode())


# ----------------------------------------------------------------------------- device buffers
class Dev:
    """A device allocation owned by Python (gpt2_dmalloc / gpt2_dfree)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = lib().gpt2_dmalloc(max(1, self.nbytes))
        if not self.ptr:
            check("gpt2_dmalloc")
            raise GPUError(f"gpt2_dmalloc({nbytes}) failed")

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "Dev":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        if lib().gpt2_h2d(self.ptr, a.ctypes.data, a.nbytes):
            check("gpt2_h2d")

    def numpy(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        if lib().gpt2_d2h(out.ctypes.data, self.ptr, out.nbytes):
            check("gpt2_d2h")
        return out

    def at(self, byte_offset: int) -> int:
        return self.ptr + int(byte_offset)

    def free(self) -> None:
        if self.ptr:
            lib().gpt2_dfree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def f16(a) -> np.ndarray:
    """float32 values -> float16 storage (numpy's conversion rounds to nearest even)."""
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16))


def to_dev_f16(a) -> Dev:
    return Dev.from_numpy(f16(a))


# ----------------------------------------------------------------------------- model helpers
class Model:
    """fp16 device weights uploaded from a host fp32 body in file order (gpt2_upload_fp16)."""

    def __init__(self, body: np.ndarray):
        body = np.ascontiguousarray(body, np.float32)
        assert body.size == TOTAL_PARAMS
        self.body = body
        self.host = GPT2Weights()
        used = lib().gpt2_bind_weights(C.byref(self.host), body.ctypes.data)
        assert used == TOTAL_PARAMS
        self.gpu = GPT2WeightsGPU()
        lib().gpt2_upload_fp16(C.byref(self.host), C.byref(self.gpu))
        check("gpt2_upload_fp16")
        self.q = None

    def quantize(self, keep=None) -> None:
        """Attach INT8 weights quantized on the GPU (default: head kept fp16)."""
        self.q = GPT2QWeightsGPU()
        kp = None
        if keep is not None:
            self._keep = (C.c_int * N_QTENSORS)(*[int(k) for k in keep])
            kp = C.cast(self._keep, _vp)
        if lib().gpt2_quant_build(C.byref(self.gpu), C.byref(self.q), kp):
            check("gpt2_quant_build")
            raise GPUError("gpt2_quant_build failed")

    def free(self) -> None:
        if self.q is not None:
            lib().gpt2_quant_free(C.byref(self.q))
            self.q = None
            self.gpu.q = None
        lib().gpt2_free_gpu(C.byref(self.gpu))


class Scratch:
    def __init__(self, maxT: int):
        self.s = GPT2ScratchGPU()
        lib().gpt2_scratch_alloc(C.byref(self.s), maxT)
        check("gpt2_scratch_alloc")

    def free(self) -> None:
        lib().gpt2_scratch_free(C.byref(self.s))


class KVCache:
    def __init__(self, maxT: int = N_CTX):
        self.kv = GPT2KVCache()
        if lib().gpt2_kv_alloc(C.byref(self.kv), maxT):
            check("gpt2_kv_alloc")
            raise GPUError("gpt2_kv_alloc failed")

    def free(self) -> None:
        lib().gpt2_kv_free(C.byref(self.kv))


def half_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)
