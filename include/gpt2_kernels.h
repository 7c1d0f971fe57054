/* gpt2_kernels.h -- C-ABI boundary of the MI355X (gfx950) matmul path of bare-metal-gpt2.
 *
 * Drop-in for the reference's launcher API, cuda/kernels.cuh:19-117: same struct layouts, same
 * function names, same parameter order and meaning.  Differences a caller can see:
 *   - `gpt2_half` (uint16_t, IEEE binary16 bits) stands where the reference has CUDA's `half`.  Both
 *     are 2-byte, 2-aligned storage types, so pointers and structs have identical layout, and no
 *     GPU vendor header is needed to include this file.
 *   - every symbol has C linkage (the reference's are C++), so cgo/ctypes/JNI can bind them.
 *   - launchers enqueue on the stream chosen by gpt2_set_stream() (default: the null stream),
 *     which lets a caller capture them into a graph; the reference always uses the null stream.
 *   - launchers check their arguments on the host.  A bad shape or pointer records an error that
 *     gpt2_last_error() returns (the reference launches unchecked and leaves the caller to call
 *     cudaGetLastError, cuda/common.cuh:17-18); nothing is launched in that case.
 * All tensor pointers are device pointers unless stated.  The caller owns every buffer.
 *
 * GEMM contract everywhere (cuda/kernels.cuh:72):  C[M,N] = A[M,K] . W[N,K]^T + bias[N]
 *   A row-major [M,K] fp16; W row-major [N,K] (row n = output channel n, contiguous in k);
 *   bias fp16 [N] or NULL; C row-major [M,N] fp16, fully overwritten; fp32 accumulation.
 * INT8 weight-only form (cuda/kernels.cuh:79-80, cuda/kernels_quant.cu:38-60):
 *   C[m,n] = s[n] * (sum_k A[m,k] * q[n,k]) + bias[n]   (scale after the fp32 sum, bias last)
 */
#ifndef GPT2_KERNELS_H
#define GPT2_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#include "gpt2_config.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t gpt2_half;

/* ---- host fp32 master weights (model/weights.h:9-29) ------------------------------------- */
typedef struct {
    float *ln1_g, *ln1_b;
    float *qkv_w, *qkv_b;             /* [2304,768], [2304] */
    float *attn_proj_w, *attn_proj_b; /* [768,768], [768] */
    float *ln2_g, *ln2_b;
    float *fc_w, *fc_b;               /* [3072,768], [3072] */
    float *proj_w, *proj_b;           /* [768,3072], [768] */
} GPT2Layer;

typedef struct {
    float *data;     /* owns the body when filled by gpt2_load_weights */
    size_t n_floats;
    float *wte;      /* [50257,768], also the tied output head */
    float *wpe;      /* [1024,768] */
    GPT2Layer layers[GPT2_N_LAYER];
    float *lnf_g, *lnf_b;
} GPT2Weights;

/* 'GPT2' v1 fp32 file (model/weights.c:13-61): 16 x int32 header {magic 0x47505432, version 1,
 * n_layer, n_head, n_embd, vocab, n_ctx, ffn, qkv, dtype 0, 0...}, then GPT2_TOTAL_PARAMS floats.
 * Returns 0 on success; 1 open, 2 short header, 3 magic/version, 4 dims, 5 dtype, 6 OOM, 7 short
 * body, 8 trailing bytes, 9 layout (the reference's codes). */
int gpt2_load_weights(const char *path, GPT2Weights *w);
void gpt2_free_weights(GPT2Weights *w);
/* Point every tensor of `w` into a caller-owned body of GPT2_TOTAL_PARAMS floats in file order
 * (no copy, no ownership).  Has no reference counterpart: it lets in-memory (synthetic) weights
 * use the same layout the loader produces.  Returns the number of floats the layout uses. */
size_t gpt2_bind_weights(GPT2Weights *w, float *body);

/* ---- fp16 device weights (cuda/kernels.cuh:20-23,41-48) ---------------------------------- */
typedef struct {
    gpt2_half *ln1_g, *ln1_b, *qkv_w, *qkv_b, *attn_proj_w, *attn_proj_b,
              *ln2_g, *ln2_b, *fc_w, *fc_b, *proj_w, *proj_b;
} GPT2LayerGPU;

/* one quantized tensor: q int8 [N,K] row-major, s fp32 [N] (cuda/kernels.cuh:28) */
typedef struct { const int8_t *q; const float *s; } GPT2QW;

typedef struct { GPT2QW qkv_w, attn_proj_w, fc_w, proj_w; } GPT2QLayerGPU;

typedef struct {
    int8_t *qdata;          /* owns all int8 codes (device) */
    float *sdata;           /* owns all scales (device) */
    size_t nq, ns;
    size_t streamed_bytes;  /* int8 bytes + 4*scales + 2*kept-fp16 elements: decode weight traffic */
    GPT2QW wte;             /* the tied head; q == NULL when it is kept fp16 */
    GPT2QLayerGPU layers[GPT2_N_LAYER];
} GPT2QWeightsGPU;

typedef struct {
    gpt2_half *data;        /* owns the whole fp16 body (device) */
    size_t n;
    gpt2_half *wte, *wpe;
    GPT2LayerGPU layers[GPT2_N_LAYER];
    gpt2_half *lnf_g, *lnf_b;
    const GPT2QWeightsGPU *q; /* NULL unless INT8 weights are attached */
} GPT2WeightsGPU;

/* fp32 master -> fp16 device blob, IEEE round-to-nearest-even (cuda/forward_cuda.cu:33-54).  The
 * conversion runs on the GPU; the tensor offsets equal the host body's. */
void gpt2_upload_fp16(const GPT2Weights *cpu, GPT2WeightsGPU *gpu);
void gpt2_free_gpu(GPT2WeightsGPU *gpu);

/* ---- activation scratch (cuda/kernels.cuh:54-56) ----------------------------------------- */
typedef struct { gpt2_half *x, *ln, *qkv, *att, *ao, *fc, *ff; int maxT; } GPT2ScratchGPU;
void gpt2_scratch_alloc(GPT2ScratchGPU *s, int maxT);
void gpt2_scratch_free(GPT2ScratchGPU *s);

/* ---- captures (cuda/kernels.cuh:64-65) --------------------------------------------------- */
struct GPT2KVCache;
typedef struct {
    gpt2_half *embed, *blocks, *final_ln, *logits;
    int logits_all;
    struct GPT2KVCache *kv;
} GPT2CapsGPU;

/* ---- the swappable backend table (cuda/kernels.cuh:68-86) -------------------------------- */
typedef struct {
    const char *name;
    void (*embed)(gpt2_half *x, const gpt2_half *wte, const gpt2_half *wpe, const int *ids, int T, int E);
    void (*layernorm)(gpt2_half *out, const gpt2_half *x, const gpt2_half *g, const gpt2_half *b, int M, int E);
    void (*matmul)(gpt2_half *C, const gpt2_half *A, const gpt2_half *W, const gpt2_half *bias, int M, int N, int K);
    void (*attention)(gpt2_half *att, const gpt2_half *qkv, int T, int E, int H, int D);
    void (*gelu)(gpt2_half *x, size_t n);
    void (*add)(gpt2_half *x, const gpt2_half *y, size_t n);
    void (*matmul_q)(gpt2_half *C, const gpt2_half *A, const int8_t *Wq, const float *Ws,
                     const gpt2_half *bias, int M, int N, int K);
    void (*gemv)(gpt2_half *C, const gpt2_half *A, const gpt2_half *W, const gpt2_half *bias, int N, int K);
    void (*gemv_q)(gpt2_half *C, const gpt2_half *A, const int8_t *Wq, const float *Ws,
                   const gpt2_half *bias, int N, int K);
} GPT2Backend;

/* Backends by the reference's names (cuda/kernels.cuh:88-92).  Here every one of them is built on
 * the MI355X kernels; they differ in which slots are filled, exactly as in the reference:
 *   naive  : one-thread-per-output matmul; no matmul_q / gemv / gemv_q
 *   tiled  : naive + the MFMA GEMM in .matmul
 *   flash  : tiled + the prefill attention kernel in .attention
 *   int8   : flash + .matmul_q (INT8 MFMA GEMM) + .gemv (fp16) + .gemv_q (INT8)
 *   gemv   : flash + .gemv (fp16) */
extern const GPT2Backend GPT2_BACKEND_NAIVE;
extern const GPT2Backend GPT2_BACKEND_TILED;
extern const GPT2Backend GPT2_BACKEND_FLASH;
extern const GPT2Backend GPT2_BACKEND_INT8;
extern const GPT2Backend GPT2_BACKEND_GEMV;

/* Prefill GEMM (replaces gpt2_matmul_tiled, cuda/kernels.cuh:96 / kernels_tiled.cu:48-53): fp16 MFMA
 * (v_mfma_f32_16x16x32_f16), LDS double-buffered tiles, per-shape tile table.  No alignment
 * preconditions: shapes or pointers the MFMA path cannot take run a generic LDS-tiled kernel. */
void gpt2_matmul_tiled(gpt2_half *C, const gpt2_half *A, const gpt2_half *W, const gpt2_half *bias,
                       int M, int N, int K);
/* Weight-only INT8 GEMM (replaces the file-static int8_matmul, cuda/kernels_quant.cu:62-67). */
void gpt2_matmul_int8(gpt2_half *C, const gpt2_half *A, const int8_t *Wq, const float *Ws,
                      const gpt2_half *bias, int M, int N, int K);
/* One thread per output, bias first (replaces naive_matmul, cuda/kernels_naive.cu:44-53,106-108). */
void gpt2_matmul_naive(gpt2_half *C, const gpt2_half *A, const gpt2_half *W, const gpt2_half *bias,
                       int M, int N, int K);
/* Causal prefill attention over qkv[T,3E] (replaces gpt2_attention_flash, cuda/kernels.cuh:98). */
void gpt2_attention_flash(gpt2_half *att, const gpt2_half *qkv, int T, int E, int H, int D);

/* Support ops (the naive backend's slots, cuda/kernels_naive.cu:17-97). */
void gpt2_embed(gpt2_half *x, const gpt2_half *wte, const gpt2_half *wpe, const int *ids, int T, int E);
void gpt2_layernorm(gpt2_half *out, const gpt2_half *x, const gpt2_half *g, const gpt2_half *b, int M, int E);
void gpt2_gelu(gpt2_half *x, size_t n);
void gpt2_add(gpt2_half *x, const gpt2_half *y, size_t n);

/* name in {naive, tiled, flash, int8, gemv}; NULL or unknown -> naive (cuda/kernels.cuh:101) */
const GPT2Backend *gpt2_backend_by_name(const char *name);

/* INT8 iff be->matmul_q && Wq && Wq->q, else fp16 (cuda/kernels.cuh:105-106, forward_cuda.cu:27-31) */
void gpt2_matmul_dispatch(const GPT2Backend *be, gpt2_half *C, const gpt2_half *A, const gpt2_half *Wh,
                          const GPT2QW *Wq, const gpt2_half *bias, int M, int N, int K);

/* ---- INT8 weights ------------------------------------------------------------------------ */
/* 'GPQ8' v2 file (cuda/kernels_quant.cu:87-155, tools/quantize.py:153-163): loads, uploads and
 * attaches to gpu->q.  Returns 0 on success, 1 on any format error. */
int gpt2_quant_load_upload(const char *path, GPT2WeightsGPU *gpu, GPT2QWeightsGPU *q);
void gpt2_quant_free(GPT2QWeightsGPU *q);
/* Loads GPT2_INT8_WEIGHTS (default weights/gpt2_124m_int8_kt.bin) iff be->matmul_q != NULL
 * (cuda/kernels.cuh:113, kernels_quant.cu:169-174). */
int gpt2_quant_attach_if_needed(const GPT2Backend *be, GPT2WeightsGPU *gpu, GPT2QWeightsGPU *q);
/* Quantizes the attached fp16 device weights on the GPU with tools/quantize.py's scheme
 * (tools/quantize.py:58-73: per output row, s = absmax/127 or 1 for a zero row,
 * q = clamp(rint(w/s), -127, 127)) and attaches the result to gpu->q, with no file.  keep[49] (may
 * be NULL) marks tensors left fp16, in the order wte, 12 x {qkv, attn_proj, fc, proj}; NULL keeps
 * only the head fp16 (the file the engine loads by default, weights/gpt2_124m_int8_kt.bin, is built
 * that way); all-zero keep quantizes the head too (quantize.py's own default, --fp16-keep none).  No
 * reference counterpart: it replaces the offline quantize.py + file round trip.  Returns 0 on
 * success. */
int gpt2_quant_build(GPT2WeightsGPU *gpu, GPT2QWeightsGPU *q, const int *keep);
/* Device quantizer of one fp16 [N,K] tensor (the kernel gpt2_quant_build runs per tensor). */
void gpt2_quantize_rows(int8_t *q, float *s, const gpt2_half *w, int N, int K);
/* Writes q/s as a 'GPQ8' v2 file for the attached weights; returns 0 on success. */
int gpt2_quant_write_file(const char *path, const GPT2QWeightsGPU *q, const int *keep);

/* ---- forward ----------------------------------------------------------------------------- */
/* cuda/kernels.cuh:116-117, forward_cuda.cu:77-116 */
void gpt2_forward_cuda(const GPT2Backend *be, const GPT2WeightsGPU *w, const int *d_ids, int T,
                       GPT2ScratchGPU *s, GPT2CapsGPU *caps);
/* No counterpart in the reference.  gpt2_forward_cuda without the scratch argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): it calls no allocator; the activations live in a static device array of
 * GPT2_NOALLOC_MAX_T tokens (2.25 MiB) that each GPU holds until the process ends.  T above the
 * limit records E_CAPACITY (gpt2_last_error) and launches nothing.  Every call on one GPU shares that
 * GPU's array, so calls that overlap on one GPU race. */
#define GPT2_NOALLOC_MAX_T 128
void gpt2_forward_noalloc(const GPT2Backend *be, const GPT2WeightsGPU *w, const int *d_ids, int T,
                          GPT2CapsGPU *caps);

/* ---- runtime: stream, errors, device memory (the cuda/common.cuh:17-66 helpers) ---------- */
/* Stream used by every launcher from now on (a hipStream_t; NULL = the null stream). */
void gpt2_set_stream(void *stream);
void *gpt2_get_stream(void);
/* First error since the last call (0 = none), then cleared.  Covers host-side argument checks
 * and HIP launch/runtime errors. */
int gpt2_last_error(void);
const char *gpt2_error_string(int code);
void *gpt2_dmalloc(size_t bytes);
void gpt2_dfree(void *p);
int gpt2_h2d(void *dst, const void *src, size_t bytes);
int gpt2_d2h(void *dst, const void *src, size_t bytes);
int gpt2_d2d(void *dst, const void *src, size_t bytes);
int gpt2_memset(void *dst, int value, size_t bytes);
int gpt2_sync(void);
/* fp32 -> fp16 (round to nearest even) on the GPU. */
void gpt2_f32_to_f16(gpt2_half *dst, const float *src, size_t n);

#ifdef __cplusplus
}
#endif
#endif
