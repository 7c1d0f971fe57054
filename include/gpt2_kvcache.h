/* gpt2_kvcache.h -- KV cache, M=1 GEMVs and the decode step.  Replaces cuda/kvcache.cuh:139-215
 * (same names, layouts and parameter order; C linkage; gpt2_half for CUDA's half), and adds the
 * graph-captured decode loop.
 *
 * GEMV contract (cuda/kvcache.cuh:206-208):  C[1,N] = A[1,K] . W[N,K]^T + bias[N]
 *   INT8:  C[n] = s[n] * sum_k A[k] q[n,k] + bias[n]
 * The reference needs K even (fp16) / K % 4 == 0 (INT8) (cuda/kvcache.cu:160,185).  Here any K works:
 * K % 8 == 0 (fp16) / K % 16 == 0 (INT8) with 16-byte aligned rows take the vector kernels, the rest
 * a generic kernel.
 */
#ifndef GPT2_KVCACHE_H
#define GPT2_KVCACHE_H

#include "gpt2_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One arena [L][K|V][H][maxT][D] fp16 (cuda/kvcache.cuh:158-163). */
typedef struct GPT2KVCache {
    gpt2_half *data;
    size_t bytes;
    int maxT, nLayer, nHead, headDim;
    int len; /* positions cached, [0, len) */
} GPT2KVCache;

/* 0 on success; 1 if the arena plus 64 MiB of headroom does not fit (cuda/kvcache.cu:29-46). */
int gpt2_kv_alloc(GPT2KVCache *kv, int maxT);
void gpt2_kv_scatter_prefill(GPT2KVCache *kv, int L, const gpt2_half *qkv, int T);
void gpt2_embed_one(gpt2_half *x, const gpt2_half *wte, const gpt2_half *wpe, int token, int pos);
void gpt2_kv_append_one(GPT2KVCache *kv, int L, const gpt2_half *qkv, int pos);
void gpt2_attn_decode(gpt2_half *att, const gpt2_half *qkv, const GPT2KVCache *kv, int L, int len);
void gpt2_kv_free(GPT2KVCache *kv);
void gpt2_kv_reset(GPT2KVCache *kv);
double gpt2_kv_step_bytes(const GPT2KVCache *kv, int len);

static inline gpt2_half *gpt2_kv_K(const GPT2KVCache *kv, int L) {
    return kv->data + (size_t)(2 * L + 0) * kv->nHead * kv->maxT * kv->headDim;
}
static inline gpt2_half *gpt2_kv_V(const GPT2KVCache *kv, int L) {
    return kv->data + (size_t)(2 * L + 1) * kv->nHead * kv->maxT * kv->headDim;
}

/* One token at `pos`; requires kv->len == pos, leaves kv->len == pos+1 (cuda/kvcache.cuh:193-195).
 * caps_blocks (optional) holds GPT2_DECODE_CAPS_ROWS x E: per-block hidden, final_ln, embed. */
#define GPT2_DECODE_CAPS_ROWS (GPT2_N_LAYER + 2)
void gpt2_decode_step_cuda(const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv, int token,
                           int pos, GPT2ScratchGPU *s, gpt2_half *logits, gpt2_half *caps_blocks);
void gpt2_prefill_fill_cache(const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv,
                             const int *d_ids, int T, GPT2ScratchGPU *s, GPT2CapsGPU *caps);

/* M=1 GEMVs (cuda/kvcache.cuh:206-208): 128-bit weight loads, fp32 accumulation, wave64 DPP
 * reductions, per-row scale then bias. */
void gpt2_gemv_fp16(gpt2_half *C, const gpt2_half *A, const gpt2_half *W, const gpt2_half *bias, int N, int K);
void gpt2_gemv_int8(gpt2_half *C, const gpt2_half *A, const int8_t *Wq, const float *Ws,
                    const gpt2_half *bias, int N, int K);
/* gemv_q if quantized, else gemv, else the backend's M=1 matmul (cuda/kvcache.cuh:212-213) */
void gpt2_gemv_dispatch(const GPT2Backend *be, gpt2_half *C, const gpt2_half *A, const gpt2_half *Wh,
                        const GPT2QW *Wq, const gpt2_half *bias, int N, int K);

/* ---- graph-captured greedy decode (no reference counterpart; replaces the host loop around
 * gpt2_decode_step_cuda in bench/bench_decode.cu:101-102 and bench/kv_gate.cu:67-79) ----------
 * The step (the same kernels as gpt2_decode_step_cuda with the backend's GEMV choice) is captured
 * once into a hipGraph on a private stream.  The current token and position live in device memory,
 * so one instantiated graph replays every step: each replay appends K/V at pos, writes logits[V],
 * picks the greedy next token (lowest index among equal maxima), stores it in tokens[pos+1] and
 * advances pos.  `tokens` is a device int array of at least kv->maxT entries. */
typedef struct GPT2DecodeGraph GPT2DecodeGraph;
GPT2DecodeGraph *gpt2_decode_graph_create(const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv,
                                          GPT2ScratchGPU *s, gpt2_half *logits, int *tokens);
/* How the captured step runs:
 *   GPT2_DECODE_MULTI       the step's kernels one after another (~62 launches per token);
 *   GPT2_DECODE_PERSISTENT  one persistent kernel per token: 256 work-groups run every phase of the
 *                           step and exchange the small activation vectors through coherent
 *                           flag words instead of kernel boundaries.  Needs this library's GEMV
 *                           backend slots (int8 / gemv backends) and the GPU to itself while a step
 *                           runs (its work-groups must be resident together; if they are not, the
 *                           step gives up after a bounded wait and gpt2_decode_graph_sync reports
 *                           an error).  Being one kernel per token, 16 consecutive steps are
 *                           captured as one graph (one replay decodes 16 tokens); single steps and
 *                           the rest of a run are launched directly on the private stream;
 *   GPT2_DECODE_AUTO        persistent when the backend allows it (env GPT2_DECODE_PERSISTENT=0
 *                           forces the multi-kernel step).
 * gpt2_decode_graph_create uses GPT2_DECODE_AUTO.  No reference counterpart. */
#define GPT2_DECODE_AUTO (-1)
#define GPT2_DECODE_MULTI 0
#define GPT2_DECODE_PERSISTENT 1
GPT2DecodeGraph *gpt2_decode_graph_create_mode(const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv,
                                               GPT2ScratchGPU *s, gpt2_half *logits, int *tokens, int mode);
/* The mode the graph actually runs (a persistent request falls back to GPT2_DECODE_MULTI). */
int gpt2_decode_graph_mode(const GPT2DecodeGraph *g);
/* Set the device-side state: next step consumes `token` at position `pos` (kv must hold pos rows). */
int gpt2_decode_graph_set(GPT2DecodeGraph *g, int token, int pos);
/* Replay `steps` steps back to back on the graph's stream; no host synchronisation inside. Steps
 * past kv->maxT-1 are refused (returns nonzero, nothing launched). */
int gpt2_decode_graph_run(GPT2DecodeGraph *g, int steps);
/* Wait for the graph's stream, read the device state back, set kv->len = pos. */
int gpt2_decode_graph_sync(GPT2DecodeGraph *g, int *token, int *pos);
void gpt2_decode_graph_destroy(GPT2DecodeGraph *g);

#ifdef __cplusplus
}
#endif
#endif
