/* oracle.h -- CPU restatement of bare-metal-gpt2's matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or calls this code: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as the checker.
 *
 * What it restates (reference file:line):
 *   or_matmul        cpu/forward_cpu.c:35-50    C = A.W^T + b, float storage, double accumulation,
 *                                               bias first, k ascending, OpenMP over flattened M*N
 *   or_layernorm     cpu/forward_cpu.c:53-71    biased variance, eps 1e-5 inside the sqrt, double
 *   or_gelu_new      cpu/forward_cpu.c:74-78    tanh form, double
 *   or_attention     cpu/forward_cpu.c:83-116   causal MHA over qkv[T,3E], scale 1/sqrt(64), double
 *   or_forward       cpu/forward_cpu.c:118-166  op order, residuals, ln_f, tied head, logits_all
 *   or_f32_to_f16    cuda/forward_cuda.cu:36 and tools/quantize.py:109 (IEEE round-to-nearest-even)
 *   or_quantize_rows tools/quantize.py:58-73    symmetric per-output-row INT8 of the fp16 view
 *   or_dequantize    tools/quantize.py:65, tools/dequant_check.py:65   fl32((float)q * s)
 *
 * How each is pinned (tests/test_oracle_*.py):
 *   - or_matmul / or_layernorm / or_gelu_new / or_attention / or_forward: bit-exact against the
 *     reference's own cpu/forward_cpu.c compiled from /root/reference into oracle/_ref/ (when it is
 *     buildable), against committed golden vectors written from that build (tests/golden/), and
 *     against closed forms (one-hot and small-integer matmuls, constant-row LayerNorm, the sigmoid
 *     form of gelu_new, T=1 and equal-key attention, causality).
 *   - or_f32_to_f16 / or_f16_to_f32: exhaustively over all 2^32 float patterns against the host's
 *     F16C VCVTPS2PH / VCVTPH2PS instructions.
 *   - or_quantize_rows: closed-form invariants (|q|<=127, absmax row element at |q|=127, odd
 *     symmetry, dead row -> s=1,q=0, exact ties round half to even), a long-double brute force, and
 *     golden vectors written by the reference's own tools/quantize.py:quantize_rows.
 */
#ifndef GPT2_ORACLE_H
#define GPT2_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GPT-2-124M dimensions (model/config.h:11-19). */
#define OR_N_LAYER 12
#define OR_N_HEAD 12
#define OR_N_EMBD 768
#define OR_VOCAB 50257
#define OR_N_CTX 1024
#define OR_HEAD_DIM 64
#define OR_FFN 3072
#define OR_QKV 2304
#define OR_LN_EPS 1e-5f
#define OR_TOTAL_PARAMS 124439808L

/* Per-layer tensor pointers, in the order the fp32 weight file lays them out (model/weights.c:44-55). */
typedef struct {
    const float *ln1_g, *ln1_b, *qkv_w, *qkv_b, *attn_proj_w, *attn_proj_b;
    const float *ln2_g, *ln2_b, *fc_w, *fc_b, *proj_w, *proj_b;
} OrLayer;

typedef struct {
    const float *wte, *wpe;
    OrLayer layers[OR_N_LAYER];
    const float *lnf_g, *lnf_b;
} OrWeights;

/* Bind an OrWeights view onto one flat buffer of OR_TOTAL_PARAMS floats in file order.
 * Returns the number of floats consumed (== OR_TOTAL_PARAMS). */
size_t or_bind_weights(OrWeights *w, const float *flat);

void or_matmul(float *C, const float *A, const float *W, const float *bias, int M, int N, int K);
void or_layernorm(float *out, const float *x, const float *g, const float *b, int M, int E);
float or_gelu_new(float x);
void or_gelu_inplace(float *x, size_t n);
void or_attention(float *att, const float *qkv, int T);

/* Forward over ids[0..T-1]. Any NULL capture is skipped.
 *   embed [T*E], blocks [12*T*E], final_ln [T*E], logits [T*V] (logits_all) or [V] (last row). */
void or_forward(const OrWeights *w, const int *ids, int T, float *embed, float *blocks,
                float *final_ln, float *logits, int logits_all);

/* IEEE binary32 <-> binary16, round to nearest even, subnormals and inf/NaN handled. */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);
void or_f32_to_f16_array(uint16_t *dst, const float *src, size_t n);
void or_f16_to_f32_array(float *dst, const uint16_t *src, size_t n);

/* Symmetric per-output-row INT8 of an fp16-valued [N,K] fp32 matrix (values already fp16-rounded).
 * Returns the number of dead (all-zero) rows. */
int or_quantize_rows(int8_t *q, float *s, const float *w16, int N, int K);
/* fp16 view + quantize in one call: w32 -> fl32(fl16_RNE(w32)) -> or_quantize_rows. */
int or_quantize_fp16_view(int8_t *q, float *s, const float *w32, int N, int K);
void or_dequantize(float *w, const int8_t *q, const float *s, int N, int K);

/* Test-only helpers (pinning the above, not part of the restatement). */
/* Exhaustive comparison of or_f32_to_f16 / or_f16_to_f32 with the F16C instructions over the
 * 32-bit pattern range [lo, hi). Returns the number of mismatches; *first gets the first one. */
uint64_t or_check_f16c_range(uint64_t lo, uint64_t hi, uint32_t *first);
uint64_t or_check_f16c_back(void);
/* Long-double second implementation of the quantizer, for brute-force cross-checks. */
int or_quantize_rows_ld(int8_t *q, float *s, const float *w16, int N, int K);

#ifdef __cplusplus
}
#endif
#endif
