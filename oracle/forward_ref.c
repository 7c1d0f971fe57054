/* forward_ref.c -- CPU fp32 GPT-2-124M forward, restated from the reference's cpu/forward_cpu.c.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).
 *
 * Numerics contract, which must hold bit-for-bit so that this file can stand in for the reference:
 *   - activations are stored as float; every reduction (matmul dot, LayerNorm moments, attention
 *     scores/softmax/context) accumulates in double and is rounded to float once at the end;
 *   - the matmul starts its accumulator at the bias and walks k upward (cpu/forward_cpu.c:46-47);
 *   - LayerNorm uses the biased variance of (x - mean) and adds (double)1e-5f inside the sqrt
 *     (cpu/forward_cpu.c:60-69);
 *   - gelu_new is 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))) in double (cpu/forward_cpu.c:74-78);
 *   - attention: scores scaled by 1/sqrt(64) = 0.125, max-subtracted exp, then context divided by
 *     the exp-sum (cpu/forward_cpu.c:83-116);
 *   - residual adds and the embedding sum are float adds (cpu/forward_cpu.c:132,144,150).
 * OpenMP splits only over independent outputs, so results do not depend on the thread count.
 * Build with -ffp-contract=off: a fused multiply-add would change the double roundings.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

size_t or_bind_weights(OrWeights *w, const float *flat) {
    /* Tensor order of the 'GPT2' v1 file body (model/weights.c:44-55). */
    const float *p = flat;
    const size_t E = OR_N_EMBD, V = OR_VOCAB, CX = OR_N_CTX, Q = OR_QKV, F = OR_FFN;
    w->wte = p; p += V * E;
    w->wpe = p; p += CX * E;
    for (int L = 0; L < OR_N_LAYER; ++L) {
        OrLayer *ly = &w->layers[L];
        ly->ln1_g = p; p += E;
        ly->ln1_b = p; p += E;
        ly->qkv_w = p; p += Q * E;
        ly->qkv_b = p; p += Q;
        ly->attn_proj_w = p; p += E * E;
        ly->attn_proj_b = p; p += E;
        ly->ln2_g = p; p += E;
        ly->ln2_b = p; p += E;
        ly->fc_w = p; p += F * E;
        ly->fc_b = p; p += F;
        ly->proj_w = p; p += E * F;
        ly->proj_b = p; p += E;
    }
    w->lnf_g = p; p += E;
    w->lnf_b = p; p += E;
    return (size_t)(p - flat);
}

/* cpu/forward_cpu.c:35-50 */
void or_matmul(float *C, const float *A, const float *W, const float *bias, int M, int N, int K) {
    const long total = (long)M * (long)N;
    long o;
#pragma omp parallel for schedule(static)
    for (o = 0; o < total; ++o) {
        const long row = o / N;
        const long col = o - row * N;
        const float *arow = A + (size_t)row * (size_t)K;
        const float *wrow = W + (size_t)col * (size_t)K;
        double sum = (bias != NULL) ? (double)bias[col] : 0.0;
        for (int k = 0; k < K; ++k) sum += (double)arow[k] * (double)wrow[k];
        C[o] = (float)sum;
    }
}

/* cpu/forward_cpu.c:53-71 (E is a parameter here; the reference fixes it at 768). */
void or_layernorm(float *out, const float *x, const float *g, const float *b, int M, int E) {
    int r;
#pragma omp parallel for schedule(static)
    for (r = 0; r < M; ++r) {
        const float *xr = x + (size_t)r * (size_t)E;
        float *yr = out + (size_t)r * (size_t)E;
        double mu = 0.0;
        for (int e = 0; e < E; ++e) mu += (double)xr[e];
        mu /= E;
        double var = 0.0;
        for (int e = 0; e < E; ++e) {
            const double c = (double)xr[e] - mu;
            var += c * c;
        }
        var /= E;
        const double rstd = 1.0 / sqrt(var + (double)OR_LN_EPS);
        for (int e = 0; e < E; ++e)
            yr[e] = (float)(((double)xr[e] - mu) * rstd * (double)g[e] + (double)b[e]);
    }
}

/* cpu/forward_cpu.c:74-78 */
float or_gelu_new(float xf) {
    const double x = (double)xf;
    const double z = 0.7978845608028654 * (x + 0.044715 * x * x * x);
    return (float)(0.5 * x * (1.0 + tanh(z)));
}

void or_gelu_inplace(float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = or_gelu_new(x[i]);
}

/* cpu/forward_cpu.c:83-116. qkv rows are [q | k | v], head h at columns [h*64, h*64+64). */
void or_attention(float *att, const float *qkv, int T) {
    const int E = OR_N_EMBD, D = OR_HEAD_DIM, S = OR_QKV;
    const double scale = 1.0 / sqrt((double)D);
    const long pairs = (long)OR_N_HEAD * T;
    long hq;
#pragma omp parallel for schedule(static)
    for (hq = 0; hq < pairs; ++hq) {
        const int h = (int)(hq / T);
        const int i = (int)(hq - (long)h * T);
        const float *q = qkv + (size_t)i * S + h * D;
        double p[OR_N_CTX];
        double top = -1e300;
        for (int j = 0; j <= i; ++j) {
            const float *k = qkv + (size_t)j * S + E + h * D;
            double dot = 0.0;
            for (int d = 0; d < D; ++d) dot += (double)q[d] * (double)k[d];
            dot *= scale;
            p[j] = dot;
            if (dot > top) top = dot;
        }
        double denom = 0.0;
        for (int j = 0; j <= i; ++j) {
            p[j] = exp(p[j] - top);
            denom += p[j];
        }
        const double rden = 1.0 / denom;
        double ctx[OR_HEAD_DIM];
        for (int d = 0; d < D; ++d) ctx[d] = 0.0;
        for (int j = 0; j <= i; ++j) {
            const float *v = qkv + (size_t)j * S + 2 * E + h * D;
            for (int d = 0; d < D; ++d) ctx[d] += p[j] * (double)v[d];
        }
        float *o = att + (size_t)i * E + h * D;
        for (int d = 0; d < D; ++d) o[d] = (float)(ctx[d] * rden);
    }
}

/* cpu/forward_cpu.c:118-166 */
void or_forward(const OrWeights *w, const int *ids, int T, float *embed, float *blocks,
                float *final_ln, float *logits, int logits_all) {
    const size_t E = OR_N_EMBD, Q = OR_QKV, F = OR_FFN;
    const size_t TE = (size_t)T * E;
    float *x = (float *)malloc(TE * sizeof(float));
    float *ln = (float *)malloc(TE * sizeof(float));
    float *qkv = (float *)malloc((size_t)T * Q * sizeof(float));
    float *att = (float *)malloc(TE * sizeof(float));
    float *ao = (float *)malloc(TE * sizeof(float));
    float *fc = (float *)malloc((size_t)T * F * sizeof(float));
    float *ff = (float *)malloc(TE * sizeof(float));

    for (int t = 0; t < T; ++t) {
        const float *te = w->wte + (size_t)ids[t] * E;
        const float *pe = w->wpe + (size_t)t * E;
        for (size_t e = 0; e < E; ++e) x[(size_t)t * E + e] = te[e] + pe[e];
    }
    if (embed) memcpy(embed, x, TE * sizeof(float));

    for (int L = 0; L < OR_N_LAYER; ++L) {
        const OrLayer *ly = &w->layers[L];
        or_layernorm(ln, x, ly->ln1_g, ly->ln1_b, T, (int)E);
        or_matmul(qkv, ln, ly->qkv_w, ly->qkv_b, T, (int)Q, (int)E);
        or_attention(att, qkv, T);
        or_matmul(ao, att, ly->attn_proj_w, ly->attn_proj_b, T, (int)E, (int)E);
        for (size_t i = 0; i < TE; ++i) x[i] += ao[i];
        or_layernorm(ln, x, ly->ln2_g, ly->ln2_b, T, (int)E);
        or_matmul(fc, ln, ly->fc_w, ly->fc_b, T, (int)F, (int)E);
        or_gelu_inplace(fc, (size_t)T * F);
        or_matmul(ff, fc, ly->proj_w, ly->proj_b, T, (int)E, (int)F);
        for (size_t i = 0; i < TE; ++i) x[i] += ff[i];
        if (blocks) memcpy(blocks + (size_t)L * TE, x, TE * sizeof(float));
    }

    or_layernorm(ln, x, w->lnf_g, w->lnf_b, T, (int)E);
    if (final_ln) memcpy(final_ln, ln, TE * sizeof(float));
    if (logits) {
        if (logits_all)
            or_matmul(logits, ln, w->wte, NULL, T, OR_VOCAB, (int)E);
        else
            or_matmul(logits, ln + (size_t)(T - 1) * E, w->wte, NULL, 1, OR_VOCAB, (int)E);
    }
    free(x); free(ln); free(qkv); free(att); free(ao); free(fc); free(ff);
}
