// engine.hip -- host side of the matmul path: backend table and dispatch, fp16 upload, scratch,
// prefill forward, KV cache, the decode step and its hipGraph replay, and the two weight formats.
//
// Call order and data flow follow the reference host code (cuda/forward_cuda.cu, cuda/kvcache.cu,
// cuda/kernels_quant.cu, model/weights.c); everything runs on the stream set by gpt2_set_stream.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"
#include "decode.h"
#include "prefill.h"

namespace g2 {
void gemv(uint16_t *C, const uint16_t *x, const void *W, const float *Ws, const uint16_t *bias, int N, int K, bool qw,
          int cfg);
void embed_one(uint16_t *x, const uint16_t *wte, const uint16_t *wpe, StepArg st);
bool gemm_fused(uint16_t *C, const uint16_t *A, const void *W, const float *Ws, const uint16_t *bias, int M, int N,
                int K, bool qw, int epi, const uint16_t *resid);
bool gemm_ln(uint16_t *C, const uint16_t *X, const uint16_t *ln_g, const uint16_t *ln_b, const void *W,
             const float *Ws, const uint16_t *bias, int M, int N, int K, bool qw, int epi, int cfg);
void attention_prefill(uint16_t *att, const uint16_t *qkv, int T, uint16_t *Kc, uint16_t *Vc, int maxT);
void kv_append(uint16_t *K, uint16_t *V, const uint16_t *qkv, StepArg st, int maxT);
void attn_decode(uint16_t *att, const uint16_t *qkv, const uint16_t *K, const uint16_t *V, int maxT, StepArg st,
                 int len_imm);
void argmax_advance(const uint16_t *logits, int V, int *state, int *tokens, int max_pos);
void attn_decode_append(uint16_t *att, const uint16_t *qkv, uint16_t *K, uint16_t *V, int maxT, StepArg st);
bool gemv_fused(uint16_t *C, const uint16_t *x, const void *W, const float *Ws, const uint16_t *bias, int N, int K,
                bool qw, const uint16_t *ln_g, const uint16_t *ln_b, int epi, const uint16_t *resid);
int gemm_ln_forced();
bool gemm_skinny(uint16_t *C, const uint16_t *A, const void *W, const float *Ws, const uint16_t *bias, int M, int N,
                 int K, bool qw, int epi, const uint16_t *resid, const uint16_t *ln_g, const uint16_t *ln_b);
int skinny_max_m(bool qw);
bool gemm_lnfold(int epi, uint16_t *C, const uint16_t *A, const void *W, const float *Ws, const uint16_t *bias, int M,
                 int N, int K, bool qw, const uint16_t *resid, const LnFold &lf);
void embed_lnf(uint16_t *x, uint16_t *xg, float2 *stats, const uint16_t *wte, const uint16_t *wpe, const int *ids,
               int T, const uint16_t *gamma);
void ln_fold_consts(float2 *gh, const void *W, const float *Ws, const uint16_t *gamma, const uint16_t *beta, int N,
                    int K, bool qw);
}  // namespace g2

using namespace g2;

// ============================================================================ backends
// Composed exactly like the reference's (cuda/kernels_quant.cu:190-200, kvcache.cu:282-290): each
// stage fills more slots.  All members are addresses of extern "C" functions, so the tables are
// constant-initialized.  They exist in the host pass only (the device pass would otherwise treat
// these const globals as __constant__ data referring to host functions).
#if !defined(__HIP_DEVICE_COMPILE__)
extern "C" const GPT2Backend GPT2_BACKEND_NAIVE = {
    "naive", gpt2_embed, gpt2_layernorm, gpt2_matmul_naive, gpt2_attention_flash, gpt2_gelu, gpt2_add,
    nullptr, nullptr, nullptr};
extern "C" const GPT2Backend GPT2_BACKEND_TILED = {
    "tiled", gpt2_embed, gpt2_layernorm, gpt2_matmul_tiled, gpt2_attention_flash, gpt2_gelu, gpt2_add,
    nullptr, nullptr, nullptr};
extern "C" const GPT2Backend GPT2_BACKEND_FLASH = {
    "flash", gpt2_embed, gpt2_layernorm, gpt2_matmul_tiled, gpt2_attention_flash, gpt2_gelu, gpt2_add,
    nullptr, nullptr, nullptr};
extern "C" const GPT2Backend GPT2_BACKEND_INT8 = {
    "int8", gpt2_embed, gpt2_layernorm, gpt2_matmul_tiled, gpt2_attention_flash, gpt2_gelu, gpt2_add,
    gpt2_matmul_int8, gpt2_gemv_fp16, gpt2_gemv_int8};
extern "C" const GPT2Backend GPT2_BACKEND_GEMV = {
    "gemv", gpt2_embed, gpt2_layernorm, gpt2_matmul_tiled, gpt2_attention_flash, gpt2_gelu, gpt2_add,
    nullptr, gpt2_gemv_fp16, nullptr};
#endif

extern "C" const GPT2Backend *gpt2_backend_by_name(const char *name) {
    if (!name) return &GPT2_BACKEND_NAIVE;
    if (!strcmp(name, "tiled")) return &GPT2_BACKEND_TILED;
    if (!strcmp(name, "flash")) return &GPT2_BACKEND_FLASH;
    if (!strcmp(name, "int8")) return &GPT2_BACKEND_INT8;
    if (!strcmp(name, "gemv")) return &GPT2_BACKEND_GEMV;
    return &GPT2_BACKEND_NAIVE;
}

extern "C" void gpt2_matmul_dispatch(const GPT2Backend *be, gpt2_half *C, const gpt2_half *A, const gpt2_half *Wh,
                                     const GPT2QW *Wq, const gpt2_half *bias, int M, int N, int K) {
    if (be->matmul_q && Wq && Wq->q) be->matmul_q(C, A, Wq->q, Wq->s, bias, M, N, K);
    else be->matmul(C, A, Wh, bias, M, N, K);
}

extern "C" void gpt2_gemv_dispatch(const GPT2Backend *be, gpt2_half *C, const gpt2_half *A, const gpt2_half *Wh,
                                   const GPT2QW *Wq, const gpt2_half *bias, int N, int K) {
    if (be->gemv_q && Wq && Wq->q) be->gemv_q(C, A, Wq->q, Wq->s, bias, N, K);
    else if (be->gemv) be->gemv(C, A, Wh, bias, N, K);
    else gpt2_matmul_dispatch(be, C, A, Wh, Wq, bias, 1, N, K);
}

// ============================================================================ host fp32 weights
static const int kMagicW = 0x47505432;  // 'GPT2'
static const int kMagicQ = 0x38515047;  // 'GPQ8'

extern "C" size_t gpt2_bind_weights(GPT2Weights *w, float *body) {
    // tensor order of the file body (model/weights.c:44-55)
    const size_t E = GPT2_N_EMBD, V = GPT2_VOCAB, CX = GPT2_N_CTX, Q = GPT2_QKV_DIM, F = GPT2_FFN_DIM;
    float *c = body;
    auto take = [&](size_t n) { float *p = c; c += n; return p; };
    w->data = body;
    w->n_floats = (size_t)GPT2_TOTAL_PARAMS;
    w->wte = take(V * E);
    w->wpe = take(CX * E);
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        GPT2Layer *l = &w->layers[L];
        l->ln1_g = take(E); l->ln1_b = take(E);
        l->qkv_w = take(Q * E); l->qkv_b = take(Q);
        l->attn_proj_w = take(E * E); l->attn_proj_b = take(E);
        l->ln2_g = take(E); l->ln2_b = take(E);
        l->fc_w = take(F * E); l->fc_b = take(F);
        l->proj_w = take(E * F); l->proj_b = take(E);
    }
    w->lnf_g = take(E);
    w->lnf_b = take(E);
    return (size_t)(c - body);
}

// A loader's diagnostic on stderr (the return code carries the reason to the caller).
static int load_reject(const char *loader, const char *path, const char *why, int code) {
    fprintf(stderr, "%s: %s: %s\n", loader, path, why);
    return code;
}

extern "C" int gpt2_load_weights(const char *path, GPT2Weights *w) {
    static const char *me = "gpt2_load_weights";
    memset(w, 0, sizeof(*w));
    FILE *f = fopen(path, "rb");
    if (!f) return load_reject(me, path, "cannot be opened for reading", 1);
    int32_t head[16];
    const bool whole = fread(head, 4, 16, f) == 16;
    if (!whole) { fclose(f); return load_reject(me, path, "the file ends inside its 64-byte header", 2); }
    if (head[0] != kMagicW || head[1] != 1) { fclose(f); return load_reject(me, path, "not a 'GPT2' version 1 file", 3); }
    const int32_t dims[7] = {GPT2_N_LAYER, GPT2_N_HEAD, GPT2_N_EMBD, GPT2_VOCAB, GPT2_N_CTX, GPT2_FFN_DIM, GPT2_QKV_DIM};
    if (memcmp(head + 2, dims, sizeof dims) != 0) {
        fclose(f);
        return load_reject(me, path, "its model dimensions are not GPT-2-124M's", 4);
    }
    if (head[9] != 0) { fclose(f); return load_reject(me, path, "its tensors are not stored as fp32", 5); }
    const size_t n = (size_t)GPT2_TOTAL_PARAMS;
    float *body = (float *)malloc(n * sizeof(float));
    if (!body) { fclose(f); return 6; }
    const size_t got = fread(body, sizeof(float), n, f);
    const long at = ftell(f);
    fseek(f, 0, SEEK_END);
    const long past_end = ftell(f) - at;
    fclose(f);
    if (got != n) { free(body); return load_reject(me, path, "the file ends inside the tensor data", 7); }
    if (past_end != 0) { free(body); return load_reject(me, path, "bytes follow the last tensor", 8); }
    if (gpt2_bind_weights(w, body) != n) { free(body); memset(w, 0, sizeof(*w)); return 9; }
    return 0;
}

extern "C" void gpt2_free_weights(GPT2Weights *w) {
    if (w && w->data) {
        free(w->data);
        w->data = nullptr;
    }
}

// ============================================================================ fp16 upload
extern "C" void gpt2_upload_fp16(const GPT2Weights *cpu, GPT2WeightsGPU *gpu) {
    memset(gpu, 0, sizeof(*gpu));
    if (!cpu || !cpu->data || cpu->n_floats == 0) { arg_fail("gpt2_upload_fp16: no host body"); return; }
    const size_t n = cpu->n_floats;
    uint16_t *dst = (uint16_t *)gpt2_dmalloc(n * 2);
    if (!dst) return;
    // Stage the fp32 body through one bounded device buffer and convert on the GPU.
    const size_t chunk = (size_t)32 << 20;   // floats per pass (128 MiB)
    float *stage = (float *)gpt2_dmalloc((n < chunk ? n : chunk) * 4);
    if (!stage) { gpt2_dfree(dst); return; }
    for (size_t off = 0; off < n; off += chunk) {
        const size_t m = (n - off < chunk) ? n - off : chunk;
        if (gpt2_h2d(stage, cpu->data + off, m * 4)) break;
        gpt2_f32_to_f16(dst + off, stage, m);
        gpt2_sync();
    }
    gpt2_dfree(stage);
    gpu->data = dst;
    gpu->n = n;
    auto OFF = [&](const float *p) { return dst + (p - cpu->data); };
    gpu->wte = OFF(cpu->wte);
    gpu->wpe = OFF(cpu->wpe);
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        const GPT2Layer *c = &cpu->layers[L];
        GPT2LayerGPU *g = &gpu->layers[L];
        g->ln1_g = OFF(c->ln1_g); g->ln1_b = OFF(c->ln1_b);
        g->qkv_w = OFF(c->qkv_w); g->qkv_b = OFF(c->qkv_b);
        g->attn_proj_w = OFF(c->attn_proj_w); g->attn_proj_b = OFF(c->attn_proj_b);
        g->ln2_g = OFF(c->ln2_g); g->ln2_b = OFF(c->ln2_b);
        g->fc_w = OFF(c->fc_w); g->fc_b = OFF(c->fc_b);
        g->proj_w = OFF(c->proj_w); g->proj_b = OFF(c->proj_b);
    }
    gpu->lnf_g = OFF(cpu->lnf_g);
    gpu->lnf_b = OFF(cpu->lnf_b);
    gpu->q = nullptr;
}

static void fold_consts_drop(const void *wdata, const void *qdata);

extern "C" void gpt2_free_gpu(GPT2WeightsGPU *g) {
    if (g && g->data) {
        fold_consts_drop(g->data, nullptr);
        gpt2_dfree(g->data);
        g->data = nullptr;
    }
}

extern "C" void gpt2_scratch_alloc(GPT2ScratchGPU *s, int maxT) {
    memset(s, 0, sizeof(*s));
    if (maxT <= 0) { arg_fail("gpt2_scratch_alloc: maxT <= 0"); return; }
    s->maxT = maxT;
    const size_t E = GPT2_N_EMBD, Q = GPT2_QKV_DIM, F = GPT2_FFN_DIM, T = (size_t)maxT;
    s->x = (gpt2_half *)gpt2_dmalloc(T * E * 2);
    s->ln = (gpt2_half *)gpt2_dmalloc(T * E * 2);
    s->qkv = (gpt2_half *)gpt2_dmalloc(T * Q * 2);
    s->att = (gpt2_half *)gpt2_dmalloc(T * E * 2);
    s->ao = (gpt2_half *)gpt2_dmalloc(T * E * 2);
    s->fc = (gpt2_half *)gpt2_dmalloc(T * F * 2);
    s->ff = (gpt2_half *)gpt2_dmalloc(T * E * 2);
}

extern "C" void gpt2_scratch_free(GPT2ScratchGPU *s) {
    gpt2_dfree(s->x); gpt2_dfree(s->ln); gpt2_dfree(s->qkv); gpt2_dfree(s->att);
    gpt2_dfree(s->ao); gpt2_dfree(s->fc); gpt2_dfree(s->ff);
    memset(s, 0, sizeof(*s));
}

// ============================================================================ prefill forward
static void capcpy(gpt2_half *dst, const gpt2_half *src, size_t n) { gpt2_d2d(dst, src, n * 2); }

// When the backend's matmul, gelu, add and attention slots are this library's, the prefill runs
// fused: gelu in the fc GEMM's epilogue, the residual adds in the attn-proj and mlp-proj epilogues,
// the K/V cache fill inside the attention launch -- 5 launches per layer instead of 9, each result
// bit-identical to the unfused sequence (same fp16 rounding points; the LayerNorm fold below, taken
// by default for short prompts, is the exception).  Other backends, and shapes the fused GEMM does
// not take, run the reference's sequence (cuda/forward_cuda.cu:90-106).
static bool g_prefill_fused = true;   // gpt2_tune_prefill_fused (tests compare both sequences)
static bool fused_prefill_ok(const GPT2Backend *be) {
    return g_prefill_fused && be->matmul == gpt2_matmul_tiled &&
           (be->matmul_q == nullptr || be->matmul_q == gpt2_matmul_int8) && be->gelu == gpt2_gelu && be->add == gpt2_add;
}

// Tuning/test hook (not part of the reference interface): 0 makes every prefill run the unfused
// reference sequence, 1 (the default) restores the fused one.
extern "C" void gpt2_tune_prefill_fused(int on) { g_prefill_fused = on != 0; }

// One prefill matmul site followed by `epi` (gelu in place, or C = resid + product): fused when
// allowed and the GEMM takes it, else the backend's matmul into `tmp` (EPI_RESID) or C, then gelu/add.
static void matmul_site(const GPT2Backend *be, bool fused, gpt2_half *C, const gpt2_half *A, const gpt2_half *Wh,
                        const GPT2QW *Wq, const gpt2_half *bias, int M, int N, int K, int epi, gpt2_half *tmp) {
    const bool q = be->matmul_q && Wq && Wq->q;
    if (fused && gemm_fused(C, A, q ? (const void *)Wq->q : (const void *)Wh, q ? Wq->s : nullptr, bias, M, N, K, q,
                            epi, epi == EPI_RESID ? C : nullptr))
        return;
    if (epi == EPI_RESID) {
        gpt2_matmul_dispatch(be, tmp, A, Wh, Wq, bias, M, N, K);
        be->add(C, tmp, (size_t)M * N);
    } else {
        gpt2_matmul_dispatch(be, C, A, Wh, Wq, bias, M, N, K);
        if (epi == EPI_GELU) be->gelu(C, (size_t)M * N);
    }
}

// LayerNorm(X) followed by a matmul site (QKV: no epilogue; fc: gelu), when the fused prefill may
// fuse them (ln_fuse also requires this library's LayerNorm, whose arithmetic both fused forms repeat
// bit for bit): one LayerNorm-panel GEMM launch when a panel config is forced
// (gpt2_tune_gemm_ln_force; off by default, slower than the two launches); else, for a few rows, the
// skinny GEMM with its LayerNorm prologue; else the backend's LayerNorm into lnbuf, then the site.
static void ln_matmul_site(const GPT2Backend *be, bool fused, bool ln_fuse, gpt2_half *C, const gpt2_half *X,
                           const gpt2_half *ln_g, const gpt2_half *ln_b, gpt2_half *lnbuf, const gpt2_half *Wh,
                           const GPT2QW *Wq, const gpt2_half *bias, int M, int N, int K, int epi) {
    const bool q = be->matmul_q && Wq && Wq->q;
    const void *W = q ? (const void *)Wq->q : (const void *)Wh;
    if (ln_fuse && gemm_ln(C, X, ln_g, ln_b, W, q ? Wq->s : nullptr, bias, M, N, K, q, epi, -1)) return;
    if (ln_fuse && gemm_ln_forced() < 0 &&
        gemm_skinny(C, X, W, q ? Wq->s : nullptr, bias, M, N, K, q, epi, nullptr, ln_g, ln_b))
        return;
    be->layernorm(lnbuf, X, ln_g, ln_b, M, K);
    if (epi == EPI_NONE) gpt2_matmul_dispatch(be, C, lnbuf, Wh, Wq, bias, M, N, K);
    else matmul_site(be, fused, C, lnbuf, Wh, Wq, bias, M, N, K, epi, nullptr);
}

// ---------------------------------------------------------------------------- LayerNorm fold
// The fused prefill folds LN1 and LN2 into the GEMMs that consume them.  With mu, rstd the row's
// mean and 1/sqrt(var + eps) and x*gamma the row scaled by the LayerNorm's gamma,
//     LayerNorm(x) . W_n = rstd (x*gamma . W_n - mu G_n) + H_n,  G_n = sum_k gamma_k W_nk,
//                                                                H_n = sum_k beta_k W_nk,
// so the GEMM producing x (the embedding, attn-proj, mlp-proj) also writes x*gamma of the next
// LayerNorm and 48 partial row sums (sum x, sum x^2 over each 16-column slice, fp32), and the
// consumer (QKV, fc) multiplies x*gamma by W and finishes the LayerNorm in its epilogue -- 24
// LayerNorm launches, and their read and write of the activations, fewer per forward.  The result is
// not bit-identical to LayerNorm-then-GEMM: the fp16 rounding moves from the normalized row to
// x*gamma (same relative size), and the variance comes from the sums (E[x^2] - mu^2, fp32).
//
// G and H depend on the weights only: computed once per weights (and INT8 codes) on first use,
// cached per device, dropped by gpt2_free_gpu / gpt2_quant_free.  Weights changed in place need
// gpt2_tune_prefill_lnfold(0) or a fresh upload.
//
// By default the fold runs where it measured faster (interleaved A/B of the whole prefill, fold on
// against off, MI355X): T <= 128 for both weight formats (7-13% faster), INT8 up to T = 256 (4-5%).
// Past that the fold's per-tile costs (the partials' loads and the producer's extra stores in every
// work-group) outgrow the two LayerNorm launches it removes per layer: even at T = 384-512, 0.97-0.92
// at T = 768-1024.
static int g_lnfold = -1;       // gpt2_tune_prefill_lnfold: -1 default (by T), 0 off, 1 on at every T > 1
static int g_lnfold_sites = 0;  // sites that ran folded in the last forward (test hook)

extern "C" void gpt2_tune_prefill_lnfold(int on) { g_lnfold = on < 0 ? -1 : (on != 0); }
extern "C" int gpt2_tune_prefill_lnfold_sites(void) { return g_lnfold_sites; }

static bool lnfold_wanted(int T, bool int8) {
    if (g_lnfold >= 0) return g_lnfold == 1;
    if (T <= skinny_max_m(int8)) return false;   // the skinny GEMM's LayerNorm prologue takes these
    return T <= (int8 ? 256 : 128);
}

constexpr int FOLD_ROW = GPT2_QKV_DIM + GPT2_FFN_DIM;   // (G, H) pairs per layer: QKV's, then fc's

struct FoldConsts {
    const void *wdata;   // fp16 body
    const void *qdata;   // INT8 codes in use, or null
    int dev;
    float2 *gh;          // [layer][FOLD_ROW]
};
static std::mutex g_fold_mu;
static std::vector<FoldConsts> g_fold;

static void fold_consts_drop(const void *wdata, const void *qdata) {
    std::lock_guard<std::mutex> lock(g_fold_mu);
    for (size_t i = 0; i < g_fold.size();) {
        if ((wdata && g_fold[i].wdata == wdata) || (qdata && g_fold[i].qdata == qdata)) {
            int cur = 0;
            (void)hipGetDevice(&cur);
            if (cur != g_fold[i].dev) (void)hipSetDevice(g_fold[i].dev);
            gpt2_dfree(g_fold[i].gh);
            if (cur != g_fold[i].dev) (void)hipSetDevice(cur);
            g_fold[i] = g_fold.back();
            g_fold.pop_back();
        } else {
            ++i;
        }
    }
}

// The (G, H) table of these weights on the current device, computed on the stream when first asked
// for; null when it cannot be had now (no allocation under stream capture, allocation failure).
static const float2 *fold_consts(const GPT2Backend *be, const GPT2WeightsGPU *w) {
    const GPT2QWeightsGPU *qw = be->matmul_q ? w->q : nullptr;
    const void *qdata = qw ? (const void *)qw->qdata : nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_fold_mu);
    for (const FoldConsts &f : g_fold)
        if (f.wdata == w->data && f.qdata == qdata && f.dev == dev) return f.gh;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream(), &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return nullptr;
    }
    // an allocation failure is not the caller's (the unfolded sequence runs instead); an error the
    // caller has not read yet stays recorded
    const int pending = gpt2_last_error();
    float2 *gh = (float2 *)gpt2_dmalloc((size_t)GPT2_N_LAYER * FOLD_ROW * sizeof(float2));
    (void)gpt2_last_error();
    if (pending) set_error(pending, "an earlier call (recorded before the LayerNorm fold's set-up)");
    if (!gh) return nullptr;
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        const GPT2LayerGPU *ly = &w->layers[L];
        const GPT2QLayerGPU *qy = qw ? &qw->layers[L] : nullptr;
        const bool qq = qy && qy->qkv_w.q, qf = qy && qy->fc_w.q;
        ln_fold_consts(gh + (size_t)L * FOLD_ROW, qq ? (const void *)qy->qkv_w.q : ly->qkv_w, qq ? qy->qkv_w.s : nullptr,
                       ly->ln1_g, ly->ln1_b, GPT2_QKV_DIM, GPT2_N_EMBD, qq);
        ln_fold_consts(gh + (size_t)L * FOLD_ROW + GPT2_QKV_DIM, qf ? (const void *)qy->fc_w.q : ly->fc_w,
                       qf ? qy->fc_w.s : nullptr, ly->ln2_g, ly->ln2_b, GPT2_FFN_DIM, GPT2_N_EMBD, qf);
    }
    g_fold.push_back(FoldConsts{w->data, qdata, dev, gh});
    return gh;
}

// may_alloc: the trunk may run as the persistent kernel, and the LayerNorm fold may build its
// constants (both allocate on first use, so the no-allocation entry point runs the unfolded launch
// sequence instead).
static void forward_impl(const GPT2Backend *be, const GPT2WeightsGPU *w, const int *d_ids, int T, GPT2ScratchGPU *s,
                         GPT2CapsGPU *caps, bool may_alloc);

extern "C" void gpt2_forward_cuda(const GPT2Backend *be, const GPT2WeightsGPU *w, const int *d_ids, int T,
                                  GPT2ScratchGPU *s, GPT2CapsGPU *caps) {
    forward_impl(be, w, d_ids, T, s, caps, true);
}

static void forward_impl(const GPT2Backend *be, const GPT2WeightsGPU *w, const int *d_ids, int T, GPT2ScratchGPU *s,
                         GPT2CapsGPU *caps, bool may_alloc) {
    if (!be || !w || !w->data || !s || !d_ids || T <= 0 || T > s->maxT || T > GPT2_N_CTX) {
        arg_fail("gpt2_forward_cuda: bad arguments (T must be in [1, min(maxT, 1024)])");
        return;
    }
    const int E = GPT2_N_EMBD, Q = GPT2_QKV_DIM, F = GPT2_FFN_DIM, V = GPT2_VOCAB, H = GPT2_N_HEAD, D = GPT2_HEAD_DIM;
    const GPT2QWeightsGPU *qw = w->q;
    GPT2KVCache *kv = caps ? caps->kv : nullptr;
    if (kv && T > kv->maxT) { arg_fail("gpt2_forward_cuda: T exceeds the KV cache"); return; }

    const bool fused = fused_prefill_ok(be);
    // With the persistent prefill switched on (off by default: slower than the launch sequence),
    // the 12-layer trunk runs as one kernel (prefill.hip); the final LayerNorm, the head and the
    // captures follow as launches.
    g_lnfold_sites = 0;
    if (fused && may_alloc) {
        const uint16_t *x0 = nullptr, *xl[GPT2_N_LAYER];
        const uint16_t *xf = prefill_persist(be, w, d_ids, T, kv, &x0, xl);
        if (xf) {
            if (caps && caps->embed) capcpy(caps->embed, x0, (size_t)T * E);
            if (caps && caps->blocks)
                for (int L = 0; L < GPT2_N_LAYER; ++L) capcpy(caps->blocks + (size_t)L * T * E, xl[L], (size_t)T * E);
            be->layernorm(s->ln, xf, w->lnf_g, w->lnf_b, T, E);
            if (caps && caps->final_ln) capcpy(caps->final_ln, s->ln, (size_t)T * E);
            if (caps && caps->logits) {
                const GPT2QW *qh = qw ? &qw->wte : nullptr;
                if (caps->logits_all) gpt2_matmul_dispatch(be, caps->logits, s->ln, w->wte, qh, nullptr, T, V, E);
                else gpt2_matmul_dispatch(be, caps->logits, s->ln + (size_t)(T - 1) * E, w->wte, qh, nullptr, 1, V, E);
            }
            return;
        }
    }
    // the attention launch fills the cache itself when it is this library's prefill attention
    const bool attn_kv = fused && be->attention == gpt2_attention_flash && kv && kv->data;
    const bool ln_fuse = fused && be->layernorm == gpt2_layernorm;
    // The LayerNorm fold (above): this library's embedding and LayerNorm, T > 1 (the single-row GEMMs
    // are GEMVs), no forced LayerNorm-panel config.  x*gamma lives in s->ln, the row partials in
    // s->ao (48 x lnfold_stride(T) float2, at most T + 31 rows: within its T x 1536 bytes from T = 11
    // up, and T itself below 16); `have_stats` says whether the partials of the current x are there
    // -- a site whose fold kernel is not available runs unfolded and clears it, and the next
    // LayerNorm then runs as a launch.
    const float2 *gh = nullptr;
    if (fused && may_alloc && T > 1 && lnfold_wanted(T, be->matmul_q && qw) && be->embed == gpt2_embed &&
        be->layernorm == gpt2_layernorm && gemm_ln_forced() < 0)
        gh = fold_consts(be, w);
    float2 *stats = reinterpret_cast<float2 *>(s->ao);
    bool have_stats = false;
    if (gh) {
        embed_lnf(s->x, s->ln, stats, w->wte, w->wpe, d_ids, T, w->layers[0].ln1_g);
        have_stats = true;
    } else {
        be->embed(s->x, w->wte, w->wpe, d_ids, T, E);
    }
    if (caps && caps->embed) capcpy(caps->embed, s->x, (size_t)T * E);
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        const GPT2LayerGPU *ly = &w->layers[L];
        const GPT2QLayerGPU *qy = qw ? &qw->layers[L] : nullptr;
        const bool qq = be->matmul_q && qy && qy->qkv_w.q, qf = be->matmul_q && qy && qy->fc_w.q;
        const bool qa = be->matmul_q && qy && qy->attn_proj_w.q, qp = be->matmul_q && qy && qy->proj_w.q;
        LnFold lf{};
        lf.stats_in = stats;
        lf.stride = lnfold_stride(T);
        lf.gh = gh ? gh + (size_t)L * FOLD_ROW : nullptr;
        if (have_stats && gemm_lnfold(EPI_LNF, s->qkv, s->ln, qq ? (const void *)qy->qkv_w.q : ly->qkv_w,
                                      qq ? qy->qkv_w.s : nullptr, ly->qkv_b, T, Q, E, qq, nullptr, lf))
            ++g_lnfold_sites;
        else
            ln_matmul_site(be, fused, ln_fuse, s->qkv, s->x, ly->ln1_g, ly->ln1_b, s->ln, ly->qkv_w,
                           qy ? &qy->qkv_w : nullptr, ly->qkv_b, T, Q, E, EPI_NONE);
        have_stats = false;
        if (attn_kv && L < kv->nLayer) {
            attention_prefill(s->att, s->qkv, T, gpt2_kv_K(kv, L), gpt2_kv_V(kv, L), kv->maxT);
        } else {
            if (kv) gpt2_kv_scatter_prefill(kv, L, s->qkv, T);
            be->attention(s->att, s->qkv, T, E, H, D);
        }
        lf = LnFold{};
        lf.gamma = ly->ln2_g;
        lf.xg = s->ln;
        lf.stats_out = stats;
        lf.stride = lnfold_stride(T);
        if (gh && gemm_lnfold(EPI_RESID_LN, s->x, s->att, qa ? (const void *)qy->attn_proj_w.q : ly->attn_proj_w,
                              qa ? qy->attn_proj_w.s : nullptr, ly->attn_proj_b, T, E, E, qa, s->x, lf)) {
            ++g_lnfold_sites;
            have_stats = true;
        } else {
            matmul_site(be, fused, s->x, s->att, ly->attn_proj_w, qy ? &qy->attn_proj_w : nullptr, ly->attn_proj_b, T,
                        E, E, EPI_RESID, s->ao);
        }
        lf = LnFold{};
        lf.stats_in = stats;
        lf.stride = lnfold_stride(T);
        lf.gh = gh ? gh + (size_t)L * FOLD_ROW + Q : nullptr;
        if (have_stats && gemm_lnfold(EPI_LNF_GELU, s->fc, s->ln, qf ? (const void *)qy->fc_w.q : ly->fc_w,
                                      qf ? qy->fc_w.s : nullptr, ly->fc_b, T, F, E, qf, nullptr, lf))
            ++g_lnfold_sites;
        else
            ln_matmul_site(be, fused, ln_fuse, s->fc, s->x, ly->ln2_g, ly->ln2_b, s->ln, ly->fc_w,
                           qy ? &qy->fc_w : nullptr, ly->fc_b, T, F, E, EPI_GELU);
        have_stats = false;
        lf = LnFold{};
        lf.gamma = L + 1 < GPT2_N_LAYER ? w->layers[L + 1].ln1_g : nullptr;
        lf.xg = s->ln;
        lf.stats_out = stats;
        lf.stride = lnfold_stride(T);
        if (gh && lf.gamma &&
            gemm_lnfold(EPI_RESID_LN, s->x, s->fc, qp ? (const void *)qy->proj_w.q : ly->proj_w,
                        qp ? qy->proj_w.s : nullptr, ly->proj_b, T, E, F, qp, s->x, lf)) {
            ++g_lnfold_sites;
            have_stats = true;
        } else {
            matmul_site(be, fused, s->x, s->fc, ly->proj_w, qy ? &qy->proj_w : nullptr, ly->proj_b, T, E, F, EPI_RESID,
                        s->ff);
        }
        if (caps && caps->blocks) capcpy(caps->blocks + (size_t)L * T * E, s->x, (size_t)T * E);
    }
    be->layernorm(s->ln, s->x, w->lnf_g, w->lnf_b, T, E);
    if (caps && caps->final_ln) capcpy(caps->final_ln, s->ln, (size_t)T * E);
    if (caps && caps->logits) {
        const GPT2QW *qh = qw ? &qw->wte : nullptr;
        if (caps->logits_all) gpt2_matmul_dispatch(be, caps->logits, s->ln, w->wte, qh, nullptr, T, V, E);
        else gpt2_matmul_dispatch(be, caps->logits, s->ln + (size_t)(T - 1) * E, w->wte, qh, nullptr, 1, V, E);
    }
}

// ============================================================================ forward, no allocation
// gpt2_forward_cuda for callers that cannot allocate device memory (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc): the activations live in one file-scope device
// array instead of a GPT2ScratchGPU.  Each GPU that runs it holds its own copy of the array until
// the process ends; every call on a GPU reuses that GPU's copy, so calls that overlap on one GPU
// (two host threads, two streams) race.  Nothing in the array needs clearing: every buffer is
// written before it is read within a call.
constexpr size_t NOALLOC_ROW = 5 * GPT2_N_EMBD + GPT2_QKV_DIM + GPT2_FFN_DIM;   // halves per token
static __device__ __align__(256) uint16_t scratch[(size_t)GPT2_NOALLOC_MAX_T * NOALLOC_ROW];

// The device address of `scratch` on the current device, looked up once per device.  (In host code
// the array's name is a host-side stand-in, not a device address.)
static std::mutex g_scratch_mu;
static uint16_t *g_scratch_ptr[64];

static uint16_t *scratch_ptr() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_scratch_ptr[dev] = static_cast<uint16_t *>(p);
    }
    return g_scratch_ptr[dev];
}

void g2::noalloc_prepare() { (void)scratch_ptr(); }

extern "C" void gpt2_forward_noalloc(const GPT2Backend *be, const GPT2WeightsGPU *w, const int *d_ids, int T,
                                     GPT2CapsGPU *caps) {
    if (T > GPT2_NOALLOC_MAX_T) {
        set_error(E_CAPACITY, "gpt2_forward_noalloc: T exceeds GPT2_NOALLOC_MAX_T (128 tokens of static scratch)");
        return;
    }
    uint16_t *base = scratch_ptr();
    if (!base) {
        set_error(E_STATE, "gpt2_forward_noalloc: no device address for the static scratch");
        return;
    }
    // the GPT2ScratchGPU buffers carved from the array, rows of T tokens (16-byte aligned: every width
    // is a multiple of 8 halves)
    const size_t t = (size_t)(T > 0 ? T : 0), E = GPT2_N_EMBD;
    GPT2ScratchGPU s;
    s.x = base;
    s.ln = s.x + t * E;
    s.qkv = s.ln + t * E;
    s.att = s.qkv + t * GPT2_QKV_DIM;
    s.ao = s.att + t * E;
    s.fc = s.ao + t * E;
    s.ff = s.fc + t * GPT2_FFN_DIM;
    s.maxT = GPT2_NOALLOC_MAX_T;
    forward_impl(be, w, d_ids, T, &s, caps, false);
}

// ============================================================================ KV cache
extern "C" int gpt2_kv_alloc(GPT2KVCache *kv, int maxT) {
    memset(kv, 0, sizeof(*kv));
    if (maxT <= 0 || maxT > GPT2_N_CTX) { arg_fail("gpt2_kv_alloc: maxT out of range"); return 1; }
    kv->maxT = maxT;
    kv->nLayer = GPT2_N_LAYER;
    kv->nHead = GPT2_N_HEAD;
    kv->headDim = GPT2_HEAD_DIM;
    kv->bytes = (size_t)2 * GPT2_N_LAYER * GPT2_N_HEAD * maxT * GPT2_HEAD_DIM * 2;
    size_t freeB = 0, totB = 0;
    if (hipMemGetInfo(&freeB, &totB) != hipSuccess) return 1;
    if (kv->bytes + ((size_t)64 << 20) > freeB) return 1;   // keep 64 MiB of headroom (cuda/kvcache.cu:32-37)
    kv->data = (gpt2_half *)gpt2_dmalloc(kv->bytes);
    return kv->data ? 0 : 1;
}

extern "C" void gpt2_kv_free(GPT2KVCache *kv) {
    if (kv && kv->data) {
        gpt2_dfree(kv->data);
        kv->data = nullptr;
    }
}

extern "C" void gpt2_kv_reset(GPT2KVCache *kv) {
    if (kv) kv->len = 0;
}

extern "C" double gpt2_kv_step_bytes(const GPT2KVCache *kv, int len) {
    return 2.0 * kv->nLayer * kv->nHead * (double)len * kv->headDim * 2.0;
}

// ============================================================================ decode step
// One token (cuda/kvcache.cu:233-269).  With st.state set, token/pos come from device memory and
// the step ends with the greedy argmax that advances that state (the graph-replayed form).
//
// When the backend's GEMV slots are this library's GEMVs, the step runs fused: each LayerNorm is
// computed inside the GEMV that consumes it, gelu and the residual adds run in the GEMV epilogues,
// and the K/V append runs inside decode attention -- 5 launches per layer instead of 11.  Other
// backends (no .gemv: the M=1 matmul fallback) run the reference's unfused sequence.
static bool fused_decode_ok(const GPT2Backend *be) {
    return be->gemv == gpt2_gemv_fp16 && (be->gemv_q == nullptr || be->gemv_q == gpt2_gemv_int8) &&
           be->layernorm == gpt2_layernorm && be->add == gpt2_add && be->gelu == gpt2_gelu;
}

// One weight-matmul site: (LayerNorm(in) ->) GEMV (-> gelu | + residual into C).  Fused when the
// backend allows and a fused kernel covers the shape, else the unfused sequence through the
// backend (LayerNorm into s->ln, GEMV into `tmp` when a residual follows, then gelu / add).
static void gemv_site(const GPT2Backend *be, bool fused, GPT2ScratchGPU *s, gpt2_half *C, const gpt2_half *in,
                      const gpt2_half *Wh, const GPT2QW *Wq, const gpt2_half *bias, int N, int K,
                      const gpt2_half *ln_g, const gpt2_half *ln_b, int epi, gpt2_half *tmp) {
    const bool q = be->gemv_q && Wq && Wq->q;
    if (fused && gemv_fused(C, in, q ? (const void *)Wq->q : (const void *)Wh, q ? Wq->s : nullptr, bias, N, K, q,
                            ln_g, ln_b, epi, epi == EPI_RESID ? C : nullptr))
        return;
    const gpt2_half *x = in;
    if (ln_g) {
        be->layernorm(s->ln, in, ln_g, ln_b, 1, K);
        x = s->ln;
    }
    gpt2_half *out = (epi == EPI_RESID) ? tmp : C;
    gpt2_gemv_dispatch(be, out, x, Wh, Wq, bias, N, K);
    if (epi == EPI_GELU) be->gelu(C, (size_t)N);
    if (epi == EPI_RESID) be->add(C, tmp, (size_t)N);
}

static void decode_step(const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv, StepArg st,
                        GPT2ScratchGPU *s, gpt2_half *logits, gpt2_half *caps, int *state, int *tokens) {
    const int E = GPT2_N_EMBD, Q = GPT2_QKV_DIM, F = GPT2_FFN_DIM, V = GPT2_VOCAB;
    const GPT2QWeightsGPU *qw = w->q;
    const bool fused = fused_decode_ok(be);
    embed_one(s->x, w->wte, w->wpe, st);
    if (caps) capcpy(caps + (size_t)(GPT2_N_LAYER + 1) * E, s->x, E);
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        const GPT2LayerGPU *ly = &w->layers[L];
        const GPT2QLayerGPU *qy = qw ? &qw->layers[L] : nullptr;
        gemv_site(be, fused, s, s->qkv, s->x, ly->qkv_w, qy ? &qy->qkv_w : nullptr, ly->qkv_b, Q, E, ly->ln1_g,
                  ly->ln1_b, EPI_NONE, nullptr);
        if (fused) {
            attn_decode_append(s->att, s->qkv, gpt2_kv_K(kv, L), gpt2_kv_V(kv, L), kv->maxT, st);
        } else {
            kv_append(gpt2_kv_K(kv, L), gpt2_kv_V(kv, L), s->qkv, st, kv->maxT);
            attn_decode(s->att, s->qkv, gpt2_kv_K(kv, L), gpt2_kv_V(kv, L), kv->maxT, st, st.state ? 0 : st.pos + 1);
        }
        gemv_site(be, fused, s, s->x, s->att, ly->attn_proj_w, qy ? &qy->attn_proj_w : nullptr, ly->attn_proj_b, E, E,
                  nullptr, nullptr, EPI_RESID, s->ao);
        gemv_site(be, fused, s, s->fc, s->x, ly->fc_w, qy ? &qy->fc_w : nullptr, ly->fc_b, F, E, ly->ln2_g, ly->ln2_b,
                  EPI_GELU, nullptr);
        gemv_site(be, fused, s, s->x, s->fc, ly->proj_w, qy ? &qy->proj_w : nullptr, ly->proj_b, E, F, nullptr, nullptr,
                  EPI_RESID, s->ff);
        if (caps) capcpy(caps + (size_t)L * E, s->x, E);
    }
    if (caps) {
        be->layernorm(s->ln, s->x, w->lnf_g, w->lnf_b, 1, E);
        capcpy(caps + (size_t)GPT2_N_LAYER * E, s->ln, E);
    }
    if (logits)
        gemv_site(be, fused, s, logits, s->x, w->wte, qw ? &qw->wte : nullptr, nullptr, V, E, w->lnf_g, w->lnf_b,
                  EPI_NONE, nullptr);
    if (state) argmax_advance(logits, V, state, tokens, kv->maxT);
}

extern "C" void gpt2_decode_step_cuda(const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv, int token,
                                      int pos, GPT2ScratchGPU *s, gpt2_half *logits, gpt2_half *caps_blocks) {
    if (!be || !w || !w->data || !kv || !kv->data || !s || s->maxT < 1) { arg_fail("gpt2_decode_step_cuda: null argument"); return; }
    if (pos < 0 || pos >= kv->maxT || pos > kv->len || token < 0 || token >= GPT2_VOCAB) {
        arg_fail("gpt2_decode_step_cuda: need 0 <= pos <= kv->len, pos < maxT, token < vocab");
        return;
    }
    decode_step(be, w, kv, StepArg{token, pos, nullptr}, s, logits, caps_blocks, nullptr, nullptr);
    kv->len = pos + 1;
}

extern "C" void gpt2_prefill_fill_cache(const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv,
                                        const int *d_ids, int T, GPT2ScratchGPU *s, GPT2CapsGPU *caps) {
    GPT2CapsGPU c;
    if (caps) c = *caps;
    else memset(&c, 0, sizeof(c));
    c.kv = kv;
    const int before = gpt2_last_error();
    gpt2_forward_cuda(be, w, d_ids, T, s, &c);
    const int err = gpt2_last_error();
    if (before) set_error(before, "before gpt2_prefill_fill_cache");
    if (err) set_error(err, "gpt2_prefill_fill_cache");
    else kv->len = T;
}

// ============================================================================ graph replay
constexpr int PERSIST_CHUNK = 16;   // persistent steps per graph replay

struct GPT2DecodeGraph {
    hipStream_t stream;
    hipGraph_t graph;       // one step (multi-kernel) or PERSIST_CHUNK steps (persistent)
    hipGraphExec_t exec;
    int *state;       // device {token, pos, epoch, error, poll limit}
    GPT2KVCache *kv;
    int host_pos;     // position the next replay consumes, tracked on the host
    int mode;         // GPT2_DECODE_MULTI or GPT2_DECODE_PERSISTENT
    PDPlan plan;      // persistent mode only
    uint64_t *ll;     // persistent mode: exchange arena
};

static void graph_free(GPT2DecodeGraph *g) {
    if (g->stream) hipStreamDestroy(g->stream);
    gpt2_dfree(g->ll);
    gpt2_dfree(g->state);
    delete g;
}

extern "C" GPT2DecodeGraph *gpt2_decode_graph_create_mode(const GPT2Backend *be, const GPT2WeightsGPU *w,
                                                          GPT2KVCache *kv, GPT2ScratchGPU *s, gpt2_half *logits,
                                                          int *tokens, int mode) {
    if (!be || !w || !w->data || !kv || !kv->data || !s || !logits) { arg_fail("gpt2_decode_graph_create: null argument"); return nullptr; }
    if (mode == GPT2_DECODE_AUTO) {
        const char *e = getenv("GPT2_DECODE_PERSISTENT");
        mode = (e && e[0] == '0') ? GPT2_DECODE_MULTI : GPT2_DECODE_PERSISTENT;
    }
    if (mode != GPT2_DECODE_MULTI && mode != GPT2_DECODE_PERSISTENT) { arg_fail("gpt2_decode_graph_create: bad mode"); return nullptr; }
    GPT2DecodeGraph *g = new GPT2DecodeGraph();
    g->kv = kv;
    g->host_pos = kv->len;
    g->mode = GPT2_DECODE_MULTI;
    if (hipStreamCreate(&g->stream) != hipSuccess) { g->stream = nullptr; graph_free(g); set_error(E_STATE, "hipStreamCreate"); return nullptr; }
    g->state = (int *)gpt2_dmalloc(8 * sizeof(int));
    if (!g->state) { graph_free(g); return nullptr; }
    const int init[5] = {0, kv->len, 1, 0, persist_spin()};   // epoch 1: the zeroed exchange arena holds flag 0
    if (hipMemcpy(g->state, init, sizeof(init), hipMemcpyHostToDevice) != hipSuccess) {
        graph_free(g);
        set_error(E_STATE, "decode graph state");
        return nullptr;
    }
    // The persistent step needs this library's fused GEMV path; otherwise the multi-kernel step runs.
    if (mode == GPT2_DECODE_PERSISTENT && fused_decode_ok(be)) {
        g->ll = (uint64_t *)gpt2_dmalloc(persist_ll_bytes());
        if (g->ll && hipMemset(g->ll, 0, persist_ll_bytes()) == hipSuccess &&
            persist_plan(g->plan, be, w, kv, logits, g->state, tokens, g->ll, g->state + 3))
            g->mode = GPT2_DECODE_PERSISTENT;
        else {
            gpt2_dfree(g->ll);
            g->ll = nullptr;
            gpt2_last_error();   // fall back quietly to the multi-kernel step
        }
    }

    hipStream_t prev = stream();
    // The multi-kernel step is captured once and replayed per token.  The persistent step is one
    // kernel: PERSIST_CHUNK consecutive steps are captured as one graph (one replay decodes that many
    // tokens), and single steps or the remainder of a run are launched directly (a one-kernel graph
    // per token only adds launch latency, ~8 us measured).
    gpt2_set_stream(g->stream);
    hipError_t e = hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
        if (g->mode == GPT2_DECODE_PERSISTENT)
            for (int i = 0; i < PERSIST_CHUNK; ++i) persist_launch(g->plan, g->stream);
        else decode_step(be, w, kv, StepArg{0, 0, g->state}, s, logits, nullptr, g->state, tokens);
        e = hipStreamEndCapture(g->stream, &g->graph);
    }
    gpt2_set_stream(prev);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        set_error((int)e, "decode graph capture/instantiate");
        graph_free(g);
        return nullptr;
    }
    return g;
}

extern "C" GPT2DecodeGraph *gpt2_decode_graph_create(const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv,
                                                     GPT2ScratchGPU *s, gpt2_half *logits, int *tokens) {
    return gpt2_decode_graph_create_mode(be, w, kv, s, logits, tokens, GPT2_DECODE_AUTO);
}

extern "C" int gpt2_decode_graph_mode(const GPT2DecodeGraph *g) { return g ? g->mode : -1; }

extern "C" int gpt2_decode_graph_set(GPT2DecodeGraph *g, int token, int pos) {
    if (!g || token < 0 || token >= GPT2_VOCAB || pos < 0 || pos >= g->kv->maxT) { set_error(E_ARG, "gpt2_decode_graph_set"); return 1; }
    // {token, pos, epoch + 1, 0, poll limit}: the error word of a step that timed out is cleared,
    // and the next epoch makes every exchange word that step left behind stale (its sequence numbers
    // can no longer match a poll).
    int st[5];
    hipError_t e = hipMemcpyAsync(st, g->state, sizeof(st), hipMemcpyDeviceToHost, g->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g->stream);
    if (e == hipSuccess) {
        st[0] = token;
        st[1] = pos;
        st[2] += 1;
        st[3] = 0;
        st[4] = persist_spin();
        e = hipMemcpyAsync(g->state, st, sizeof(st), hipMemcpyHostToDevice, g->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(g->stream);
    if (e != hipSuccess) { set_error((int)e, "gpt2_decode_graph_set"); return (int)e; }
    g->host_pos = pos;
    return 0;
}

extern "C" int gpt2_decode_graph_run(GPT2DecodeGraph *g, int steps) {
    if (!g || steps < 0) { set_error(E_ARG, "gpt2_decode_graph_run"); return 1; }
    if (g->host_pos + steps > g->kv->maxT) { set_error(E_CAPACITY, "gpt2_decode_graph_run: past the cache"); return 1; }
    for (int i = 0; i < steps;) {
        hipError_t e;
        if (g->mode != GPT2_DECODE_PERSISTENT) {
            e = hipGraphLaunch(g->exec, g->stream);
            ++i;
        } else if (steps - i >= PERSIST_CHUNK) {
            e = hipGraphLaunch(g->exec, g->stream);
            i += PERSIST_CHUNK;
        } else {
            persist_launch(g->plan, g->stream);
            e = hipGetLastError();
            ++i;
        }
        if (e != hipSuccess) { set_error((int)e, "decode step launch"); return (int)e; }
    }
    g->host_pos += steps;
    return 0;
}

extern "C" int gpt2_decode_graph_sync(GPT2DecodeGraph *g, int *token, int *pos) {
    if (!g) return 1;
    int st[4];
    hipError_t e = hipMemcpyAsync(st, g->state, sizeof(st), hipMemcpyDeviceToHost, g->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g->stream);
    if (e != hipSuccess) { set_error((int)e, "gpt2_decode_graph_sync"); return (int)e; }
    if (st[3]) {
        // A persistent step gave up waiting for another work-group's output: its results are void.
        set_error(E_STATE, "persistent decode step: an exchange timed out (work-groups not co-resident?)");
        return E_STATE;
    }
    if (token) *token = st[0];
    if (pos) *pos = st[1];
    g->kv->len = st[1];
    g->host_pos = st[1];
    return 0;
}

// Bench hook: mean milliseconds per replay over `steps` back-to-back replays, timed with events on
// the graph's own stream.
extern "C" int gpt2_decode_graph_time(GPT2DecodeGraph *g, int steps, float *ms) {
    if (!g || steps <= 0 || !ms) return 1;
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
    hipEventRecord(a, g->stream);
    const int rc = gpt2_decode_graph_run(g, steps);
    hipEventRecord(b, g->stream);
    hipEventSynchronize(b);
    float t = 0.f;
    hipEventElapsedTime(&t, a, b);
    *ms = t / steps;
    hipEventDestroy(a);
    hipEventDestroy(b);
    return rc;
}

extern "C" void gpt2_decode_graph_destroy(GPT2DecodeGraph *g) {
    if (!g) return;
    hipStreamSynchronize(g->stream);
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    graph_free(g);
}

// ============================================================================ INT8 weights
namespace {
// The 49 quantizable matrices in file order: the tied head wte, then per layer qkv, attn_proj, fc,
// proj (row count N = output features, column count K = input features).
const int kNQ = 1 + 4 * GPT2_N_LAYER;

struct MatDims {
    int rows, cols;
    size_t elems() const { return (size_t)rows * cols; }
};

MatDims matrix_dims(int i) {
    if (i == 0) return {GPT2_VOCAB, GPT2_N_EMBD};
    switch ((i - 1) % 4) {
        case 0: return {GPT2_QKV_DIM, GPT2_N_EMBD};
        case 1: return {GPT2_N_EMBD, GPT2_N_EMBD};
        case 2: return {GPT2_FFN_DIM, GPT2_N_EMBD};
        default: return {GPT2_N_EMBD, GPT2_FFN_DIM};
    }
}

GPT2QW *qw_slot(GPT2QWeightsGPU *q, int i) {
    if (i == 0) return &q->wte;
    GPT2QLayerGPU &l = q->layers[(i - 1) / 4];
    switch ((i - 1) % 4) {
        case 0: return &l.qkv_w;
        case 1: return &l.attn_proj_w;
        case 2: return &l.fc_w;
        default: return &l.proj_w;
    }
}

const gpt2_half *fp16_tensor(const GPT2WeightsGPU *w, int i) {
    if (i == 0) return w->wte;
    const GPT2LayerGPU &l = w->layers[(i - 1) / 4];
    switch ((i - 1) % 4) {
        case 0: return l.qkv_w;
        case 1: return l.attn_proj_w;
        case 2: return l.fc_w;
        default: return l.proj_w;
    }
}

// Arena sizes of the quantized matrices (quantized[i] != 0): int8 codes and fp32 row scales.
void arena_sizes(const int *quantized, size_t *codes, size_t *scales) {
    *codes = *scales = 0;
    for (int i = 0; i < kNQ; ++i)
        if (quantized[i]) { *codes += matrix_dims(i).elems(); *scales += matrix_dims(i).rows; }
}

// Points each GPT2QW view into the arenas, matrix after matrix; an unquantized matrix gets q = s =
// NULL (it stays fp16) and counts its fp16 bytes in the per-step stream.
void q_attach(GPT2QWeightsGPU *q, const int *quantized) {
    size_t code_at = 0, scale_at = 0, fp16_elems = 0;
    for (int i = 0; i < kNQ; ++i) {
        GPT2QW *v = qw_slot(q, i);
        const MatDims d = matrix_dims(i);
        if (!quantized[i]) {
            v->q = nullptr;
            v->s = nullptr;
            fp16_elems += d.elems();
            continue;
        }
        v->q = q->qdata + code_at;
        v->s = q->sdata + scale_at;
        code_at += d.elems();
        scale_at += d.rows;
    }
    q->streamed_bytes = q->nq + q->ns * 4 + fp16_elems * 2;
}
}  // namespace

extern "C" void gpt2_quant_free(GPT2QWeightsGPU *q) {
    if (!q) return;
    if (q->qdata) fold_consts_drop(nullptr, q->qdata);
    gpt2_dfree(q->qdata);
    gpt2_dfree(q->sdata);
    q->qdata = nullptr;
    q->sdata = nullptr;
}

extern "C" int gpt2_quant_build(GPT2WeightsGPU *gpu, GPT2QWeightsGPU *q, const int *keep) {
    memset(q, 0, sizeof(*q));
    if (!gpu || !gpu->data) { arg_fail("gpt2_quant_build: no fp16 weights"); return 1; }
    int quantized[kNQ];
    for (int i = 0; i < kNQ; ++i) quantized[i] = keep ? !keep[i] : (i != 0);
    arena_sizes(quantized, &q->nq, &q->ns);
    q->qdata = (int8_t *)gpt2_dmalloc(q->nq ? q->nq : 1);
    q->sdata = (float *)gpt2_dmalloc((q->ns ? q->ns : 1) * 4);
    if (!q->qdata || !q->sdata) { gpt2_quant_free(q); return 1; }
    q_attach(q, quantized);
    for (int i = 0; i < kNQ; ++i) {
        if (!quantized[i]) continue;
        GPT2QW *v = qw_slot(q, i);
        gpt2_quantize_rows((int8_t *)v->q, (float *)v->s, fp16_tensor(gpu, i), matrix_dims(i).rows, matrix_dims(i).cols);
    }
    if (gpt2_sync()) { gpt2_quant_free(q); return 1; }
    gpu->q = q;
    return 0;
}

extern "C" int gpt2_quant_load_upload(const char *path, GPT2WeightsGPU *gpu, GPT2QWeightsGPU *q) {
    static const char *me = "gpt2_quant_load_upload";
    memset(q, 0, sizeof(*q));
    FILE *f = fopen(path, "rb");
    if (!f) return load_reject(me, path, "cannot be opened for reading", 1);
    auto reject = [&](const char *why) { fclose(f); return load_reject(me, path, why, 1); };
    int32_t head[16];
    if (fread(head, 4, 16, f) != 16) return reject("the file ends inside its 64-byte header");
    if (head[0] != kMagicQ || head[1] != 2) return reject("not a 'GPQ8' version 2 file");
    const int32_t dims[6] = {GPT2_N_LAYER, GPT2_N_EMBD, GPT2_VOCAB, GPT2_FFN_DIM, GPT2_QKV_DIM, kNQ};
    if (memcmp(head + 2, dims, sizeof dims) != 0) return reject("its model dimensions are not GPT-2-124M's");
    int quantized[kNQ];
    if (fread(quantized, 4, kNQ, f) != (size_t)kNQ) return reject("the file ends inside its per-matrix flags");
    for (int i = 0; i < kNQ; ++i) quantized[i] = quantized[i] != 0;
    arena_sizes(quantized, &q->nq, &q->ns);
    // the file holds, per quantized matrix in order, its codes then its row scales; both go to host
    // staging arenas laid out as the device arenas are
    std::vector<int8_t> codes(q->nq ? q->nq : 1);
    std::vector<float> scales(q->ns ? q->ns : 1);
    size_t code_at = 0, scale_at = 0;
    for (int i = 0; i < kNQ; ++i) {
        if (!quantized[i]) continue;
        const MatDims d = matrix_dims(i);
        if (fread(codes.data() + code_at, 1, d.elems(), f) != d.elems()) return reject("the file ends inside a matrix's codes");
        if (fread(scales.data() + scale_at, 4, d.rows, f) != (size_t)d.rows) return reject("the file ends inside a matrix's scales");
        code_at += d.elems();
        scale_at += d.rows;
    }
    const long at = ftell(f);
    fseek(f, 0, SEEK_END);
    const long past_end = ftell(f) - at;
    fclose(f);
    if (past_end != 0) return load_reject(me, path, "bytes follow the last matrix", 1);
    q->qdata = (int8_t *)gpt2_dmalloc(q->nq ? q->nq : 1);
    q->sdata = (float *)gpt2_dmalloc((q->ns ? q->ns : 1) * 4);
    if (!q->qdata || !q->sdata) { gpt2_quant_free(q); return 1; }
    if (gpt2_h2d(q->qdata, codes.data(), q->nq) || gpt2_h2d(q->sdata, scales.data(), q->ns * 4)) {
        gpt2_quant_free(q);
        return 1;
    }
    q_attach(q, quantized);
    if (gpu) gpu->q = q;
    return 0;
}

extern "C" int gpt2_quant_write_file(const char *path, const GPT2QWeightsGPU *q, const int *keep) {
    if (!q || !path) return 1;
    GPT2QWeightsGPU *views = const_cast<GPT2QWeightsGPU *>(q);
    int quantized[kNQ];
    for (int i = 0; i < kNQ; ++i) quantized[i] = qw_slot(views, i)->q != nullptr;
    if (keep)
        for (int i = 0; i < kNQ; ++i)
            if (keep[i] && quantized[i]) return 1;   // asked to keep a tensor that is quantized
    FILE *f = fopen(path, "wb");
    if (!f) return 1;
    int32_t head[16] = {kMagicQ, 2, GPT2_N_LAYER, GPT2_N_EMBD, GPT2_VOCAB, GPT2_FFN_DIM, GPT2_QKV_DIM, kNQ};
    bool ok = fwrite(head, 4, 16, f) == 16 && fwrite(quantized, 4, kNQ, f) == (size_t)kNQ;
    for (int i = 0; ok && i < kNQ; ++i) {
        if (!quantized[i]) continue;
        const MatDims d = matrix_dims(i);
        const GPT2QW *v = qw_slot(views, i);
        std::vector<int8_t> codes(d.elems());
        std::vector<float> scales(d.rows);
        ok = !gpt2_d2h(codes.data(), v->q, d.elems()) && !gpt2_d2h(scales.data(), v->s, (size_t)d.rows * 4) &&
             fwrite(codes.data(), 1, d.elems(), f) == d.elems() && fwrite(scales.data(), 4, d.rows, f) == (size_t)d.rows;
    }
    return (fclose(f) == 0 && ok) ? 0 : 1;
}

extern "C" int gpt2_quant_attach_if_needed(const GPT2Backend *be, GPT2WeightsGPU *gpu, GPT2QWeightsGPU *q) {
    memset(q, 0, sizeof(*q));
    if (!be->matmul_q) return 0;
    const char *p = getenv("GPT2_INT8_WEIGHTS");
    return gpt2_quant_load_upload(p ? p : "weights/gpt2_124m_int8_kt.bin", gpu, q);
}
