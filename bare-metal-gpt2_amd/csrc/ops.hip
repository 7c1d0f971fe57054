// ops.hip -- the non-matmul kernels a running GPT-2 needs around the matmul path, plus the device
// quantizer.  Plain and correct; the matmul kernels are where the tuning goes.
//
// Numerics follow the reference's GPU kernels: fp16 storage, fp32 arithmetic inside every op,
//   embed  x = fp16(wte[id] + wpe[t])                          (cuda/kernels_naive.cu:17-23)
//   LN     mean, then biased variance of (x - mean), eps 1e-5 inside the sqrt
//                                                              (cuda/kernels_naive.cu:26-41)
//   gelu   0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3)))  (cuda/kernels_naive.cu:85-91)
//   attention: causal, scale 1/sqrt(64), online softmax       (cuda/kernels_fused.cu:58-140)
//   decode attention over the [H][maxT][D] cache               (cuda/kvcache.cu:88-129)
// The INT8 quantizer restates tools/quantize.py:58-73 on the GPU (see k_quantize_rows).
#include <cmath>

#include "common.h"
#include "attn.h"

namespace g2 {
void attention_prefill(uint16_t *att, const uint16_t *qkv, int T, uint16_t *Kc = nullptr, uint16_t *Vc = nullptr,
                       int maxT = 0);   // attn_prefill.hip

// ------------------------------------------------------------------ embed
__global__ void k_embed(uint16_t *__restrict__ x, const uint16_t *__restrict__ wte, const uint16_t *__restrict__ wpe,
                        const int *__restrict__ ids, int T, int E) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)T * E) return;
    const int t = (int)(idx / E), e = (int)(idx - (long)t * E);
    const int id = ids[t];
    // Out-of-vocabulary ids read nothing (an unchecked gather would fault) and embed as wpe alone.
    const float te = ((unsigned)id < (unsigned)GPT2_VOCAB) ? h2f(wte[(size_t)id * E + e]) : 0.f;
    x[idx] = f2h(te + h2f(wpe[(size_t)t * E + e]));
}

__global__ void k_embed_one(uint16_t *__restrict__ x, const uint16_t *__restrict__ wte,
                            const uint16_t *__restrict__ wpe, StepArg st, int E) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int id = st.tok(), pos = st.p();
    const float te = ((unsigned)id < (unsigned)GPT2_VOCAB) ? h2f(wte[(size_t)id * E + e]) : 0.f;
    const float pe = ((unsigned)pos < (unsigned)GPT2_N_CTX) ? h2f(wpe[(size_t)pos * E + e]) : 0.f;
    x[e] = f2h(te + pe);
}

// The embedding for the prefill's LayerNorm fold (LnFold): one wave per row writes x = wte + wpe,
// xg = x * gamma (gamma of the first layer's LN1) and the row's 48 partial sums (sum x, sum x^2 over
// each 16-column slice) of the fp16 x, slot-major ([slot][stride], as the fold's GEMMs read them).  Lane l holds columns 256 i + 4 l + c (i < 3, c < 4), so
// slice 16 i + l / 4 is the four lanes 4 (l / 4) .. +3, reduced with two fixed lane exchanges.
__global__ __launch_bounds__(256) void k_embed_lnf(uint16_t *__restrict__ x, uint16_t *__restrict__ xg,
                                                   float2 *__restrict__ stats, const uint16_t *__restrict__ wte,
                                                   const uint16_t *__restrict__ wpe, const int *__restrict__ ids,
                                                   const uint16_t *__restrict__ gamma, int T, int stride) {
    constexpr int E = GPT2_N_EMBD;
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (row >= T) return;   // wave-uniform
    const int id = ids[row];
    const bool in_vocab = (unsigned)id < (unsigned)GPT2_VOCAB;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int c0 = 256 * i + 4 * lane;
        uint16_t o[4], g[4];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float te = in_vocab ? h2f(wte[(size_t)id * E + c0 + c]) : 0.f;
            o[c] = f2h(te + h2f(wpe[(size_t)row * E + c0 + c]));
            const float xv = h2f(o[c]);
            s1 += xv;
            s2 = __builtin_fmaf(xv, xv, s2);
            g[c] = f2h(xv * h2f(gamma[c0 + c]));
        }
        *reinterpret_cast<uint2 *>(x + (size_t)row * E + c0) =
            uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
        *reinterpret_cast<uint2 *>(xg + (size_t)row * E + c0) =
            uint2{(uint32_t)g[0] | ((uint32_t)g[1] << 16), (uint32_t)g[2] | ((uint32_t)g[3] << 16)};
        s1 += __shfl_xor(s1, 1);
        s2 += __shfl_xor(s2, 1);
        s1 += __shfl_xor(s1, 2);
        s2 += __shfl_xor(s2, 2);
        if ((lane & 3) == 0) stats[(size_t)(16 * i + lane / 4) * stride + row] = float2{s1, s2};
    }
}

// The LayerNorm fold's per-column constants of one consumer matrix W [N, K] (fp16, or INT8 codes with
// row scales): G_n = sum_k gamma_k W_nk, H_n = sum_k beta_k W_nk, fp32 (INT8: the code sums times
// s_n, as the consumer scales its code sums).  One wave per row.
template <bool QW>
__global__ __launch_bounds__(256) void k_ln_fold_consts(float2 *__restrict__ gh, const void *__restrict__ Wv,
                                                        const float *__restrict__ Ws, const uint16_t *__restrict__ gamma,
                                                        const uint16_t *__restrict__ beta, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int n = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (n >= N) return;
    float g = 0.f, h = 0.f;
    for (int k = lane; k < K; k += 64) {
        const float w = QW ? (float)reinterpret_cast<const int8_t *>(Wv)[(size_t)n * K + k]
                           : h2f(reinterpret_cast<const uint16_t *>(Wv)[(size_t)n * K + k]);
        g = __builtin_fmaf(h2f(gamma[k]), w, g);
        h = __builtin_fmaf(h2f(beta[k]), w, h);
    }
    g = wave_sum(g);
    h = wave_sum(h);
    const float s = QW ? Ws[n] : 1.f;
    if (lane == 0) gh[n] = float2{g * s, h * s};
}

void embed_lnf(uint16_t *x, uint16_t *xg, float2 *stats, const uint16_t *wte, const uint16_t *wpe, const int *ids,
               int T, const uint16_t *gamma) {
    hipLaunchKernelGGL(k_embed_lnf, dim3(cdiv(T, 4)), dim3(256), 0, stream(), x, xg, stats, wte, wpe, ids, gamma, T,
                       lnfold_stride(T));
    check_launch("k_embed_lnf");
}

void ln_fold_consts(float2 *gh, const void *W, const float *Ws, const uint16_t *gamma, const uint16_t *beta, int N,
                    int K, bool qw) {
    if (qw)
        hipLaunchKernelGGL(k_ln_fold_consts<true>, dim3(cdiv(N, 4)), dim3(256), 0, stream(), gh, W, Ws, gamma, beta, N, K);
    else
        hipLaunchKernelGGL(k_ln_fold_consts<false>, dim3(cdiv(N, 4)), dim3(256), 0, stream(), gh, W, Ws, gamma, beta, N, K);
    check_launch("k_ln_fold_consts");
}

// ------------------------------------------------------------------ LayerNorm: one wave per row
template <bool VEC768>
__global__ __launch_bounds__(256) void k_layernorm(uint16_t *__restrict__ out, const uint16_t *__restrict__ x,
                                                   const uint16_t *__restrict__ g, const uint16_t *__restrict__ b,
                                                   int M, int E) {
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (row >= M) return;
    const uint16_t *xr = x + (size_t)row * E;
    uint16_t *o = out + (size_t)row * E;
    if constexpr (VEC768) {
        // E = 768 = 3 x (64 lanes x 4 halves): the row stays in registers between the passes; gamma
        // and beta are loaded with the row, so their latency hides behind the two reductions.  The
        // arithmetic is ln_row768's, shared with the GEMMs that normalize their own A panel.
        f16x4 h[3], gg[3], bb[3], r[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            h[i] = *reinterpret_cast<const f16x4 *>(xr + 256 * i + 4 * lane);
            gg[i] = *reinterpret_cast<const f16x4 *>(g + 256 * i + 4 * lane);
            bb[i] = *reinterpret_cast<const f16x4 *>(b + 256 * i + 4 * lane);
        }
        ln_row768(h, gg, bb, r);
#pragma unroll
        for (int i = 0; i < 3; ++i) *reinterpret_cast<f16x4 *>(o + 256 * i + 4 * lane) = r[i];
        return;
    } else {
    float s = 0.f;
    for (int e = lane; e < E; e += 64) s += h2f(xr[e]);
    const float mean = wave_sum(s) / E;
    float q = 0.f;
    for (int e = lane; e < E; e += 64) {
        const float d = h2f(xr[e]) - mean;
        q += d * d;
    }
    const float rstd = 1.0f / sqrtf(wave_sum(q) / E + GPT2_LN_EPS);
    for (int e = lane; e < E; e += 64) o[e] = f2h((h2f(xr[e]) - mean) * rstd * h2f(g[e]) + h2f(b[e]));
    }
}

// ------------------------------------------------------------------ gelu / add
__global__ void k_gelu(uint16_t *__restrict__ x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    x[i] = gelu_f16(h2f(x[i]));
}

__global__ void k_gelu8(f16x8 *__restrict__ x, size_t n8) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n8) return;
    f16x8 v = x[i];
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = __builtin_bit_cast(f16, gelu_f16((float)v[c]));
    x[i] = v;
}

__global__ void k_add(uint16_t *__restrict__ x, const uint16_t *__restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    x[i] = f2h(h2f(x[i]) + h2f(y[i]));
}

__global__ void k_add8(f16x8 *__restrict__ x, const f16x8 *__restrict__ y, size_t n8) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n8) return;
    f16x8 a = x[i];
    const f16x8 b = y[i];
#pragma unroll
    for (int c = 0; c < 8; ++c) a[c] = (f16)((float)a[c] + (float)b[c]);
    x[i] = a;
}

// Merge the NW waves' partial (m, l, c) states of one head through LDS and write the context.
template <int NW>
__device__ __forceinline__ void merge_waves(const AttnState &st, uint16_t *__restrict__ out) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __shared__ float sm[NW], sl[NW], sc[NW][GPT2_HEAD_DIM];
    if (lane == 0) {
        sm[w] = st.m;
        sl[w] = st.l;
    }
    if (lane < 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sc[w][8 * lane + e] = st.c[e];
    }
    __syncthreads();
    if (w == 0) {
        float mx = -INFINITY;
        for (int i = 0; i < NW; ++i) mx = fmaxf(mx, sm[i]);
        float L = 0.f, c = 0.f;
        for (int i = 0; i < NW; ++i) {
            if (sl[i] == 0.f) continue;   // wave had no keys
            const float f = __expf(sm[i] - mx);
            L += sl[i] * f;
            c += sc[i][lane] * f;
        }
        out[lane] = f2h(c / L);
    }
}

// Decode: one work-group per head, NW waves split the keys [0, len); partial (m, l, c) states are
// merged through LDS.  len = pos + 1 comes from the step argument.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_attn_decode(uint16_t *__restrict__ att, const uint16_t *__restrict__ qkv,
                                                         const uint16_t *__restrict__ Kc, const uint16_t *__restrict__ Vc,
                                                         int maxT, StepArg st_arg, int len_imm) {
    constexpr int D = GPT2_HEAD_DIM;
    const int w = threadIdx.x >> 6, h = blockIdx.x;
    const int len = min(len_imm > 0 ? len_imm : st_arg.p() + 1, maxT);
    const int per = ((len + NW - 1) / NW + 7) & ~7;   // keys per wave (multiple of 8)
    const int j0 = min(len, w * per), j1 = min(len, j0 + per);
    f16x8 q[8];
    load_q(q, qkv + h * D);
    AttnState st;
    init_state(st);
    const uint16_t *kb = Kc + (size_t)h * maxT * D, *vb = Vc + (size_t)h * maxT * D;
    if (j0 < j1) attend_range(q, kb, vb, D, j0, j1, 0.125f, st);
    reduce_slots(st);
    merge_waves<NW>(st, att + h * D);
}

// Decode step, fused: appends this position's K and V (head h's 64 values of each) to the cache and
// attends over [0, pos], reading key/value pos from the qkv row itself.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_attn_decode_append(uint16_t *__restrict__ att, const uint16_t *__restrict__ qkv,
                                                                uint16_t *__restrict__ Kc, uint16_t *__restrict__ Vc,
                                                                int maxT, StepArg st_arg) {
    constexpr int E = GPT2_N_EMBD, D = GPT2_HEAD_DIM;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, h = blockIdx.x;
    const int pos = st_arg.p();
    if ((unsigned)pos >= (unsigned)maxT) return;   // uniform over the grid: nothing to attend
    const size_t hoff = (size_t)h * maxT * D;
    if (w == 0) {
        Kc[hoff + (size_t)pos * D + lane] = qkv[E + h * D + lane];
        Vc[hoff + (size_t)pos * D + lane] = qkv[2 * E + h * D + lane];
    }
    const int len = pos + 1;
    const int per = ((len + NW - 1) / NW + 7) & ~7;   // keys per wave (multiple of 8)
    const int j0 = min(len, w * per), j1 = min(len, j0 + per);
    f16x8 q[8];
    load_q(q, qkv + h * D);
    AttnState st;
    init_state(st);
    if (j0 < j1)
        attend_range(q, Kc + hoff, Vc + hoff, D, j0, j1, 0.125f, st, pos, qkv + E + h * D, qkv + 2 * E + h * D);
    reduce_slots(st);
    merge_waves<NW>(st, att + h * D);
}

// ------------------------------------------------------------------ KV cache writes
// Layout per layer: K[h][pos][d], V[h][pos][d] with d fastest (cuda/kvcache.cuh:150-151).
__global__ void k_kv_scatter(uint16_t *__restrict__ K, uint16_t *__restrict__ V, const uint16_t *__restrict__ qkv,
                             int T, int maxT) {
    constexpr int E = GPT2_N_EMBD, D = GPT2_HEAD_DIM;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;   // one 8-half chunk each
    if (idx >= (long)T * (E / 8)) return;
    const int t = (int)(idx / (E / 8)), c = (int)(idx % (E / 8));
    const int e = c * 8, h = e / D, d = e % D;
    const size_t off = ((size_t)h * maxT + t) * D + d;
    const uint16_t *row = qkv + (size_t)t * 3 * E;
    *reinterpret_cast<f16x8 *>(K + off) = *reinterpret_cast<const f16x8 *>(row + E + e);
    *reinterpret_cast<f16x8 *>(V + off) = *reinterpret_cast<const f16x8 *>(row + 2 * E + e);
}

__global__ void k_kv_append(uint16_t *__restrict__ K, uint16_t *__restrict__ V, const uint16_t *__restrict__ qkv,
                            StepArg st, int maxT) {
    constexpr int E = GPT2_N_EMBD, D = GPT2_HEAD_DIM;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= E) return;
    const int pos = st.p();
    if ((unsigned)pos >= (unsigned)maxT) return;
    const int h = i / D, d = i % D;
    const size_t off = ((size_t)h * maxT + pos) * D + d;
    K[off] = qkv[E + i];
    V[off] = qkv[2 * E + i];
}

// ------------------------------------------------------------------ greedy next token
// Argmax over fp16 logits[V] (lowest index among equal maxima, like argmax in
// bench/kv_gate.cu:56); writes tokens[pos+1] and advances the device state {token, pos}.
__global__ __launch_bounds__(1024) void k_argmax_advance(const uint16_t *__restrict__ logits, int V, int *__restrict__ state,
                                                         int *__restrict__ tokens, int max_pos) {
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < V; i += blockDim.x) {
        const float v = h2f(logits[i]);
        if (v > best) { best = v; bi = i; }   // i increases, so ties keep the first
    }
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
    }
    __shared__ float sv[16];
    __shared__ int si[16];
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = best; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nw = blockDim.x >> 6;
        for (int i = 1; i < nw; ++i)
            if (sv[i] > best || (sv[i] == best && si[i] < bi)) { best = sv[i]; bi = si[i]; }
        if (bi == 0x7fffffff) bi = 0;   // all NaN: token 0
        const int next = state[1] + 1;
        if (tokens && next < max_pos) tokens[next] = bi;
        state[0] = bi;
        state[1] = next;
    }
}

// ------------------------------------------------------------------ INT8 quantizer
// One wave per output row of an fp16 [N,K] tensor (tools/quantize.py:58-73):
//   absmax = max_k |w|;  s = absmax == 0 ? 1 : fl32(absmax / 127);  q = clamp(rint(fl32(w / s)), +-127)
// The divisions are IEEE float divisions (this file is built without fast-math; HIP's default
// float division is correctly rounded) and rintf is v_rndne_f32 (half to even).
__global__ __launch_bounds__(256) void k_quantize_rows(int8_t *__restrict__ q, float *__restrict__ s,
                                                       const uint16_t *__restrict__ w, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (row >= N) return;
    const uint16_t *wr = w + (size_t)row * K;
    float peak = 0.f;
    for (int k = lane; k < K; k += 64) peak = fmaxf(peak, fabsf(h2f(wr[k])));
    peak = wave_max(peak);
    const float scale = (peak == 0.f) ? 1.0f : peak / 127.0f;
    if (lane == 0) s[row] = scale;
    int8_t *qr = q + (size_t)row * K;
    for (int k = lane; k < K; k += 64) {
        float r = rintf(h2f(wr[k]) / scale);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        qr[k] = (int8_t)(int)r;
    }
}

// ------------------------------------------------------------------ host launchers (internal)
void embed_one(uint16_t *x, const uint16_t *wte, const uint16_t *wpe, StepArg st) {
    hipLaunchKernelGGL(k_embed_one, dim3(cdiv(GPT2_N_EMBD, 256)), dim3(256), 0, stream(), x, wte, wpe, st, GPT2_N_EMBD);
    check_launch("k_embed_one");
}

void kv_append(uint16_t *K, uint16_t *V, const uint16_t *qkv, StepArg st, int maxT) {
    hipLaunchKernelGGL(k_kv_append, dim3(cdiv(GPT2_N_EMBD, 256)), dim3(256), 0, stream(), K, V, qkv, st, maxT);
    check_launch("k_kv_append");
}

void attn_decode(uint16_t *att, const uint16_t *qkv, const uint16_t *K, const uint16_t *V, int maxT, StepArg st,
                 int len_imm) {
    hipLaunchKernelGGL(k_attn_decode<16>, dim3(GPT2_N_HEAD), dim3(1024), 0, stream(), att, qkv, K, V, maxT, st, len_imm);
    check_launch("k_attn_decode");
}

void attn_decode_append(uint16_t *att, const uint16_t *qkv, uint16_t *K, uint16_t *V, int maxT, StepArg st) {
    hipLaunchKernelGGL(k_attn_decode_append<16>, dim3(GPT2_N_HEAD), dim3(1024), 0, stream(), att, qkv, K, V, maxT, st);
    check_launch("k_attn_decode_append");
}

void argmax_advance(const uint16_t *logits, int V, int *state, int *tokens, int max_pos) {
    hipLaunchKernelGGL(k_argmax_advance, dim3(1), dim3(1024), 0, stream(), logits, V, state, tokens, max_pos);
    check_launch("k_argmax_advance");
}

}  // namespace g2

using namespace g2;

extern "C" void gpt2_embed(gpt2_half *x, const gpt2_half *wte, const gpt2_half *wpe, const int *ids, int T, int E) {
    if (T <= 0 || E <= 0) return;
    if (!x || !wte || !wpe || !ids) { arg_fail("gpt2_embed: null pointer"); return; }
    const long n = (long)T * E;
    hipLaunchKernelGGL(k_embed, dim3(cdiv(n, 256)), dim3(256), 0, stream(), x, wte, wpe, ids, T, E);
    check_launch("k_embed");
}

extern "C" void gpt2_layernorm(gpt2_half *out, const gpt2_half *x, const gpt2_half *g, const gpt2_half *b, int M,
                               int E) {
    if (M <= 0 || E <= 0) return;
    if (!out || !x || !g || !b) { arg_fail("gpt2_layernorm: null pointer"); return; }
    if (E == GPT2_N_EMBD && !(((uintptr_t)x | (uintptr_t)out | (uintptr_t)g | (uintptr_t)b) & 7u))
        hipLaunchKernelGGL(k_layernorm<true>, dim3(cdiv(M, 2)), dim3(128), 0, stream(), out, x, g, b, M, E);   // 2 rows per block
    else
        hipLaunchKernelGGL(k_layernorm<false>, dim3(cdiv(M, 4)), dim3(256), 0, stream(), out, x, g, b, M, E);
    check_launch("k_layernorm");
}

extern "C" void gpt2_gelu(gpt2_half *x, size_t n) {
    if (n == 0) return;
    if (!x) { arg_fail("gpt2_gelu: null pointer"); return; }
    if (n % 8 == 0 && aligned16(x)) {
        hipLaunchKernelGGL(k_gelu8, dim3(cdiv((long)(n / 8), 256)), dim3(256), 0, stream(), (f16x8 *)x, n / 8);
    } else {
        hipLaunchKernelGGL(k_gelu, dim3(cdiv((long)n, 256)), dim3(256), 0, stream(), x, n);
    }
    check_launch("k_gelu");
}

extern "C" void gpt2_add(gpt2_half *x, const gpt2_half *y, size_t n) {
    if (n == 0) return;
    if (!x || !y) { arg_fail("gpt2_add: null pointer"); return; }
    if (n % 8 == 0 && aligned16(x) && aligned16(y)) {
        hipLaunchKernelGGL(k_add8, dim3(cdiv((long)(n / 8), 256)), dim3(256), 0, stream(), (f16x8 *)x,
                           (const f16x8 *)y, n / 8);
    } else {
        hipLaunchKernelGGL(k_add, dim3(cdiv((long)n, 256)), dim3(256), 0, stream(), x, y, n);
    }
    check_launch("k_add");
}

extern "C" void gpt2_attention_flash(gpt2_half *att, const gpt2_half *qkv, int T, int E, int H, int D) {
    if (T <= 0) return;
    if (E != GPT2_N_EMBD || H != GPT2_N_HEAD || D != GPT2_HEAD_DIM || T > GPT2_N_CTX) {
        arg_fail("gpt2_attention_flash: only E=768, H=12, D=64, T<=1024");
        return;
    }
    if (!att || !qkv || !aligned16(att) || !aligned16(qkv)) { arg_fail("gpt2_attention_flash: null/unaligned"); return; }
    attention_prefill(att, qkv, T);
}

extern "C" void gpt2_quantize_rows(int8_t *q, float *s, const gpt2_half *w, int N, int K) {
    if (N <= 0 || K <= 0) return;
    if (!q || !s || !w) { arg_fail("gpt2_quantize_rows: null pointer"); return; }
    hipLaunchKernelGGL(k_quantize_rows, dim3(cdiv(N, 4)), dim3(256), 0, stream(), q, s, w, N, K);
    check_launch("k_quantize_rows");
}

extern "C" void gpt2_kv_scatter_prefill(GPT2KVCache *kv, int L, const gpt2_half *qkv, int T) {
    if (T <= 0) return;
    if (!kv || !kv->data || !qkv || L < 0 || L >= kv->nLayer || T > kv->maxT || !aligned16(qkv)) {
        arg_fail("gpt2_kv_scatter_prefill: bad cache, layer or length");
        return;
    }
    const long n = (long)T * (GPT2_N_EMBD / 8);
    hipLaunchKernelGGL(k_kv_scatter, dim3(cdiv(n, 256)), dim3(256), 0, stream(), gpt2_kv_K(kv, L), gpt2_kv_V(kv, L),
                       qkv, T, kv->maxT);
    check_launch("k_kv_scatter");
}

extern "C" void gpt2_embed_one(gpt2_half *x, const gpt2_half *wte, const gpt2_half *wpe, int token, int pos) {
    if (!x || !wte || !wpe) { arg_fail("gpt2_embed_one: null pointer"); return; }
    if (token < 0 || token >= GPT2_VOCAB || pos < 0 || pos >= GPT2_N_CTX) { arg_fail("gpt2_embed_one: token/pos range"); return; }
    embed_one(x, wte, wpe, StepArg{token, pos, nullptr});
}

extern "C" void gpt2_kv_append_one(GPT2KVCache *kv, int L, const gpt2_half *qkv, int pos) {
    if (!kv || !kv->data || !qkv || L < 0 || L >= kv->nLayer || pos < 0 || pos >= kv->maxT) {
        arg_fail("gpt2_kv_append_one: bad cache, layer or position");
        return;
    }
    kv_append(gpt2_kv_K(kv, L), gpt2_kv_V(kv, L), qkv, StepArg{0, pos, nullptr}, kv->maxT);
}

extern "C" void gpt2_attn_decode(gpt2_half *att, const gpt2_half *qkv, const GPT2KVCache *kv, int L, int len) {
    if (!kv || !kv->data || !att || !qkv || L < 0 || L >= kv->nLayer || len <= 0 || len > kv->maxT || !aligned16(qkv)) {
        arg_fail("gpt2_attn_decode: bad cache, layer or length");
        return;
    }
    attn_decode(att, qkv, gpt2_kv_K(kv, L), gpt2_kv_V(kv, L), kv->maxT, StepArg{0, 0, nullptr}, len);
}
