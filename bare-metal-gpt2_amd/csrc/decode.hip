// decode.hip -- the per-token decode step as ONE persistent kernel launch (gfx950).
//
// Replaces the ~62-launch step (cuda/kvcache.cu:233-269 in the reference, 135 launches there) for
// the backends whose GEMV slots are this library's GEMVs.  Why: on MI355X a dependent kernel
// launch costs ~2.4 us back to back and every small GEMV adds its own memory latency, so a token
// cost ~350 us while its weights (162 MB) stream from HBM in ~30 us.
//
// Design:
//   * PD_G work-groups (one per CU) run the whole step.  Work is split by output rows in every
//     phase; 12 layers x {LN1+QKV, attention, proj+residual, LN2+fc+gelu, mlp-proj+residual}, then
//     LN_f + tied head + argmax.
//   * Phases exchange their (small) output vectors through "flag words": 64-bit words holding 32 bits
//     of data and the 32-bit sequence number of the phase that wrote them, stored and loaded with
//     agent-scope (coherent, sc1) atomic accesses.  A consumer polls the words it needs until every
//     flag matches; there is no fence, no counter and no grid barrier (measured: a fenced grid barrier
//     costs 16 us at 256 work-groups, a flag-word phase ~2.3 us).  64-bit accesses are single-copy
//     atomic, so data and flag arrive together.
//   * Each phase issues its weight loads (straight into registers) before it polls for its input,
//     so HBM latency hides behind the exchange.
//   * Sequence numbers are epoch*64 + phase, with the epoch a device counter advanced once per token,
//     so buffers are reused without clearing and a replay at a repeated position cannot match a
//     stale word.  Every buffer is rewritten only after all of its readers have provably finished
//     (each phase reads the complete output of the phase before it).
//   * Every poll is bounded; on timeout (or once another work-group reported one) the work-group
//     records an error in `err` and leaves, so the kernel always terminates.
//   * KV rows of this token are appended to the cache with ordinary stores; later tokens read them
//     in later launches (kernel boundaries make them visible), this token's attention reads its own
//     key/value from the exchanged qkv vector.
//
// Numerics follow the multi-kernel fused step: fp16 activations between phases, fp32 inside,
// LayerNorm with biased variance and eps inside the sqrt, gelu_new, scale after the fp32 sum then
// bias (then residual), online-softmax attention with scale 1/8, greedy argmax over the fp16 logits
// with the lowest index among equal maxima.
#include <cmath>
#include <type_traits>

#include "attn.h"
#include "common.h"
#include "decode.h"

namespace g2 {

constexpr int PD_G = 256;                          // work-groups
constexpr int PD_T = 256;                          // threads per work-group (4 waves)
constexpr int PD_S = 2;                            // key splits per head (attention work-groups: H*S)
constexpr int PD_NC = 2;                           // 64-key chunks per attention wave
constexpr int PD_E = GPT2_N_EMBD, PD_Q = GPT2_QKV_DIM, PD_F = GPT2_FFN_DIM, PD_V = GPT2_VOCAB;
constexpr int PD_D = GPT2_HEAD_DIM, PD_H = GPT2_N_HEAD;
constexpr int PD_PW = 2 + PD_D;                    // words per attention partial: m, l, c[64]
constexpr int RQ = PD_Q / PD_G, RP = PD_E / PD_G, RF = PD_F / PD_G, RM = PD_E / PD_G;
constexpr int RH = (PD_V + PD_G - 1) / PD_G;       // head rows per work-group (the last has fewer)
static_assert(RQ * PD_G == PD_Q && RP * PD_G == PD_E && RF * PD_G == PD_F, "rows split evenly");
static_assert(RF % 2 == 0, "fc rows are exchanged in pairs");
static_assert(PD_G == PD_T, "the final argmax gives each thread one work-group's candidate");
static_assert(PD_H * PD_S <= PD_G, "one work-group per attention split");
static_assert(PD_S * 4 * 64 * PD_NC >= GPT2_N_CTX, "the attention waves cover every key of a full cache");

// Exchange arena (64-bit flag words).
constexpr int LL_X = 0;                            // residual stream: 768 words, one fp16 each
constexpr int LL_QKV = LL_X + PD_E;                // qkv: 2304 words, one fp16 each
constexpr int LL_ATT = LL_QKV + PD_Q;              // attention partials: H*S*66 words, fp32
constexpr int LL_HID = LL_ATT + PD_H * PD_S * PD_PW;  // gelu(fc): 1536 words, two fp16 each
constexpr int LL_CAND = LL_HID + PD_F / 2;         // argmax candidates: G words
constexpr int LL_WORDS = LL_CAND + PD_G;
constexpr int PD_SPIN = 1 << 15;                   // default poll rounds before a work-group gives up

__device__ __forceinline__ uint64_t ll_ld(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_st(uint64_t *p, uint32_t data, uint32_t flag) {
    __hip_atomic_store(p, ((uint64_t)flag << 32) | data, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls words idx(i), i in [0, n), of `base` (R per thread, all loads in flight before any check)
// until every flag equals `flag`, then calls sink(i, data).  Returns false (for the whole
// work-group) if a word did not arrive within `spin` rounds or another work-group reported an
// error; the caller then leaves.
template <int R, class Idx, class Sink>
__device__ bool ll_read(const uint64_t *base, int n, uint32_t flag, int *err, int spin, Idx idx, Sink sink) {
    uint64_t v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + PD_T * r;
        v[r] = (i < n) ? ll_ld(base + idx(i)) : ((uint64_t)flag << 32);
    }
    bool bad = false;
    for (int round = 0;; ++round) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < R; ++r) ok &= (uint32_t)(v[r] >> 32) == flag;
        if (ok) break;
        if (round >= spin || ((round & 63) == 63 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
            bad = true;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = threadIdx.x + PD_T * r;
            if (i < n && (uint32_t)(v[r] >> 32) != flag) v[r] = ll_ld(base + idx(i));
        }
    }
    if (__syncthreads_or(bad)) {
        if (threadIdx.x == 0) atomicOr(err, 1);
        return false;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + PD_T * r;
        if (i < n) sink(i, (uint32_t)v[r]);
    }
    __syncthreads();
    return true;
}

// ------------------------------------------------------------------------------ row GEMV pieces
// One wave computes one output row: lane l holds K/64 consecutive-in-groups elements of the row.
//   K=768  int8 : 3 x 4 codes  at element 4l + 256i      fp16: 3 x 4 halves at 4l + 256i
//   K=3072 int8 : 3 x 16 codes at element 16l + 1024i    fp16: 6 x 8 halves at 8l + 512i
template <int K, bool Q8> struct RowSpec;
template <> struct RowSpec<768, true> { static constexpr int NL = 3, EL = 4; using T = uint32_t; };
template <> struct RowSpec<768, false> { static constexpr int NL = 3, EL = 4; using T = uint2; };
template <> struct RowSpec<3072, true> { static constexpr int NL = 3, EL = 16; using T = uint4; };
template <> struct RowSpec<3072, false> { static constexpr int NL = 6, EL = 8; using T = uint4; };

template <int K, bool Q8>
struct RowW {
    typename RowSpec<K, Q8>::T w[RowSpec<K, Q8>::NL];
};

template <int K, bool Q8>
__device__ __forceinline__ void load_row(RowW<K, Q8> &r, const void *W, int row, int lane) {
    using S = RowSpec<K, Q8>;
    const char *base = reinterpret_cast<const char *>(W) + (size_t)row * K * (Q8 ? 1 : 2);
#pragma unroll
    for (int i = 0; i < S::NL; ++i) {
        const int e = S::EL * lane + 64 * S::EL * i;
        r.w[i] = *reinterpret_cast<const typename S::T *>(base + (size_t)e * (Q8 ? 1 : 2));
    }
}

template <int K, bool Q8>
__device__ __forceinline__ float dot_row(const RowW<K, Q8> &r, const f16 *x, int lane) {
    using S = RowSpec<K, Q8>;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < S::NL; ++i) {
        const int e = S::EL * lane + 64 * S::EL * i;
        if constexpr (S::EL == 4) {
            const f16x4 xv = *reinterpret_cast<const f16x4 *>(x + e);
            f16x2 a, b;
            if constexpr (Q8) {
                i8x4_to_f16x4_v(r.w[i], a, b);
            } else {
                a = __builtin_bit_cast(f16x2, r.w[i].x);
                b = __builtin_bit_cast(f16x2, r.w[i].y);
            }
            acc = __builtin_amdgcn_fdot2(a, f16x2{xv[0], xv[1]}, acc, false);
            acc = __builtin_amdgcn_fdot2(b, f16x2{xv[2], xv[3]}, acc, false);
        } else if constexpr (S::EL == 8) {
            const f16x8 xv = *reinterpret_cast<const f16x8 *>(x + e);
            const uint32_t wd[4] = {r.w[i].x, r.w[i].y, r.w[i].z, r.w[i].w};
#pragma unroll
            for (int t = 0; t < 4; ++t)
                acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, wd[t]), f16x2{xv[2 * t], xv[2 * t + 1]}, acc, false);
        } else {
            const f16x8 x0 = *reinterpret_cast<const f16x8 *>(x + e);
            const f16x8 x1 = *reinterpret_cast<const f16x8 *>(x + e + 8);
            const uint32_t wd[4] = {r.w[i].x, r.w[i].y, r.w[i].z, r.w[i].w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                f16x2 a, b;
                i8x4_to_f16x4_v(wd[t], a, b);
                const f16x8 &xv = (t < 2) ? x0 : x1;
                const int o = (t & 1) * 4;
                acc = __builtin_amdgcn_fdot2(a, f16x2{xv[o], xv[o + 1]}, acc, false);
                acc = __builtin_amdgcn_fdot2(b, f16x2{xv[o + 2], xv[o + 3]}, acc, false);
            }
        }
    }
    return acc;
}

// The rows r0 + wave + 4j (j < J) of this work-group's share, loaded before the phase's input
// arrives, with their scale and bias.
template <int K, bool Q8, int ROWS>
struct PhaseW {
    static constexpr int J = (ROWS + 3) / 4;
    RowW<K, Q8> r[J];
    float s[J], b[J];
};

template <int K, bool Q8, int ROWS>
__device__ __forceinline__ void load_phase(PhaseW<K, Q8, ROWS> &P, const void *W, const float *S, const uint16_t *B,
                                           int r0, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < PhaseW<K, Q8, ROWS>::J; ++j) {
        const int k = wave + 4 * j;
        if (k < ROWS) {
            load_row<K, Q8>(P.r[j], W, r0 + k, lane);
            P.s[j] = Q8 ? S[r0 + k] : 1.0f;
            P.b[j] = B ? h2f(B[r0 + k]) : 0.0f;
        }
    }
}

// acc * scale + bias for each of the wave's rows; out(k, value) gets the row index inside the share.
template <int K, bool Q8, int ROWS, class Out>
__device__ __forceinline__ void run_phase(const PhaseW<K, Q8, ROWS> &P, const f16 *x, int wave, int lane, Out out) {
    constexpr int J = PhaseW<K, Q8, ROWS>::J;
    float acc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = (wave + 4 * j < ROWS) ? dot_row<K, Q8>(P.r[j], x, lane) : 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = wave_sum_u(acc[j]);   // independent reductions, interleaved
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int k = wave + 4 * j;
        if (k < ROWS) out(k, acc[j] * P.s[j] + P.b[j]);
    }
}

// LayerNorm of the 768-vector xs into xn (fp16): every wave computes the statistics (same order,
// same result), then thread t writes elements t, t+256, t+512.
// gamma and beta of the thread's three elements, loaded before the phase's input arrives.
struct LNParams {
    float g[3], b[3];
};
__device__ __forceinline__ void load_ln(LNParams &p, const uint16_t *g, const uint16_t *b) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int e = threadIdx.x + PD_T * i;
        p.g[i] = h2f(g[e]);
        p.b[i] = h2f(b[e]);
    }
}

__device__ __forceinline__ void layernorm768(f16 *xn, const f16 *xs, const LNParams &p, int lane) {
    float v[12], s = 0.f;
#pragma unroll
    for (int i = 0; i < 12; ++i) {
        v[i] = (float)xs[lane + 64 * i];
        s += v[i];
    }
    const float mean = wave_sum_u(s) * (1.0f / PD_E);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < 12; ++i) {
        const float d = v[i] - mean;
        q += d * d;
    }
    const float rstd = 1.0f / sqrtf(wave_sum_u(q) * (1.0f / PD_E) + GPT2_LN_EPS);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int e = threadIdx.x + PD_T * i;
        xn[e] = (f16)(((float)xs[e] - mean) * rstd * p.g[i] + p.b[i]);
    }
    __syncthreads();
}

// ------------------------------------------------------------------------------ the step
__global__ __launch_bounds__(PD_T) void k_decode_persist(PDArgs a) {
    __shared__ __attribute__((aligned(16))) f16 xs[PD_E];     // current residual stream
    __shared__ __attribute__((aligned(16))) f16 xn[PD_E];     // normalized input / attention output
    __shared__ __attribute__((aligned(16))) f16 hs[PD_F];     // gelu(fc) for the mlp-proj phase
    __shared__ __attribute__((aligned(16))) float part[PD_H * PD_S * PD_PW];
    __shared__ __attribute__((aligned(16))) f16 qkvh[3 * PD_D];  // q, k, v of one head
    __shared__ float sm[4], sl[4];
    __shared__ __attribute__((aligned(16))) float cl[4][PD_D][8];      // attention: [wave][dim][key slot]
    __shared__ __attribute__((aligned(16))) float pl[4][PD_NC][64];    // attention: probabilities, transposed
    __shared__ uint16_t hout[RF];
    __shared__ float bv[4];
    __shared__ int bi[4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wg = blockIdx.x;
    const int token = a.state[0], pos = a.state[1];
    const uint32_t epoch = (uint32_t)a.state[2];
    if ((unsigned)pos >= (unsigned)a.maxT || (unsigned)token >= (unsigned)PD_V) return;   // uniform
    auto seq = [&](int phase) { return epoch * 64u + (uint32_t)phase; };
    auto mark = [&](int phase) {
        if (a.trace && tid == 0) a.trace[wg * 128 + phase] = __builtin_amdgcn_s_memrealtime();
    };
    mark(63);
    if (a.trace && tid == 0 && wg == 0) a.trace[126] = __builtin_amdgcn_s_memtime();
    uint64_t *LX = a.ll + LL_X, *LQ = a.ll + LL_QKV, *LA = a.ll + LL_ATT, *LHd = a.ll + LL_HID, *LC = a.ll + LL_CAND;
    const size_t hstride = (size_t)a.maxT * PD_D;


    auto read_x = [&](uint32_t flag) {
        return ll_read<3>(LX, PD_E, flag, a.err, a.spin, [](int i) { return i; },
                          [&](int i, uint32_t d) { xs[i] = __builtin_bit_cast(f16, (uint16_t)d); });
    };

    for (int l = 0; l < GPT2_N_LAYER; ++l) {
        const PDLayer &ly = a.layers[l];
        const int ph = 5 * l;
        // ---- Q: LN1 + QKV rows [wg*RQ, +RQ)
        {
            const bool q8 = ly.s[0] != nullptr;
            PhaseW<768, true, RQ> P8;
            PhaseW<768, false, RQ> P16;
            if (q8) load_phase(P8, ly.w[0], ly.s[0], ly.b[0], wg * RQ, wave, lane);
            else load_phase(P16, ly.w[0], nullptr, ly.b[0], wg * RQ, wave, lane);
            LNParams lnp;
            load_ln(lnp, ly.ln1_g, ly.ln1_b);
            if (l == 0) {
                // embed: x = fp16(wte[token] + wpe[pos]) (every work-group, no exchange)
#pragma unroll
                for (int i = 0; i < 3; ++i) {
                    const int e = tid + PD_T * i;
                    xs[e] = (f16)(h2f(a.wte[(size_t)token * PD_E + e]) + h2f(a.wpe[(size_t)pos * PD_E + e]));
                }
                __syncthreads();
            } else if (!read_x(seq(ph - 1))) {
                return;
            }
            mark(64 + ph);
            layernorm768(xn, xs, lnp, lane);
            auto out = [&](int k, float v) {
                if (lane == 0) ll_st(LQ + wg * RQ + k, __builtin_bit_cast(uint16_t, (f16)v), seq(ph));
            };
            if (q8) run_phase(P8, xn, wave, lane, out);
            else run_phase(P16, xn, wave, lane, out);
            mark(ph);
        }
        // ---- A: attention, head h, key split sp (work-groups 0 .. H*S-1); each wave takes up to
        // PD_NC chunks of 64 keys.  Keys and values of past positions do not depend on this token,
        // so each lane loads its key rows and value slices before q arrives; key `pos` comes from the
        // exchanged qkv.  One softmax pass over the wave's keys (no rescaling between chunks).
        if (wg < PD_H * PD_S) {
            const int h = wg / PD_S, sp = wg % PD_S;
            uint16_t *Kc = a.kv + (size_t)(2 * l) * PD_H * hstride + h * hstride;
            uint16_t *Vc = a.kv + (size_t)(2 * l + 1) * PD_H * hstride + h * hstride;
            const int len = pos + 1;
            const int per = (len + PD_S - 1) / PD_S;
            const int j0 = min(len, sp * per), j1 = min(len, j0 + per);
            const int w0 = min(j1, j0 + 64 * PD_NC * wave), w1 = min(j1, w0 + 64 * PD_NC);
            const int slot = lane >> 3, dg = (lane & 7) * 8;
            const f16x8 z8 = {};
            f16x8 kr[PD_NC][8], vr[PD_NC][8];
#pragma unroll
            for (int ch = 0; ch < PD_NC; ++ch) {
                const int jk = w0 + 64 * ch + lane;
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    kr[ch][c] = (jk < w1 && jk != pos) ? *reinterpret_cast<const f16x8 *>(Kc + (size_t)jk * PD_D + 8 * c) : z8;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int key = w0 + 64 * ch + slot + 8 * t;
                    vr[ch][t] = (key < w1 && key != pos) ? *reinterpret_cast<const f16x8 *>(Vc + (size_t)key * PD_D + dg) : z8;
                }
            }
            auto qidx = [h](int i) { return (i >> 6) * PD_E + h * PD_D + (i & 63); };
            if (!ll_read<1>(LQ, 3 * PD_D, seq(ph), a.err, a.spin, qidx,
                            [&](int i, uint32_t d) { qkvh[i] = __builtin_bit_cast(f16, (uint16_t)d); }))
                return;
            mark(64 + ph + 1);
            if (sp == 0 && tid < PD_D) {
                Kc[(size_t)pos * PD_D + tid] = __builtin_bit_cast(uint16_t, qkvh[PD_D + tid]);
                Vc[(size_t)pos * PD_D + tid] = __builtin_bit_cast(uint16_t, qkvh[2 * PD_D + tid]);
            }
            // Scores: lane = key of each chunk.  m and l are wave-uniform; the probabilities go to
            // LDS transposed so that lane (slot, dg) reads the eight it needs (keys slot + 8t) as two
            // 16-byte loads, and its context slice (8 dims over its 8 keys) goes back to LDS for the
            // cross-slot, cross-wave merge.
            float m_w = -INFINITY, l_w = 0.f;
            float cacc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (w0 < w1) {
                f16x8 q[8];
                load_q(q, reinterpret_cast<const uint16_t *>(qkvh));
                float sv[PD_NC], pv[PD_NC];
                float mloc = -INFINITY;
#pragma unroll
                for (int ch = 0; ch < PD_NC; ++ch) {
                    const int jk = w0 + 64 * ch + lane;
                    if (jk == pos) load_q(kr[ch], reinterpret_cast<const uint16_t *>(qkvh + PD_D));
                    sv[ch] = -INFINITY;
                    if (jk < w1) {
                        float d0 = 0.f, d1 = 0.f;
#pragma unroll
                        for (int c = 0; c < 8; ++c)
#pragma unroll
                            for (int t = 0; t < 4; t += 2) {
                                d0 = __builtin_amdgcn_fdot2(f16x2{q[c][2 * t], q[c][2 * t + 1]},
                                                            f16x2{kr[ch][c][2 * t], kr[ch][c][2 * t + 1]}, d0, false);
                                d1 = __builtin_amdgcn_fdot2(f16x2{q[c][2 * t + 2], q[c][2 * t + 3]},
                                                            f16x2{kr[ch][c][2 * t + 2], kr[ch][c][2 * t + 3]}, d1, false);
                            }
                        sv[ch] = (d0 + d1) * 0.125f;
                    }
                    mloc = fmaxf(mloc, sv[ch]);
                }
                m_w = wave_max_u(mloc);   // finite: key w0 is in range
                float psum = 0.f;
#pragma unroll
                for (int ch = 0; ch < PD_NC; ++ch) {
                    pv[ch] = (w0 + 64 * ch + lane < w1) ? __expf(sv[ch] - m_w) : 0.f;
                    psum += pv[ch];
                    pl[wave][ch][(lane & 7) * 8 + (lane >> 3)] = pv[ch];
                }
                l_w = wave_sum_u(psum);
#pragma unroll
                for (int ch = 0; ch < PD_NC; ++ch) {
                    const float4 pa = *reinterpret_cast<const float4 *>(&pl[wave][ch][slot * 8]);
                    const float4 pb = *reinterpret_cast<const float4 *>(&pl[wave][ch][slot * 8 + 4]);
                    const float pr[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const int key = w0 + 64 * ch + slot + 8 * t;
                        const f16x8 vv = (key == pos) ? *reinterpret_cast<const f16x8 *>(qkvh + 2 * PD_D + dg) : vr[ch][t];
#pragma unroll
                        for (int e = 0; e < 8; ++e) cacc[e] += pr[t] * (float)vv[e];   // p = 0 past w1
                    }
                }
            }
            // context slices to LDS: cl[wave][dim][slot]
#pragma unroll
            for (int e = 0; e < 8; ++e) cl[wave][dg + e][slot] = cacc[e];
            if (lane == 0) {
                sm[wave] = m_w;
                sl[wave] = l_w;
            }
            __syncthreads();
            // unnormalized partial over the work-group's keys: m, l, c[64]
            if (tid < PD_PW) {
                float mx = -INFINITY;
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    if (sl[w] != 0.f) mx = fmaxf(mx, sm[w]);
                float val = (tid == 0) ? mx : 0.f;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    if (sl[w] == 0.f) continue;
                    const float f = __expf(sm[w] - mx);
                    if (tid == 1) val += sl[w] * f;
                    if (tid >= 2) {
                        const float4 ca = *reinterpret_cast<const float4 *>(&cl[w][tid - 2][0]);
                        const float4 cb = *reinterpret_cast<const float4 *>(&cl[w][tid - 2][4]);
                        val += (((ca.x + ca.y) + (ca.z + ca.w)) + ((cb.x + cb.y) + (cb.z + cb.w))) * f;
                    }
                }
                ll_st(LA + (h * PD_S + sp) * PD_PW + tid, __float_as_uint(val), seq(ph + 1));
            }
            __syncthreads();
            mark(ph + 1);
        }
        // ---- P: combine heads, proj rows [wg*RP, +RP), + bias + residual
        {
            const bool q8 = ly.s[1] != nullptr;
            PhaseW<768, true, RP> P8;
            PhaseW<768, false, RP> P16;
            if (q8) load_phase(P8, ly.w[1], ly.s[1], ly.b[1], wg * RP, wave, lane);
            else load_phase(P16, ly.w[1], nullptr, ly.b[1], wg * RP, wave, lane);
            constexpr int NA = PD_H * PD_S * PD_PW;
            if (!ll_read<(NA + PD_T - 1) / PD_T>(LA, NA, seq(ph + 1), a.err, a.spin, [](int i) { return i; },
                                                 [&](int i, uint32_t d) { part[i] = __uint_as_float(d); }))
                return;
            mark(64 + ph + 2);
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const int e = tid + PD_T * i, h = e / PD_D, d = e % PD_D;
                float mx = -INFINITY;
#pragma unroll
                for (int s = 0; s < PD_S; ++s) {
                    const float *p = part + (h * PD_S + s) * PD_PW;
                    if (p[1] != 0.f) mx = fmaxf(mx, p[0]);
                }
                float L = 0.f, c = 0.f;
#pragma unroll
                for (int s = 0; s < PD_S; ++s) {
                    const float *p = part + (h * PD_S + s) * PD_PW;
                    if (p[1] == 0.f) continue;
                    const float f = __expf(p[0] - mx);
                    L += p[1] * f;
                    c += p[2 + d] * f;
                }
                xn[e] = (f16)(c / L);
            }
            __syncthreads();
            auto out = [&](int k, float v) {
                const int r = wg * RP + k;
                if (lane == 0) ll_st(LX + r, __builtin_bit_cast(uint16_t, (f16)(v + (float)xs[r])), seq(ph + 2));
            };
            if (q8) run_phase(P8, xn, wave, lane, out);
            else run_phase(P16, xn, wave, lane, out);
            mark(ph + 2);
        }
        // ---- F: LN2 + fc rows [wg*RF, +RF) + gelu, exchanged in pairs
        {
            const bool q8 = ly.s[2] != nullptr;
            PhaseW<768, true, RF> P8;
            PhaseW<768, false, RF> P16;
            if (q8) load_phase(P8, ly.w[2], ly.s[2], ly.b[2], wg * RF, wave, lane);
            else load_phase(P16, ly.w[2], nullptr, ly.b[2], wg * RF, wave, lane);
            LNParams lnp;
            load_ln(lnp, ly.ln2_g, ly.ln2_b);
            if (!read_x(seq(ph + 2))) return;
            mark(64 + ph + 3);
            layernorm768(xn, xs, lnp, lane);
            auto out = [&](int k, float v) {
                if (lane == 0) hout[k] = __builtin_bit_cast(uint16_t, (f16)gelu_tanh(v));
            };
            if (q8) run_phase(P8, xn, wave, lane, out);
            else run_phase(P16, xn, wave, lane, out);
            __syncthreads();
            if (tid < RF / 2)
                ll_st(LHd + wg * (RF / 2) + tid, (uint32_t)hout[2 * tid] | ((uint32_t)hout[2 * tid + 1] << 16), seq(ph + 3));
            mark(ph + 3);
        }
        // ---- M: mlp-proj rows [wg*RM, +RM) over gelu(fc), + bias + residual
        {
            const bool q8 = ly.s[3] != nullptr;
            PhaseW<3072, true, RM> P8;
            PhaseW<3072, false, RM> P16;
            if (q8) load_phase(P8, ly.w[3], ly.s[3], ly.b[3], wg * RM, wave, lane);
            else load_phase(P16, ly.w[3], nullptr, ly.b[3], wg * RM, wave, lane);
            if (!ll_read<PD_F / 2 / PD_T>(LHd, PD_F / 2, seq(ph + 3), a.err, a.spin, [](int i) { return i; },
                                          [&](int i, uint32_t d) {
                                              hs[2 * i] = __builtin_bit_cast(f16, (uint16_t)(d & 0xffff));
                                              hs[2 * i + 1] = __builtin_bit_cast(f16, (uint16_t)(d >> 16));
                                          }))
                return;
            mark(64 + ph + 4);
            auto out = [&](int k, float v) {
                const int r = wg * RM + k;
                if (lane == 0) ll_st(LX + r, __builtin_bit_cast(uint16_t, (f16)(v + (float)xs[r])), seq(ph + 4));
            };
            if (q8) run_phase(P8, hs, wave, lane, out);
            else run_phase(P16, hs, wave, lane, out);
            mark(ph + 4);
        }
    }

    // ---- head: LN_f, logits rows [wg*RH, ...), local argmax, then work-group 0 picks the token
    const int ph = 5 * GPT2_N_LAYER;
    LNParams lnf;
    load_ln(lnf, a.lnf_g, a.lnf_b);
    if (!read_x(seq(ph - 1))) return;
    layernorm768(xn, xs, lnf, lane);
    const int r0 = wg * RH, r1 = min(PD_V, r0 + RH);
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    // 16 lanes per row (4 rows per wave per pass, 16 rows per work-group pass), each lane CPL
    // 16-byte chunks j, j+16, ...; HD passes of loads in flight per wave (the persistent step has only
    // four waves per CU, so the memory parallelism comes from inside the wave).
    auto head_rows = [&](auto q8tag) {
        constexpr bool Q8 = decltype(q8tag)::value;
        constexpr int CPL = Q8 ? 3 : 6, HD = 4;
        const int j = lane & 15, slot = lane >> 4;
        f16x8 xr[Q8 ? 2 * CPL : CPL];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            if constexpr (Q8) {
                xr[2 * i] = *reinterpret_cast<const f16x8 *>(xn + (j + 16 * i) * 16);
                xr[2 * i + 1] = *reinterpret_cast<const f16x8 *>(xn + (j + 16 * i) * 16 + 8);
            } else {
                xr[i] = *reinterpret_cast<const f16x8 *>(xn + (j + 16 * i) * 8);
            }
        }
        constexpr int ROWB = Q8 ? PD_E : 2 * PD_E;
        const char *W = reinterpret_cast<const char *>(a.head_w);
        uint4 ring[HD][CPL];
        auto issue = [&](uint4(&buf)[CPL], int pass) {
            const int r = r0 + 16 * pass + 4 * wave + slot;
#pragma unroll
            for (int i = 0; i < CPL; ++i)
                buf[i] = (r < r1) ? *reinterpret_cast<const uint4 *>(W + (size_t)r * ROWB + (j + 16 * i) * 16)
                                  : uint4{0, 0, 0, 0};
        };
        auto consume = [&](const uint4(&buf)[CPL], int pass) {
            const int r = r0 + 16 * pass + 4 * wave + slot;
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const uint32_t wd[4] = {buf[i].x, buf[i].y, buf[i].z, buf[i].w};
                if constexpr (Q8) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        f16x2 lo, hi;
                        i8x4_to_f16x4_v(wd[t], lo, hi);
                        const f16x8 &xv = xr[2 * i + (t >> 1)];
                        const int o = (t & 1) * 4;
                        acc = __builtin_amdgcn_fdot2(lo, f16x2{xv[o], xv[o + 1]}, acc, false);
                        acc = __builtin_amdgcn_fdot2(hi, f16x2{xv[o + 2], xv[o + 3]}, acc, false);
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, wd[t]), f16x2{xr[i][2 * t], xr[i][2 * t + 1]},
                                                     acc, false);
                }
            }
            acc = row16_sum(acc);
            if (r < r1) {
                float v = acc;
                if constexpr (Q8) v *= a.head_s[r];
                const uint16_t hv = __builtin_bit_cast(uint16_t, (f16)v);
                if (j == 0) a.logits[r] = hv;
                const float fv = h2f(hv);
                if (fv > best) { best = fv; bidx = r; }   // a lane's rows ascend: ties keep the first
            }
        };
        const int npass = (r1 - r0 + 15) / 16;
#pragma unroll
        for (int d = 0; d < HD; ++d) issue(ring[d], d);
        for (int p0 = 0; p0 < npass; p0 += HD) {
#pragma unroll
            for (int d = 0; d < HD; ++d) {
                if (p0 + d < npass) {
                    consume(ring[d], p0 + d);
                    issue(ring[d], p0 + d + HD);
                }
            }
        }
        // (best, bidx) over the lanes of the wave: larger value, then lower index
        for (int o = 1; o < 64; o <<= 1) {
            const float ov = __shfl_xor(best, o, 64);
            const int oi = __shfl_xor(bidx, o, 64);
            if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
        }
    };
    mark(60);
    if (a.head_s) head_rows(std::integral_constant<bool, true>{});
    else head_rows(std::integral_constant<bool, false>{});
    mark(61);
    if (lane == 0) {
        bv[wave] = best;
        bi[wave] = bidx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w)
            if (bv[w] > best || (bv[w] == best && bi[w] < bidx)) { best = bv[w]; bidx = bi[w]; }
        const uint32_t cand = (bidx == 0x7fffffff) ? 0xffffu
                                                   : ((uint32_t)__builtin_bit_cast(uint16_t, (f16)best) << 16) | (uint32_t)bidx;
        ll_st(LC + wg, cand, seq(ph));
    }
    if (wg != 0) return;
    // work-group 0: argmax over the candidates, advance the state
    __shared__ uint32_t cands[PD_G];
    if (!ll_read<(PD_G + PD_T - 1) / PD_T>(LC, PD_G, seq(ph), a.err, a.spin, [](int i) { return i; },
                                          [&](int i, uint32_t d) { cands[i] = d; }))
        return;
    {
        // thread i holds candidate i; (larger value, then lower index) wins
        const uint32_t c = cands[tid];
        float bvv = ((c & 0xffffu) == 0xffffu) ? -INFINITY : h2f((uint16_t)(c >> 16));
        int bii = ((c & 0xffffu) == 0xffffu) ? 0x7fffffff : (int)(c & 0xffffu);
        for (int o = 1; o < 64; o <<= 1) {
            const float ov = __shfl_xor(bvv, o, 64);
            const int oi = __shfl_xor(bii, o, 64);
            if (ov > bvv || (ov == bvv && oi < bii)) { bvv = ov; bii = oi; }
        }
        if (lane == 0) {
            bv[wave] = bvv;
            bi[wave] = bii;
        }
    }
    __syncthreads();
    if (tid == 0) {
        float bvv = bv[0];
        int bii = bi[0];
        for (int w = 1; w < 4; ++w)
            if (bv[w] > bvv || (bv[w] == bvv && bi[w] < bii)) { bvv = bv[w]; bii = bi[w]; }
        if (bii == 0x7fffffff) bii = 0;   // all NaN: token 0
        const int next = pos + 1;
        if (a.tokens && next < a.maxT) a.tokens[next] = bii;
        a.state[0] = bii;
        a.state[1] = next;
        a.state[2] = (int)(epoch + 1);
    }
    mark(62);
    if (a.trace && tid == 0) a.trace[127] = __builtin_amdgcn_s_memtime();
}

// ------------------------------------------------------------------------------ host side
static int g_pd_spin = PD_SPIN;
static unsigned long long *g_pd_trace = nullptr;

// Builds the step's argument block; returns false when the backend or weights need the
// multi-kernel step (the caller falls back to it).
bool persist_plan(PDPlan &p, const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv, uint16_t *logits,
                  int *state, int *tokens, uint64_t *ll, int *err) {
    if (be->gemv != gpt2_gemv_fp16) return false;
    const bool q_ok = be->gemv_q == gpt2_gemv_int8;
    const GPT2QWeightsGPU *qw = w->q;
    PDLayer h[GPT2_N_LAYER];
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        const GPT2LayerGPU &g = w->layers[L];
        const GPT2QLayerGPU *ql = qw ? &qw->layers[L] : nullptr;
        h[L].ln1_g = g.ln1_g;
        h[L].ln1_b = g.ln1_b;
        h[L].ln2_g = g.ln2_g;
        h[L].ln2_b = g.ln2_b;
        const gpt2_half *wh[4] = {g.qkv_w, g.attn_proj_w, g.fc_w, g.proj_w};
        const gpt2_half *bh[4] = {g.qkv_b, g.attn_proj_b, g.fc_b, g.proj_b};
        const GPT2QW *wq[4] = {ql ? &ql->qkv_w : nullptr, ql ? &ql->attn_proj_w : nullptr, ql ? &ql->fc_w : nullptr,
                               ql ? &ql->proj_w : nullptr};
        for (int i = 0; i < 4; ++i) {
            const bool q = q_ok && wq[i] && wq[i]->q;
            h[L].w[i] = q ? (const void *)wq[i]->q : (const void *)wh[i];
            h[L].s[i] = q ? wq[i]->s : nullptr;
            h[L].b[i] = bh[i];
        }
    }
    p.d_layers = (PDLayer *)gpt2_dmalloc(sizeof(h));
    if (!p.d_layers || gpt2_h2d(p.d_layers, h, sizeof(h))) return false;
    PDArgs &a = p.args;
    a.layers = p.d_layers;
    a.wte = w->wte;
    a.wpe = w->wpe;
    a.lnf_g = w->lnf_g;
    a.lnf_b = w->lnf_b;
    const bool hq = q_ok && qw && qw->wte.q;
    a.head_w = hq ? (const void *)qw->wte.q : (const void *)w->wte;
    a.head_s = hq ? qw->wte.s : nullptr;
    a.kv = kv->data;
    a.maxT = kv->maxT;
    a.logits = logits;
    a.state = state;
    a.tokens = tokens;
    a.ll = ll;
    a.err = err;
    a.spin = g_pd_spin;
    a.trace = g_pd_trace;
    return true;
}

void persist_launch(const PDPlan &p, hipStream_t s) {
    hipLaunchKernelGGL(k_decode_persist, dim3(PD_G), dim3(PD_T), 0, s, p.args);
}

size_t persist_ll_bytes() { return (size_t)LL_WORDS * 8; }

}  // namespace g2

// Tuning / test hook: poll rounds before a persistent step gives up, for graphs created afterwards
// (< 0 restores the default; 0 gives up at the first poll that finds a word missing).  A tiny value
// forces the timeout path with every kernel still exiting normally.
extern "C" void gpt2_tune_decode_spin(int rounds) { g2::g_pd_spin = rounds >= 0 ? rounds : g2::PD_SPIN; }
// Profiling hook: graphs created afterwards record, per work-group, the end time of every phase of
// the persistent step (s_memrealtime, 100 MHz) into trace[wg * 64 + phase]: 5*l + {0 qkv, 1 attention,
// 2 proj, 3 fc, 4 mlp-proj}, 60 head start, 61 head end, 62 step end, 63 step start, and at 64 + p
// the time phase p's input had arrived; work-group 0 also stores the shader clock counter at step
// start and end in entries 126 / 127.  The buffer holds 256 * 128 entries; nullptr disables.
extern "C" void gpt2_tune_decode_trace(unsigned long long *trace) { g2::g_pd_trace = trace; }

namespace g2 {

void persist_free(PDPlan &p) {
    gpt2_dfree(p.d_layers);
    p.d_layers = nullptr;
}

}  // namespace g2
