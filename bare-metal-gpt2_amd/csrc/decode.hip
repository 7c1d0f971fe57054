// decode.hip -- the per-token decode step as ONE persistent kernel launch (gfx950).
//
// Replaces the ~62-launch step (cuda/kvcache.cu:233-269 in the reference, 135 launches there) for
// the backends whose GEMV slots are this library's GEMVs.  Why: on MI355X a dependent kernel
// launch costs ~2.4 us back to back and every small GEMV adds its own memory latency, so a token
// cost ~350 us while its weights (162 MB) stream from HBM in ~30 us.
//
// Design:
//   * PD_G work-groups (one per CU) run the whole step, in four phases per layer:
//       A  48 attention work-groups, four per head (key splits): LN1 of x, the head's q and the
//          split's 16-row slices of k and v of the new key (96 weight rows on the matrix cores, their
//          fragments loaded into accumulation registers during the previous layer), the K/V
//          append, attention over the split's share of the earlier keys; they send an unnormalized
//          partial (m, l, c[64]) plus the slice's part of q.k_new and its v_new slice.
//       P  192 GEMV work-groups: combine the partials (the new key is one more partial), proj rows,
//          + bias + residual.
//       F  the same work-groups: LN2, fc rows (one 16-row block on the matrix cores), gelu.
//       M  the same work-groups: mlp-proj rows + bias + residual.
//     then LN_f + tied head + argmax on every work-group, and work-group 0 picks the token.
//   * Phases exchange their (small) output vectors through "flag words": 64-bit words holding 32 bits
//     of data and the 32-bit sequence number of the phase that wrote them, stored and loaded with
//     agent-scope (coherent, sc1) atomic accesses.  A consumer polls the words it needs until every
//     flag matches; there is no fence, no counter and no grid barrier (measured: a fenced grid barrier
//     costs 16 us at 256 work-groups, a flag-word exchange ~1.5-2.5 us).  64-bit accesses are
//     single-copy atomic, so data and flag arrive together.
//   * Every phase's weights are in flight before its input arrives: GEMV rows go to registers one
//     phase ahead (issued right after the previous poll completed, so a poll never queues behind
//     them), the attention work-groups' q/k/v fragments a layer ahead.  Barriers between waves
//     wait for LDS traffic only, so they do not drain those loads; per-layer pointers come from the
//     kernel argument segment (scalar loads) and fp16 parameters stay unconverted until used, since
//     either would otherwise make the wave wait for every load it has in flight.
//   * Sequence numbers are epoch*64 + phase, with the epoch a device counter advanced once per token,
//     so buffers are reused without clearing and a replay at a repeated position cannot match a
//     stale word.  A work-group polls a buffer only in a phase it also writes from, so every writer
//     of a buffer's next version has first read everything the previous version's readers needed.
//   * Every poll is bounded; on timeout (or once another work-group reported one) the work-group
//     records an error in `err` and leaves, so the kernel always terminates.
//   * KV rows of this token are appended to the cache with ordinary stores; later tokens read them
//     in later launches (kernel boundaries make them visible); this token's attention takes the new
//     key and value from the exchanged words instead.
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

constexpr int PD_G = 256;                          // work-groups (one per CU)
constexpr int PD_T = 256;                          // threads per work-group (4 waves)
constexpr int PD_E = GPT2_N_EMBD, PD_F = GPT2_FFN_DIM, PD_V = GPT2_VOCAB;
constexpr int PD_D = GPT2_HEAD_DIM, PD_H = GPT2_N_HEAD;
constexpr int PD_S = 4;                            // attention work-groups (key splits) per head
constexpr int PD_NA = PD_H * PD_S;                 // attention work-groups: 0 .. NA-1
constexpr int PD_NG = PD_G - PD_NA;                // GEMV work-groups: NA .. G-1
constexpr int KS = PD_D / PD_S;                    // k and v rows of key `pos` per attention work-group
constexpr int QR = PD_D + 2 * KS;                  // rows it computes: q (64), its k slice, its v slice
// Words an attention work-group sends: m and l (fp32), c/l (its 64 context values divided by l: a
// weighted mean of values) as 32 fp16 pairs, its part of q.k_pos (fp32), its v_pos slice as fp16 pairs.
constexpr int AW_M = 0, AW_L = 1, AW_C = 2, AW_S = AW_C + PD_D / 2, AW_V = AW_S + 1;
constexpr int PD_PW = AW_V + KS / 2;
constexpr int RP = 4, RF = 16, RM = 4;             // rows per GEMV work-group: proj, fc, mlp-proj
constexpr int PD_NW = PD_E / RP;                   // GEMV work-groups with rows (the rest wait for the head)
constexpr int RH = (PD_V + PD_G - 1) / PD_G;       // head rows per work-group (the last has fewer)
constexpr int XW = PD_E / 2;                       // x words: two fp16 each
constexpr int XR = (XW + PD_T - 1) / PD_T;         // words of x each thread polls
static_assert(PD_E % RP == 0 && PD_F % RF == 0 && PD_E / RP == PD_F / RF && RM == RP && PD_NW <= PD_NG,
              "the same GEMV work-groups hold proj, fc and mlp-proj rows");
static_assert(RF % 2 == 0 && RP % 2 == 0, "fc rows and x rows are exchanged in pairs");
static_assert(QR % 32 == 0, "the q/k/v GEMV takes two 16-row passes at a time");
static_assert(PD_G == PD_T, "the final argmax gives each thread one work-group's candidate");
static_assert(PD_S * 4 * 64 >= GPT2_N_CTX, "an attention wave holds at most 64 keys of a full cache");

// Exchange arena (64-bit flag words).
// Each writing work-group's words start on their own 128-byte line (16 words): lines written by
// work-groups on different XCDs were measurably slower to become visible.
constexpr int LINE = 16;                           // words per 128-byte line
constexpr int pad_line(int n) { return (n + LINE - 1) / LINE * LINE; }
constexpr int XS_W = pad_line(RP / 2);             // x: RP/2 words (fp16 pairs) per GEMV work-group
constexpr int AT_W = pad_line(PD_PW);              // attention: PW words per attention work-group
constexpr int HD_W = pad_line(RF / 2);             // gelu(fc): RF/2 words (fp16 pairs) per GEMV work-group
constexpr int LL_X = 0;                            // residual stream: 384 words, two fp16 each
constexpr int LL_ATT = LL_X + PD_NW * XS_W;        // attention: NA*PW words, fp32
constexpr int LL_HID = LL_ATT + PD_NA * AT_W;      // gelu(fc): 1536 words, two fp16 each
constexpr int LL_CAND = LL_HID + PD_NW * HD_W;     // argmax candidates: one word per work-group
constexpr int LL_WORDS = LL_CAND + PD_G * LINE;
// word of element i of each buffer
__device__ __forceinline__ int x_word(int i) { return (i / (RP / 2)) * XS_W + i % (RP / 2); }   // pair i
__device__ __forceinline__ int at_word(int i) { return (i / PD_PW) * AT_W + i % PD_PW; }
__device__ __forceinline__ int hd_word(int i) { return (i / (RF / 2)) * HD_W + i % (RF / 2); }
__device__ __forceinline__ int cand_word(int i) { return i * LINE; }
constexpr int PD_SPIN = 1 << 15;                   // default poll rounds before a work-group gives up
// Hold-offs before a GEMV work-group's polls, in s_memrealtime ticks (10 ns), counted from its own
// previous store.  A poll issued right after the work-group's own store, or long before the words
// can arrive, slows the exchanges of the whole step (its loads wait behind the store's write-through
// and load the memory side while the other work-groups' stores drain).  Measured per token at
// ctx 512 (interleaved A/B): 163.5 us with none against 156.3 with 2.5 / 0.6 / 0.5 us, and 300 / 60 /
// 40 ticks 0.8% faster again; the attention words arrive ~4 us after the mlp-proj store, x and
// gelu(fc) ~1.3 us after the store before them.  Holds that follow each layer's measured arrival
// (the previous layer's arrival minus a margin of one to three poll rounds, up and down or only
// down) measured 1-1.3% slower than these constants at every margin tried.  gpt2_tune_decode_holds
// sets them per graph.
constexpr unsigned PD_HOLD_ATT = 300;              // after the mlp-proj store, before the attention words
constexpr unsigned PD_HOLD_X = 60;                 // after the proj store, before x
constexpr unsigned PD_HOLD_HID = 40;               // after the fc store, before gelu(fc)
// Phase numbers (sequence = epoch*64 + phase): per layer l, 4l attention, 4l+1 x after proj,
// 4l+2 gelu(fc), 4l+3 x after mlp-proj; 48 head candidates.
constexpr int PH_CAND = 4 * GPT2_N_LAYER;

// LDS layout (bytes).  Common: xs, xn, argmax scratch.  Attention work-groups: the four waves'
// partial sums of the q/k/v GEMV, reused for the attention scratch, and q, the k slice and the v slice;
// GEMV work-groups: gelu(fc) and the attention words (their space also takes the fc partial sums).
constexpr int LDS_XS = 0, LDS_XN = LDS_XS + 2 * PD_E, LDS_MISC = LDS_XN + 2 * PD_E;   // misc: 512 B
constexpr int LDS_ROLE = LDS_MISC + 512;
struct Lds {
    static constexpr int RED = LDS_ROLE;                  // A: [4][QR] fp32 q/k/v partial sums
    static constexpr int CL = LDS_ROLE;                   // A, after the GEMV: [4][64][8] fp32
    static constexpr int PL = CL + 4 * PD_D * 8 * 4;      // A, after the GEMV: [4][64] fp32
    static constexpr int QKVH = PL + 4 * 64 * 4;          // A: q, k slice, v slice (fp16)
    static constexpr int HS = LDS_ROLE;                   // G: gelu(fc), 3072 fp16
    static constexpr int PART = HS + 2 * PD_F;            // G: NA*PW fp32
    static constexpr int CANDS = LDS_ROLE;                // head phase: G candidates
    static constexpr int BYTES_A = QKVH + 2 * QR, BYTES_G = PART + 4 * PD_NA * PD_PW;
    static constexpr int BYTES = BYTES_A > BYTES_G ? BYTES_A : BYTES_G;
    static_assert(RED + 4 * 4 * QR <= QKVH && CANDS + 4 * PD_G <= BYTES, "LDS layout");
};

__device__ __forceinline__ uint64_t ll_ld(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_st(uint64_t *p, uint32_t data, uint32_t flag) {
    __hip_atomic_store(p, ((uint64_t)flag << 32) | data, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spins (s_sleep) until the 100 MHz real-time counter reaches t; wave-uniform, ends by itself.
__device__ __forceinline__ void hold_until(unsigned long long t) {
    while (__builtin_amdgcn_s_memrealtime() < t) __builtin_amdgcn_s_sleep(4);
}

// Polls elements [0, n) of `base` (R per thread, element tid + 256r at word idx(i); all loads in
// flight before any check)
// until every flag equals `flag`, then calls sink(i, data).  Returns false (for the whole
// work-group) if a word did not arrive within `spin` rounds or another work-group reported an
// error; the caller then leaves.  wflag: 4 ints of LDS for the work-group's verdict; dbg (optional,
// profiling): thread 0 stores the start time and the number of extra poll rounds there.
static_assert(PD_T == 256, "ll_read combines four waves");
template <int R, class Idx, class Sink>
__device__ bool ll_read(const uint64_t *base, int n, uint32_t flag, int *err, int spin, int *wflag, Idx idx,
                        Sink sink, unsigned long long *dbg = nullptr) {
    if (dbg && threadIdx.x == 0) dbg[0] = __builtin_amdgcn_s_memrealtime();
    uint64_t v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = ll_ld(base + idx(min((int)threadIdx.x + PD_T * r, n - 1)));
    bool bad = false;
    for (int round = 0;; ++round) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < R; ++r) ok &= (int)threadIdx.x + PD_T * r >= n || (uint32_t)(v[r] >> 32) == flag;
        if (__all(ok)) {
            if (dbg && threadIdx.x == 0) dbg[1] = round;
            break;
        }
        if (round >= spin || ((round & 63) == 63 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
            bad = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);   // 64 clocks between rounds (measured: 1 beats 0, 2, 4 and 8)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = threadIdx.x + PD_T * r;
            if (i < n && (uint32_t)(v[r] >> 32) != flag) v[r] = ll_ld(base + idx(i));
        }
    }
    // The loop is wave-uniform, so `bad` is too.  Barriers here wait for LDS traffic only, so they
    // do not drain loads issued before the poll.
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) wflag[wave] = bad;
    lds_barrier();
    if (wflag[0] | wflag[1] | wflag[2] | wflag[3]) {
        if (threadIdx.x == 0) atomicOr(err, 1);
        return false;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + PD_T * r;
        if (i < n) sink(i, (uint32_t)v[r]);
    }
    lds_barrier();
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
    float s[J];
    uint16_t b[J];   // fp16 bits, converted where used (a conversion here would wait for the load)
};

template <int K, bool Q8, int ROWS>
__device__ __forceinline__ void load_phase(PhaseW<K, Q8, ROWS> &P, const void *W, const float *S, const uint16_t *B,
                                           int r0, int wave, int lane, int limit = ROWS) {
#pragma unroll
    for (int j = 0; j < PhaseW<K, Q8, ROWS>::J; ++j) {
        const int k = wave + 4 * j;
        if (k < ROWS && k < limit) {
            load_row<K, Q8>(P.r[j], W, r0 + k, lane);
            P.s[j] = Q8 ? S[r0 + k] : 1.0f;
            P.b[j] = B[r0 + k];
        }
    }
}

// acc * scale + bias for each of the wave's rows; out(k, value) gets the row index inside the share.
template <int K, bool Q8, int ROWS, class Out>
__device__ __forceinline__ void run_phase(const PhaseW<K, Q8, ROWS> &P, const f16 *x, int wave, int lane, Out out,
                                          int limit = ROWS) {
    constexpr int J = PhaseW<K, Q8, ROWS>::J;
    float acc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int k = wave + 4 * j;
        acc[j] = (k < ROWS && k < limit) ? dot_row<K, Q8>(P.r[j], x, lane) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = wave_sum_u(acc[j]);   // independent reductions, interleaved
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int k = wave + 4 * j;
        if (k < ROWS && k < limit) out(k, acc[j] * P.s[j] + h2f(P.b[j]));
    }
}

// LayerNorm of the 768-vector xs into xn (fp16): every wave computes the statistics (same order,
// same result; lane l sums elements 12l .. 12l+11), then thread t writes elements t, t+256, t+512.
// gamma and beta of the thread's three elements, loaded before the phase's input arrives.
struct LNParams {
    uint16_t g[3], b[3];   // fp16 bits: converting at load time would make the load wait at once
};
__device__ __forceinline__ void load_ln(LNParams &p, const uint16_t *g, const uint16_t *b) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int e = threadIdx.x + PD_T * i;
        p.g[i] = g[e];
        p.b[i] = b[e];
    }
}

// The lane's twelve values are summed as a tree (the latency is two reductions long, not 24 adds),
// and rstd is the hardware reciprocal square root (1 ulp).
__device__ __forceinline__ float sum12(const float (&v)[12]) {
    return (((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]))) + ((v[8] + v[9]) + (v[10] + v[11]));
}
__device__ __forceinline__ void layernorm768(f16 *xn, const f16 *xs, const LNParams &p, int lane) {
    float v[12], xe[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const f16x4 x4 = *reinterpret_cast<const f16x4 *>(xs + 12 * lane + 4 * i);
#pragma unroll
        for (int t = 0; t < 4; ++t) v[4 * i + t] = (float)x4[t];
        xe[i] = (float)xs[threadIdx.x + PD_T * i];
    }
    const float mean = wave_sum_u(sum12(v)) * (1.0f / PD_E);
    float d2[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) {
        const float d = v[i] - mean;
        d2[i] = d * d;
    }
    const float rstd = __builtin_amdgcn_rsqf(wave_sum_u(sum12(d2)) * (1.0f / PD_E) + GPT2_LN_EPS);
#pragma unroll
    for (int i = 0; i < 3; ++i) xn[threadIdx.x + PD_T * i] = (f16)((xe[i] - mean) * rstd * h2f(p.g[i]) + h2f(p.b[i]));
    lds_barrier();
}

// ------------------------------------------------------------------------------ the step
// Row r of the q/k/v rows attention work-group (h, sp) computes: q rows 0-63 of head h, then k and
// v rows [KS*sp, KS*sp + KS) of head h, as row indices of the [3*768][768] c_attn weight.
__device__ __forceinline__ int qkv_row(int h, int sp, int r) {
    return r < PD_D ? h * PD_D + r
                    : (r < PD_D + KS ? PD_E : 2 * PD_E) + h * PD_D + KS * sp + ((r - PD_D) & (KS - 1));
}

// The q/k/v GEMV on the matrix cores, its weights held in accumulation registers (AGPRs).  The QR rows
// are QB blocks of 16 (v_mfma_f32_16x16x32_f16 A-fragments); wave w takes elements [192w, 192w + 192)
// of every row in QS k-steps of 32, so the GEMV is QB * QS MFMAs per wave and a four-way sum.  Lane l
// holds, for block b and k-step s, row 16b + (l & 15) at elements qk_k(w, s, l) .. +7 (k-steps paired
// so that a lane's two chunks of a pair are 16 consecutive elements: one 16-byte load of int8 codes).
// The B operand is the normalized x at the same elements in every column, so every column of D holds
// the GEMV.  These registers are otherwise unused by the attention work-groups; held there, the
// fragments cost no LDS reads (staged in LDS, the QR rows were 147 KB of LDS reads per layer: 163.7
// against 156.6 us per token, INT8, interleaved A/B).
constexpr int QB = QR / 16;                       // row blocks
constexpr int QKW = PD_E / 4;                     // elements of K per wave
constexpr int QS = QKW / 32;                      // k-steps per wave
static_assert(QR % 16 == 0 && QKW % 64 == 0, "whole blocks and whole k-step pairs");
__device__ __forceinline__ int qk_k(int wave, int s, int lane) {
    return QKW * wave + 64 * (s >> 1) + 16 * (lane >> 4) + 8 * (s & 1);
}

// Loads this wave's fragments of the QR rows (exact fp16; int8 codes widened) and moves them to the
// accumulation registers.  Called when the attention work-group is idle (after its words of a layer
// went out, before the next x arrives), so the wait for the loads costs nothing on the critical path.
// The loads are all issued before the first is consumed (the compiler barrier keeps them there).
template <bool Q8>
__device__ __forceinline__ void stage_qkv_acc(i32x4 (&wq)[QB * QS], const void *W, int h, int sp, int wave, int lane) {
    const int r = lane & 15;
    if constexpr (Q8) {
        const int8_t *Wb = reinterpret_cast<const int8_t *>(W);
        i32x4 c[QB * QS / 2];
#pragma unroll
        for (int b = 0; b < QB; ++b)
#pragma unroll
            for (int p = 0; p < QS / 2; ++p)
                c[b * QS / 2 + p] =
                    *reinterpret_cast<const i32x4 *>(Wb + (size_t)qkv_row(h, sp, 16 * b + r) * PD_E + qk_k(wave, 2 * p, lane));
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < QB * QS / 2; ++i) {
            const i32x4 v = c[i];
            const i32x4 lo = __builtin_bit_cast(i32x4, i8x8_to_f16x8(uint2{(uint32_t)v[0], (uint32_t)v[1]}));
            const i32x4 hi = __builtin_bit_cast(i32x4, i8x8_to_f16x8(uint2{(uint32_t)v[2], (uint32_t)v[3]}));
            asm volatile("" : "=a"(wq[2 * i]) : "0"(lo));
            asm volatile("" : "=a"(wq[2 * i + 1]) : "0"(hi));
        }
    } else {
        const uint16_t *Wh = reinterpret_cast<const uint16_t *>(W);
        i32x4 v[QB * QS];
#pragma unroll
        for (int b = 0; b < QB; ++b)
#pragma unroll
            for (int s = 0; s < QS; ++s)
                v[b * QS + s] =
                    *reinterpret_cast<const i32x4 *>(Wh + (size_t)qkv_row(h, sp, 16 * b + r) * PD_E + qk_k(wave, s, lane));
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < QB * QS; ++i) asm volatile("" : "=a"(wq[i]) : "0"(v[i]));
    }
}

// A GEMV work-group's RF = 16 fc rows as one block of MFMA A-fragments, k-steps laid out as in the
// q/k/v GEMV (wave w: elements [192w, 192w + 192)): fp16, six 16-byte fragments per lane; int8, three
// 16-byte groups of 16 codes, widened when used.  Threads 0-15 also hold their row's scale and bias.
static_assert(RF == 16, "the fc rows of a work-group are one 16-row MFMA block");
template <bool Q8>
struct FcW {
    i32x4 w[Q8 ? QS / 2 : QS];
    float s;
    uint16_t b;   // fp16 bits
};
template <bool Q8>
__device__ __forceinline__ void load_fc(FcW<Q8> &F, const void *W, const float *S, const uint16_t *B, int r0, int wave,
                                        int lane) {
    const int row = r0 + (lane & 15);
#pragma unroll
    for (int i = 0; i < (Q8 ? QS / 2 : QS); ++i) {
        const int k = qk_k(wave, Q8 ? 2 * i : i, lane);
        F.w[i] = Q8 ? *reinterpret_cast<const i32x4 *>(reinterpret_cast<const int8_t *>(W) + (size_t)row * PD_E + k)
                    : *reinterpret_cast<const i32x4 *>(reinterpret_cast<const uint16_t *>(W) + (size_t)row * PD_E + k);
    }
    if (threadIdx.x < RF) {
        F.s = Q8 ? S[r0 + threadIdx.x] : 1.f;
        F.b = B[r0 + threadIdx.x];
    }
}

// Q8: every layer matrix is int8 codes with per-row scales (else every one is fp16).
template <bool Q8>
__global__ __launch_bounds__(PD_T) void k_decode_persist(PDArgs a) {
    using LY = Lds;
    __shared__ __attribute__((aligned(1024))) char lds[LY::BYTES];
    f16 *xs = reinterpret_cast<f16 *>(lds + LDS_XS);      // current residual stream
    f16 *xn = reinterpret_cast<f16 *>(lds + LDS_XN);      // normalized input / attention output
    float *bv = reinterpret_cast<float *>(lds + LDS_MISC);
    int *bi = reinterpret_cast<int *>(lds + LDS_MISC + 16);
    float *sm = reinterpret_cast<float *>(lds + LDS_MISC + 32), *sl = reinterpret_cast<float *>(lds + LDS_MISC + 48);
    uint16_t *hout = reinterpret_cast<uint16_t *>(lds + LDS_MISC + 64);   // RF values
    int *wflag = reinterpret_cast<int *>(lds + LDS_MISC + 96);             // ll_read verdicts, 4 ints
    uint32_t *xout = reinterpret_cast<uint32_t *>(lds + LDS_MISC + 112);   // RP x words, one store
    // misc + 128: the q.k_pos part (attention work-groups); + 256: the heads' weights (GEMV work-groups)
    static_assert(64 + 2 * RF <= 96 && 112 + 4 * RP <= 128 && 256 + 4 * 16 * 4 <= 512, "LDS misc layout");

    // wave < 4 made explicit (PD_T = 256): a wave's share of GEMV rows (wave + 4j < ROWS) is then
    // known at compile time, with no branch around the row dot products ahead of their reductions.
    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3, wg = blockIdx.x;
    const int token = a.state[0], pos = a.state[1];
    const uint32_t epoch = (uint32_t)a.state[2];
    const int spin = a.state[4];   // poll rounds before giving up
    if ((unsigned)pos >= (unsigned)a.maxT || (unsigned)token >= (unsigned)PD_V) return;   // uniform
    auto seq = [&](int phase) { return epoch * 64u + (uint32_t)phase; };
    auto mark = [&](int phase) {
        if (a.trace && tid == 0) a.trace[wg * 128 + phase] = __builtin_amdgcn_s_memrealtime();
    };
    mark(63);
    if (a.trace && tid == 0 && wg == 0) a.trace[126] = __builtin_amdgcn_s_memtime();
    uint64_t *LX = a.ll + LL_X, *LA = a.ll + LL_ATT, *LHd = a.ll + LL_HID, *LC = a.ll + LL_CAND;
    const size_t hstride = (size_t)a.maxT * PD_D;

    auto read_x = [&](uint32_t flag, unsigned long long *dbg = nullptr) {
        return ll_read<XR>(LX, XW, flag, a.err, spin, wflag, x_word, [&](int i, uint32_t d) {
            reinterpret_cast<uint32_t *>(xs)[i] = d;   // elements 2i, 2i + 1
        }, dbg);
    };

    if (wg < PD_NA) {
        // ================================ attention work-group: head h, key split sp
        // Per layer: LN1 of x; the head's q and this split's slices of k and v of key `pos`, from
        // the weight fragments loaded during the previous layer; the K/V append of those slices;
        // attention of q over the split's share of keys [0, pos); then the unnormalized partial
        // (m, l, c[64]), the slice's share of q.k_pos and the v_pos slice to the exchange.  The
        // combiner treats key `pos` as one more partial (m = q.k_pos / 8, l = 1, c = v_pos).
        const int h = wg / PD_S, sp = wg % PD_S;
        const int per = (pos + PD_S - 1) / PD_S;
        const int j0 = min(pos, sp * per), j1 = min(pos, j0 + per);
        const int pw = (j1 - j0 + 3) / 4;                  // keys per wave, <= 64 (maxT <= N_CTX)
        const int w0 = min(j1, j0 + pw * wave), w1 = min(j1, w0 + pw);
        const int slot = lane >> 3, dg = (lane & 7) * 8;
        f16 *qkvh = reinterpret_cast<f16 *>(lds + LY::QKVH);
        float(*cl)[PD_D][8] = reinterpret_cast<float(*)[PD_D][8]>(lds + LY::CL);
        float(*pl)[64] = reinterpret_cast<float(*)[64]>(lds + LY::PL);
        // The embedding's loads go first: the memory counter completes in issue order, so loads
        // issued after the weight DMA would have to wait for it.
        uint16_t emb_t[3], emb_p[3];   // fp16 bits of wte[token], wpe[pos] at elements tid + 256i
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            emb_t[i] = a.wte[(size_t)token * PD_E + tid + PD_T * i];
            emb_p[i] = a.wpe[(size_t)pos * PD_E + tid + PD_T * i];
        }
        // The wave's keys and values of layer l (zero past w1).
        f16x8 kr[8], vr[8];
        auto load_kv = [&](int l) {
            const uint16_t *Kc = a.kv + (size_t)(2 * l) * PD_H * hstride + h * hstride;
            const uint16_t *Vc = Kc + (size_t)PD_H * hstride;
            const f16x8 z8 = {};
            const int jk = w0 + lane;
#pragma unroll
            for (int c = 0; c < 8; ++c)
                kr[c] = (jk < w1) ? *reinterpret_cast<const f16x8 *>(Kc + (size_t)jk * PD_D + 8 * c) : z8;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int key = w0 + slot + 8 * t;
                vr[t] = (key < w1) ? *reinterpret_cast<const f16x8 *>(Vc + (size_t)key * PD_D + dg) : z8;
            }
        };
        // Layer 0's keys and values go out before its weight rows, so their latency overlaps the
        // staging (later layers load theirs while waiting for x).
        load_kv(0);
        i32x4 wq[QB * QS];   // this wave's q/k/v fragments, in accumulation registers
        stage_qkv_acc<Q8>(wq, a.layers[0].w[0], h, sp, wave, lane);
        for (int l = 0; l < GPT2_N_LAYER; ++l) {
            const PDLayer &ly = a.layers[l];
            uint16_t *Kc = a.kv + (size_t)(2 * l) * PD_H * hstride + h * hstride;
            uint16_t *Vc = a.kv + (size_t)(2 * l + 1) * PD_H * hstride + h * hstride;
            // ---- before the input arrives: the wave's keys/values, LN1 params, q/k/v scales and biases
            if (l > 0) load_kv(l);
            LNParams lnp;
            load_ln(lnp, ly.ln1_g, ly.ln1_b);
            float rs = 1.f;
            uint16_t rb = 0;   // fp16 bits
            if (tid < QR) {
                const int gr = qkv_row(h, sp, tid);
                rs = Q8 ? ly.s[0][gr] : 1.f;
                rb = ly.b[0][gr];
            }
            // ---- x: embed (layer 0) or the previous layer's output
            if (l == 0) {
#pragma unroll
                for (int i = 0; i < 3; ++i) xs[tid + PD_T * i] = (f16)(h2f(emb_t[i]) + h2f(emb_p[i]));
                lds_barrier();
            } else if (!read_x(seq(4 * l - 1), (l == 1 && a.trace) ? a.trace + wg * 128 + 122 : nullptr)) {
                return;
            }
            mark(64 + 4 * l);
            if (l == 1) mark(113);
            layernorm768(xn, xs, lnp, lane);   // ends with a barrier
            if (l == 1) mark(114);
            {
                // QB * QS MFMAs per wave over its K range; lanes 0, 16, 32, 48 (column 0 of D) hold rows
                // 16b + 4(l / 16) .. +3 of block b; the four waves' partials are summed in wave order.
                f16x8 xv[QS];
#pragma unroll
                for (int s2 = 0; s2 < QS; ++s2) xv[s2] = *reinterpret_cast<const f16x8 *>(xn + qk_k(wave, s2, lane));
                f32x4 acc[QB];
#pragma unroll
                for (int b = 0; b < QB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s2 = 0; s2 < QS; ++s2)
#pragma unroll
                    for (int b = 0; b < QB; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, wq[b * QS + s2]), xv[s2],
                                                                        acc[b], 0, 0, 0);
                float *red = reinterpret_cast<float *>(lds + LY::RED);   // free until the attention scratch
                if ((lane & 15) == 0) {
#pragma unroll
                    for (int b = 0; b < QB; ++b)
                        *reinterpret_cast<f32x4 *>(red + wave * QR + 16 * b + 4 * (lane >> 4)) = acc[b];
                }
                lds_barrier();
                if (tid < QR) {
                    const float v = ((red[tid] + red[QR + tid]) + red[2 * QR + tid]) + red[3 * QR + tid];
                    qkvh[tid] = (f16)(v * rs + h2f(rb));
                }
            }
            lds_barrier();
            if (l == 1) mark(115);
            if (tid < KS) {
                Kc[(size_t)pos * PD_D + KS * sp + tid] = __builtin_bit_cast(uint16_t, qkvh[PD_D + tid]);
                Vc[(size_t)pos * PD_D + KS * sp + tid] = __builtin_bit_cast(uint16_t, qkvh[PD_D + KS + tid]);
            }
            // This split's part of q.k_pos (fp32 products of the fp16 values, summed over the 16-lane
            // row): wave 3, which has the fewest keys, before its attention.
            float *sdot = reinterpret_cast<float *>(lds + LDS_MISC + 128);
            if (__builtin_amdgcn_readfirstlane(wave) == 3) {   // a scalar branch: the DPP sum sees every lane
                const float pq = lane < KS ? (float)qkvh[KS * sp + lane] * (float)qkvh[PD_D + lane] : 0.f;
                const float d = row16_sum(pq);
                if (lane == 0) *sdot = d;
            }
            // ---- attention over the wave's keys (one softmax pass), then the work-group merge
            float m_w = -INFINITY, l_w = 0.f;
            float cacc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (w0 < w1) {
                f16x8 q[8];
                load_q(q, reinterpret_cast<const uint16_t *>(qkvh));
                const bool on = w0 + lane < w1;
                // Every lane computes its dot product (kr is zero past w1) and the out-of-range lanes
                // are masked by a select afterwards: no lane-divergent branch precedes the DPP
                // reduction, so every lane of the row holds a value the select wrote.
                float dd[4] = {0.f, 0.f, 0.f, 0.f};   // four independent chains of eight
#pragma unroll
                for (int c = 0; c < 8; ++c)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        dd[2 * (c & 1) + (t >> 1)] = __builtin_amdgcn_fdot2(f16x2{q[c][2 * t], q[c][2 * t + 1]},
                                                                            f16x2{kr[c][2 * t], kr[c][2 * t + 1]},
                                                                            dd[2 * (c & 1) + (t >> 1)], false);
                const float sv = on ? ((dd[0] + dd[1]) + (dd[2] + dd[3])) * 0.125f : -INFINITY;
                m_w = wave_max_u(sv);   // finite: key w0 is in range
                const float pv = on ? __expf(sv - m_w) : 0.f;
                pl[wave][(lane & 7) * 8 + (lane >> 3)] = pv;
                l_w = wave_sum_u(pv);
                const float4 pa = *reinterpret_cast<const float4 *>(&pl[wave][slot * 8]);
                const float4 pb = *reinterpret_cast<const float4 *>(&pl[wave][slot * 8 + 4]);
                const float pr[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
                // keys w0 + slot + 8t: past the wave's last key p is 0, so those terms are skipped
                const int nt = __builtin_amdgcn_readfirstlane((w1 - w0 + 7) >> 3);
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    if (t < nt) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) cacc[e] += pr[t] * (float)vr[t][e];
                    }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) cl[wave][dg + e][slot] = cacc[e];
            // Each wave sums its eight slots of every dimension itself (lane = dimension; its own
            // LDS writes above come first, in order), so the merge below reads one value per wave and
            // dimension.
            float *cs = &pl[wave][0];   // the wave's softmax scratch, free again
            {
                const float4 ca = *reinterpret_cast<const float4 *>(&cl[wave][lane][0]);
                const float4 cb = *reinterpret_cast<const float4 *>(&cl[wave][lane][4]);
                cs[lane] = ((ca.x + ca.y) + (ca.z + ca.w)) + ((cb.x + cb.y) + (cb.z + cb.w));
            }
            if (lane == 0) {
                sm[wave] = m_w;
                sl[wave] = l_w;
            }
            if (l == 1) mark(116);
            lds_barrier();
            if (l == 1) mark(117);
            if (tid < PD_PW) {
                uint32_t val = 0;
                if (tid < AW_S) {
                    // the four waves' partials merged, branch-free (independent LDS reads)
                    float mw[4], lw[4], fw[4];
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        mw[w] = sm[w];
                        lw[w] = sl[w];
                    }
                    float mx = -INFINITY;
#pragma unroll
                    for (int w = 0; w < 4; ++w) mx = (lw[w] != 0.f) ? fmaxf(mx, mw[w]) : mx;
                    float lsum = 0.f;
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        fw[w] = (lw[w] != 0.f) ? __expf(mw[w] - mx) : 0.f;
                        lsum += lw[w] * fw[w];
                    }
                    if (tid == AW_M) {
                        val = __float_as_uint(mx);
                    } else if (tid == AW_L) {
                        val = __float_as_uint(lsum);
                    } else {
                        const int d0 = 2 * (tid - AW_C);
                        float c2[2] = {0.f, 0.f};
#pragma unroll
                        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
                            for (int w = 0; w < 4; ++w) c2[h2] += pl[w][d0 + h2] * fw[w];
                        const float inv = lsum != 0.f ? 1.0f / lsum : 0.f;
                        val = (uint32_t)f2h(c2[0] * inv) | ((uint32_t)f2h(c2[1] * inv) << 16);
                    }
                } else if (tid == AW_S) {
                    val = __float_as_uint(*sdot);
                } else {
                    const int i = 2 * (tid - AW_V);
                    val = (uint32_t)__builtin_bit_cast(uint16_t, qkvh[PD_D + KS + i]) |
                          ((uint32_t)__builtin_bit_cast(uint16_t, qkvh[PD_D + KS + i + 1]) << 16);
                }
                ll_st(LA + at_word(wg * PD_PW + tid), val, seq(4 * l));
            }
            if (l == 1) mark(118);
            lds_barrier();   // the attention scratch is free again
            mark(4 * l);
            if (l + 1 < GPT2_N_LAYER) {
                stage_qkv_acc<Q8>(wq, a.layers[l + 1].w[0], h, sp, wave, lane);
            }
        }
    } else if (wg - PD_NA < PD_NW) {
        // ================================ GEMV work-group g: proj, fc and mlp-proj rows
        // A work-group polls a buffer only in a phase it writes from, so every writer of the next
        // version of a buffer has first read everything its readers needed.
        const int g = wg - PD_NA;
        f16 *hs = reinterpret_cast<f16 *>(lds + LY::HS);
        float *part = reinterpret_cast<float *>(lds + LY::PART);
        // Residual rows [g*RP, +RP) of x after the previous layer: this work-group wrote them itself
        // (its mlp-proj rows), layer 0 starts from the embedding.
        float xown[RP];
        uint16_t emb_t[RP], emb_p[RP];   // fp16 bits, added once the first phase's input has arrived
#pragma unroll
        for (int k = 0; k < RP; ++k) {
            emb_t[k] = a.wte[(size_t)token * PD_E + g * RP + k];
            emb_p[k] = a.wpe[(size_t)pos * PD_E + g * RP + k];
        }
        // A layer's proj, fc and mlp-proj rows (and LN2 params) are all in flight before the
        // layer's first input arrives: issued right after the previous layer's last poll (the
        // mlp-proj rows after its mlp-proj, whose registers they reuse).  Loads complete in issue
        // order, so a weight load issued shortly before a poll would hold that poll back.
        PhaseW<768, Q8, RP> WP;
        FcW<Q8> FC;
        PhaseW<3072, Q8, RM> WM;
        LNParams lnp;
        load_phase(WP, a.layers[0].w[1], a.layers[0].s[1], a.layers[0].b[1], g * RP, wave, lane);
        load_fc(FC, a.layers[0].w[2], a.layers[0].s[2], a.layers[0].b[2], g * RF, wave, lane);
        load_ln(lnp, a.layers[0].ln2_g, a.layers[0].ln2_b);
        load_phase(WM, a.layers[0].w[3], a.layers[0].s[3], a.layers[0].b[3], g * RM, wave, lane);
        unsigned long long t_st = __builtin_amdgcn_s_memrealtime();   // this work-group's last store
        for (int l = 0; l < GPT2_N_LAYER; ++l) {
            // ---- P: combine the attention words, proj rows, + bias + residual
            constexpr int NA = PD_NA * PD_PW;
            hold_until(t_st + a.hold[0]);
            if (!ll_read<(NA + PD_T - 1) / PD_T>(LA, NA, seq(4 * l), a.err, spin, wflag, at_word,
                                                 [&](int i, uint32_t d) { part[i] = __uint_as_float(d); }))
                return;
            mark(64 + 4 * l + 1);
            if (l == 0) {
#pragma unroll
                for (int k = 0; k < RP; ++k) xown[k] = (float)(f16)(h2f(emb_t[k]) + h2f(emb_p[k]));
            }
            // Element e = tid + 256i: wave w handles head w + 4i, so the per-head weights are
            // wave-uniform; every lane computes them (broadcast LDS reads, no branches).  Key `pos` is
            // one more partial: m = q.k_pos / 8 from the four slices' parts, l = 1, c = v_pos.
            static_assert(PD_S == 4 && PD_T / PD_D == 4, "four slices per head, one head per wave and element");
            auto half_of = [](float w, int hi) {
                const uint32_t u = __float_as_uint(w);
                return h2f((uint16_t)(hi ? u >> 16 : u & 0xffff));
            };
            // The heads' weights first: lanes 0-14 of wave w form, for heads w, w + 4, w + 8, the five
            // parts' weights (four splits and the new key) normalized by the head's total, into LDS;
            // the wave's own reads of them below come after its writes (in order), so no barrier.
            // Then each element is five products: sum over parts of (c / l of the part) x weight.
            float *hw = reinterpret_cast<float *>(lds + LDS_MISC + 256) + wave * 16;   // [3][5]
            if (lane < 15) {
                const int hl = lane / 5, j = lane - 5 * hl;
                const float *p = part + (wave + 4 * hl) * PD_S * PD_PW;
                float m4[PD_S], l4[PD_S], s4[PD_S], f4[PD_S];
#pragma unroll
                for (int s2 = 0; s2 < PD_S; ++s2) {
                    m4[s2] = p[s2 * PD_PW + AW_M];
                    l4[s2] = p[s2 * PD_PW + AW_L];
                    s4[s2] = p[s2 * PD_PW + AW_S];
                }
                const float spos = ((s4[0] + s4[1]) + (s4[2] + s4[3])) * 0.125f;
                float mx = spos;
#pragma unroll
                for (int s2 = 0; s2 < PD_S; ++s2) mx = (l4[s2] != 0.f) ? fmaxf(mx, m4[s2]) : mx;
#pragma unroll
                for (int s2 = 0; s2 < PD_S; ++s2) f4[s2] = (l4[s2] != 0.f) ? __expf(m4[s2] - mx) * l4[s2] : 0.f;
                const float fpos = __expf(spos - mx);
                float L = fpos, fj = fpos;
#pragma unroll
                for (int s2 = 0; s2 < PD_S; ++s2) {
                    L += f4[s2];
                    fj = (j == s2) ? f4[s2] : fj;
                }
                hw[lane] = fj * __builtin_amdgcn_rcpf(L);
            }
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const int e = tid + PD_T * i, hh = e / PD_D, d = e % PD_D;
                const float *p = part + hh * PD_S * PD_PW;
                float c = half_of(p[(d / KS) * PD_PW + AW_V + (d % KS) / 2], d & 1) * hw[5 * i + PD_S];
#pragma unroll
                for (int s2 = 0; s2 < PD_S; ++s2) c += half_of(p[s2 * PD_PW + AW_C + d / 2], d & 1) * hw[5 * i + s2];
                xn[e] = (f16)c;
            }
            if (l == 1) mark(118);
            lds_barrier();
            if (l == 1) mark(119);
            // the RP rows' words go out as one store (one instruction, one line)
            run_phase(WP, xn, wave, lane, [&](int k, float v) {
                if (lane == 0) xout[k] = __builtin_bit_cast(uint16_t, (f16)(v + xown[k]));
            });
            lds_barrier();
            if (tid < RP / 2) ll_st(LX + x_word(g * RP / 2 + tid), xout[2 * tid] | (xout[2 * tid + 1] << 16), seq(4 * l + 1));
            t_st = __builtin_amdgcn_s_memrealtime();
            mark(4 * l + 1);
            // ---- F: LN2 + fc rows [g*RF, +RF) + gelu, exchanged in pairs
            hold_until(t_st + a.hold[1]);
            if (!read_x(seq(4 * l + 1))) return;
            mark(64 + 4 * l + 2);
            layernorm768(xn, xs, lnp, lane);
            if (l == 1) mark(120);
            {
                // QS MFMAs per wave over its K range; column 0 of D (lanes 0, 16, 32, 48) holds rows
                // 4(l / 16) .. +3; the four waves' partials are summed in wave order by threads 0-15.
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s2 = 0; s2 < QS; ++s2) {
                    const f16x8 xv = *reinterpret_cast<const f16x8 *>(xn + qk_k(wave, s2, lane));
                    f16x8 wv;
                    if constexpr (Q8) {
                        const i32x4 c = FC.w[s2 >> 1];
                        wv = i8x8_to_f16x8((s2 & 1) ? uint2{(uint32_t)c[2], (uint32_t)c[3]} : uint2{(uint32_t)c[0], (uint32_t)c[1]});
                    } else {
                        wv = __builtin_bit_cast(f16x8, FC.w[s2]);
                    }
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv, xv, acc, 0, 0, 0);
                }
                float *red = part;   // the attention words are combined by now
                if ((lane & 15) == 0) *reinterpret_cast<f32x4 *>(red + wave * RF + 4 * (lane >> 4)) = acc;
                lds_barrier();
                if (tid < RF) {
                    const float v = ((red[tid] + red[RF + tid]) + red[2 * RF + tid]) + red[3 * RF + tid];
                    hout[tid] = __builtin_bit_cast(uint16_t, (f16)gelu_tanh(v * FC.s + h2f(FC.b)));
                }
            }
            if (l == 1) mark(121);
            lds_barrier();
            if (tid < RF / 2)
                ll_st(LHd + hd_word(g * RF / 2 + tid), (uint32_t)hout[2 * tid] | ((uint32_t)hout[2 * tid + 1] << 16), seq(4 * l + 2));
            t_st = __builtin_amdgcn_s_memrealtime();
            mark(4 * l + 2);
            // ---- M: mlp-proj rows [g*RM, +RM) over gelu(fc), + bias + residual
            hold_until(t_st + a.hold[2]);
            if (!ll_read<PD_F / 2 / PD_T>(LHd, PD_F / 2, seq(4 * l + 2), a.err, spin, wflag, hd_word,
                                          [&](int i, uint32_t d) {
                                              hs[2 * i] = __builtin_bit_cast(f16, (uint16_t)(d & 0xffff));
                                              hs[2 * i + 1] = __builtin_bit_cast(f16, (uint16_t)(d >> 16));
                                          }))
                return;
            mark(64 + 4 * l + 3);
            const bool next = l + 1 < GPT2_N_LAYER;
            if (next) {
                const PDLayer &ln = a.layers[l + 1];
                load_phase(WP, ln.w[1], ln.s[1], ln.b[1], g * RP, wave, lane);
                load_fc(FC, ln.w[2], ln.s[2], ln.b[2], g * RF, wave, lane);
                load_ln(lnp, ln.ln2_g, ln.ln2_b);
            }
            run_phase(WM, hs, wave, lane, [&](int k, float v) {
                const f16 o = (f16)(v + (float)xs[g * RM + k]);
                xown[k] = (float)o;
                if (lane == 0) xout[k] = __builtin_bit_cast(uint16_t, o);
            });
            lds_barrier();
            if (tid < RM / 2) ll_st(LX + x_word(g * RM / 2 + tid), xout[2 * tid] | (xout[2 * tid + 1] << 16), seq(4 * l + 3));
            t_st = __builtin_amdgcn_s_memrealtime();
            if (next) load_phase(WM, a.layers[l + 1].w[3], a.layers[l + 1].s[3], a.layers[l + 1].b[3], g * RM, wave, lane);
            mark(4 * l + 3);
        }
    }
    // ---- head: LN_f, logits rows [wg*RH, ...), local argmax, then work-group 0 picks the token
    const int ph = PH_CAND;
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
        constexpr bool HQ = decltype(q8tag)::value;
        constexpr int CPL = HQ ? 3 : 6, HD = 4;
        const int j = lane & 15, slot = lane >> 4;
        f16x8 xr[HQ ? 2 * CPL : CPL];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            if constexpr (HQ) {
                xr[2 * i] = *reinterpret_cast<const f16x8 *>(xn + (j + 16 * i) * 16);
                xr[2 * i + 1] = *reinterpret_cast<const f16x8 *>(xn + (j + 16 * i) * 16 + 8);
            } else {
                xr[i] = *reinterpret_cast<const f16x8 *>(xn + (j + 16 * i) * 8);
            }
        }
        constexpr int ROWB = HQ ? PD_E : 2 * PD_E;
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
                if constexpr (HQ) {
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
                if constexpr (HQ) v *= a.head_s[r];
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
        ll_st(LC + cand_word(wg), cand, seq(ph));
    }
    if (wg != 0) return;
    // work-group 0: argmax over the candidates, advance the state
    uint32_t *cands = reinterpret_cast<uint32_t *>(lds + LY::CANDS);
    if (!ll_read<(PD_G + PD_T - 1) / PD_T>(LC, PD_G, seq(ph), a.err, spin, wflag, cand_word,
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
static int g_pd_hold[3] = {-1, -1, -1};   // hold-off overrides for new plans (< 0: the constant)

typedef void (*PDKernel)(PDArgs);
static const PDKernel kPersist[2] = {k_decode_persist<false>, k_decode_persist<true>};

// The step's work-groups wait on each other's words, so all PD_G of them must be resident at once:
// the device must hold PD_G of them (one per CU with this LDS footprint) side by side.
static bool persist_fits(PDKernel k) {
    int dev = 0, ncu = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, PD_T, 0);
    return e == hipSuccess && (long)per * ncu >= PD_G;
}

// Builds the step's argument block; returns false when the backend or weights need the
// multi-kernel step (the caller falls back to it), or when the device cannot hold every
// work-group of the step at once.
bool persist_plan(PDPlan &p, const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv, uint16_t *logits,
                  int *state, int *tokens, uint64_t *ll, int *err) {
    if (be->gemv != gpt2_gemv_fp16) return false;
    const bool q_ok = be->gemv_q == gpt2_gemv_int8;
    const GPT2QWeightsGPU *qw = w->q;
    PDArgs &a = p.args;
    PDLayer *h = a.layers;
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
            if (!bh[i]) return false;   // the step loads every bias unconditionally
        }
    }
    // one kernel instance per weight kind: every layer matrix int8, or every one fp16
    int nq = 0;
    for (int L = 0; L < GPT2_N_LAYER; ++L)
        for (int i = 0; i < 4; ++i) nq += h[L].s[i] != nullptr;
    if (nq != 0 && nq != 4 * GPT2_N_LAYER) return false;
    if (kv->maxT > GPT2_N_CTX) return false;   // an attention wave holds at most 64 keys
    p.q8 = nq != 0;
    if (!persist_fits(kPersist[p.q8])) return false;
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
    a.trace = g_pd_trace;
    const unsigned hold0[3] = {PD_HOLD_ATT, PD_HOLD_X, PD_HOLD_HID};
    // a hold only delays a poll; capped at 100 us so that no setting can stall a step for long
    for (int i = 0; i < 3; ++i) a.hold[i] = g_pd_hold[i] >= 0 ? (unsigned)min(g_pd_hold[i], 10000) : hold0[i];
    return true;
}

void persist_launch(const PDPlan &p, hipStream_t s) {
    hipLaunchKernelGGL(kPersist[p.q8], dim3(PD_G), dim3(PD_T), 0, s, p.args);
}

size_t persist_ll_bytes() { return (size_t)LL_WORDS * 8; }

int persist_spin() { return g_pd_spin; }

}  // namespace g2

// Tuning / test hook: poll rounds before a persistent step gives up, for the steps of graphs created
// or set (gpt2_decode_graph_set) afterwards (< 0 restores the default; 0 gives up at the first poll
// that finds a word missing).  A tiny value
// forces the timeout path with every kernel still exiting normally.
extern "C" void gpt2_tune_decode_spin(int rounds) { g2::g_pd_spin = rounds >= 0 ? rounds : g2::PD_SPIN; }
// Tuning hook: the persistent step's poll hold-offs, in 10 ns ticks, for graphs created afterwards:
// before the attention words, x after proj, gelu(fc); a value < 0 keeps that hold-off's default, and
// values above 10000 (100 us) are taken as 10000.  The
// defaults were measured on MI355X (interleaved A/B); a hold only delays a poll, so any value is
// correct, and a box whose exchanges are faster or slower can re-tune them without a rebuild.
extern "C" void gpt2_tune_decode_holds(int att, int x, int hid) {
    g2::g_pd_hold[0] = att;
    g2::g_pd_hold[1] = x;
    g2::g_pd_hold[2] = hid;
}
// Profiling hook: graphs created afterwards record, per work-group, the end time of every phase of
// the persistent step (s_memrealtime, 100 MHz) into trace[wg * 128 + phase]: 4*l + {0 LN1 + q/k/v +
// attention, 1 proj, 2 fc, 3 mlp-proj}, 60 head start, 61 head end, 62 step end, 63 step start, and
// at 64 + p the time phase p's input had arrived; work-group 0 also stores the shader clock counter at step
// start and end in entries 126 / 127.  In layer 1 the attention work-groups also record 113 weights
// landed, 114 LN1 done, 115 q/k/v done, 116 attention done (wave 0), 117 waves merged, 118 words
// stored, 122 start of the poll for x, 123 the number of poll rounds it took beyond the first; the
// GEMV work-groups 118 attention combined, 119 past the barrier, 120 LN2 done, 121 fc rows done.  The buffer holds 256 * 128 entries; nullptr disables.
extern "C" void gpt2_tune_decode_trace(unsigned long long *trace) { g2::g_pd_trace = trace; }
