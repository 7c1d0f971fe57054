// gemv.hip -- M=1 decode GEMVs for gfx950: y[n] = x . W[n,:] (+bias), fp16 or weight-only INT8.
//
// Replaces k_gemv_fp16 / k_gemv_int8 (cuda/kvcache.cu:150-218).  The reference gives each 32-lane
// warp one row and stages x in shared memory.  Here, for the bandwidth-bound M=1 case:
//   * a wave64 is split into 64/LPR row slots of LPR lanes; lane j of a slot reads the row's
//     16-byte chunks j, j+LPR, j+2*LPR, ... so every load instruction of the slot covers 16*LPR
//     contiguous bytes, and all CPL loads of a lane (times U rows) are issued before any is used;
//   * the x chunks a lane needs are the same for every row, so they are loaded once into registers;
//   * fp16 products go through v_dot2_f32_f16 (two fp16 products summed into an fp32 accumulator);
//     int8 codes are turned into exact fp16 values in registers (bias trick, see i8x4_to_f16x4) and
//     take the same dot instruction, so halved weight bytes cost no extra memory instructions;
//   * the slot's partial sums are reduced with DPP row operations (and two lane swaps across 16-lane
//     rows when LPR > 16); the per-row scale is applied after the sum, then the bias
//     (cuda/kvcache.cu:194-197).
// Rows past N are neither loaded nor stored (the vocabulary head's N = 50257 tail).
#include <cstdlib>

#include "common.h"

namespace g2 {


__device__ __forceinline__ float dot8(const i32x4 w, const f16x8 x, float acc) {
    const f16x8 wh = __builtin_bit_cast(f16x8, w);
    acc = __builtin_amdgcn_fdot2(f16x2{wh[0], wh[1]}, f16x2{x[0], x[1]}, acc, false);
    acc = __builtin_amdgcn_fdot2(f16x2{wh[2], wh[3]}, f16x2{x[2], x[3]}, acc, false);
    acc = __builtin_amdgcn_fdot2(f16x2{wh[4], wh[5]}, f16x2{x[4], x[5]}, acc, false);
    acc = __builtin_amdgcn_fdot2(f16x2{wh[6], wh[7]}, f16x2{x[6], x[7]}, acc, false);
    return acc;
}

// 16 int8 codes against 16 fp16 x values (two f16x8).
__device__ __forceinline__ float dot16q(const i32x4 w, const f16x8 x0, const f16x8 x1, float acc) {
    f16x2 a, b;
    i8x4_to_f16x4_v((uint32_t)w.x, a, b);
    acc = __builtin_amdgcn_fdot2(a, f16x2{x0[0], x0[1]}, acc, false);
    acc = __builtin_amdgcn_fdot2(b, f16x2{x0[2], x0[3]}, acc, false);
    i8x4_to_f16x4_v((uint32_t)w.y, a, b);
    acc = __builtin_amdgcn_fdot2(a, f16x2{x0[4], x0[5]}, acc, false);
    acc = __builtin_amdgcn_fdot2(b, f16x2{x0[6], x0[7]}, acc, false);
    i8x4_to_f16x4_v((uint32_t)w.z, a, b);
    acc = __builtin_amdgcn_fdot2(a, f16x2{x1[0], x1[1]}, acc, false);
    acc = __builtin_amdgcn_fdot2(b, f16x2{x1[2], x1[3]}, acc, false);
    i8x4_to_f16x4_v((uint32_t)w.w, a, b);
    acc = __builtin_amdgcn_fdot2(a, f16x2{x1[4], x1[5]}, acc, false);
    acc = __builtin_amdgcn_fdot2(b, f16x2{x1[6], x1[7]}, acc, false);
    return acc;
}

// The sum over the LPR lanes of a row slot: DPP within 16 lanes, then (LPR = 32, 64) the 16-lane row
// sums read as scalars and combined in the order the xor-16 / xor-32 permutes would (same bits).
template <int LPR>
__device__ __forceinline__ float slot_sum(float v) {
    v = row16_sum(v);
    if constexpr (LPR >= 64) return cross_rows_sum(v);
    if constexpr (LPR == 32) {
        const float lo = lane_f(v, 0) + lane_f(v, 16), hi = lane_f(v, 32) + lane_f(v, 48);
        return (threadIdx.x & 32) ? hi : lo;
    }
    return v;
}

// Epilogues a decode step fuses into its GEMVs.


// LPR lanes per row, CPL 16-byte chunks per lane (row = LPR*CPL chunks), U rows per slot in flight.
// LN: x is the residual stream and the kernel applies LayerNorm(x; ln_g, ln_b) to it first.  The
//     LPR lanes of a row slot hold all K values of x between them, so the statistics need no extra
//     loads: each lane sums its values and the slot reduces (mean, then the biased variance of
//     x - mean, eps inside the sqrt -- the same formula as k_layernorm); the normalized value is
//     rounded to fp16, as the standalone LayerNorm's output would be.
// EPI: EPI_GELU applies gelu_new to (acc*s + bias); EPI_RESID writes resid[n] + (acc*s + bias)
//     (resid may alias C: each output is read and written by the same lane).
template <int LPR, int CPL, int U, bool QW, bool LN = false, int EPI = EPI_NONE>
__global__ __launch_bounds__(256) void k_gemv(uint16_t *C, const uint16_t *__restrict__ x,
                                              const void *__restrict__ Wv, const float *Ws,
                                              const uint16_t *bias, int N,
                                              const uint16_t *ln_g, const uint16_t *ln_b,
                                              const uint16_t *resid) {
    constexpr int RPW = 64 / LPR;                  // row slots per wave
    constexpr int ROWB = LPR * CPL * 16;           // bytes per weight row
    constexpr int XV = QW ? 2 * CPL : CPL;         // f16x8 x vectors per lane
    const int lane = threadIdx.x & 63, j = lane % LPR, slot = lane / LPR;
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int rbase = wave * (RPW * U) + slot;

    // element offset of x vector v of this lane
    auto xoff = [&](int v) {
        if constexpr (QW) return (j + LPR * (v >> 1)) * 16 + (v & 1) * 8;
        else return (j + LPR * v) * 8;
    };
    f16x8 xr[XV];
#pragma unroll
    for (int v = 0; v < XV; ++v) xr[v] = *reinterpret_cast<const f16x8 *>(x + xoff(v));

    const char *W = reinterpret_cast<const char *>(Wv);
    i32x4 wv[U][CPL];
    // Rows past N read row N-1 (their sums are never stored): unconditional loads keep all of them
    // in flight at once, where a branch per load would make the wave wait between them.
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int r = min(rbase + u * RPW, N - 1);
#pragma unroll
        for (int i = 0; i < CPL; ++i)
            wv[u][i] = *reinterpret_cast<const i32x4 *>(W + (size_t)r * ROWB + (j + LPR * i) * 16);
    }
    // The rows' scale, bias and residual (and the LayerNorm parameters) are loaded with the weights,
    // unconditionally at clamped rows (without a bias, x[0] stands in and is not used), each value
    // in its own register until the epilogue: loaded after the reduction, they would cost a second
    // memory round trip per launch.
    float sc_e[U];
    uint32_t bs_e[U], rs_e[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int r = min(rbase + u * RPW, N - 1);
        sc_e[u] = 1.f;
        if constexpr (QW) sc_e[u] = Ws[r];
        bs_e[u] = *(bias ? bias + r : x);
        rs_e[u] = 0u;
        if constexpr (EPI == EPI_RESID) rs_e[u] = resid[r];
    }
    f16x8 lg[LN ? XV : 1], lb[LN ? XV : 1];
    if constexpr (LN) {
#pragma unroll
        for (int v = 0; v < XV; ++v) {
            lg[v] = *reinterpret_cast<const f16x8 *>(ln_g + xoff(v));
            lb[v] = *reinterpret_cast<const f16x8 *>(ln_b + xoff(v));
        }
    }
    // keeps the compiler from sinking those loads down to their use (no wait is implied; the
    // pointers are not __restrict__, so the loads cannot move across this point)
    asm volatile("" ::: "memory");

    if constexpr (LN) {
        constexpr float invK = 1.0f / (float)(XV * 8 * LPR);
        float sum = 0.f;
#pragma unroll
        for (int v = 0; v < XV; ++v)
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += (float)xr[v][e];
        const float mean = slot_sum<LPR>(sum) * invK;
        float sq = 0.f;
#pragma unroll
        for (int v = 0; v < XV; ++v)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = (float)xr[v][e] - mean;
                sq += d * d;
            }
        const float rstd = 1.0f / sqrtf(slot_sum<LPR>(sq) * invK + GPT2_LN_EPS);
#pragma unroll
        for (int v = 0; v < XV; ++v)
#pragma unroll
            for (int e = 0; e < 8; ++e) xr[v][e] = (f16)(((float)xr[v][e] - mean) * rstd * (float)lg[v][e] + (float)lb[v][e]);
    }

#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int r = rbase + u * RPW;
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            if constexpr (QW) acc = dot16q(wv[u][i], xr[2 * i], xr[2 * i + 1], acc);
            else acc = dot8(wv[u][i], xr[i], acc);
        }
        acc = slot_sum<LPR>(acc);
        // the epilogue runs on every lane (the values were loaded for every lane), one lane stores
        float v = acc;
        if constexpr (QW) v *= sc_e[u];
        if (bias) v += h2f((uint16_t)bs_e[u]);
        if constexpr (EPI == EPI_GELU) v = gelu_tanh(v);
        if constexpr (EPI == EPI_RESID) v += h2f((uint16_t)rs_e[u]);
        if (j == 0 && r < N) C[r] = f2h(v);
    }
}

// Any K / alignment: one wave per row, scalar loads.
template <bool QW>
__global__ __launch_bounds__(256) void k_gemv_generic(uint16_t *__restrict__ C, const uint16_t *__restrict__ x,
                                                      const void *__restrict__ Wv, const float *__restrict__ Ws,
                                                      const uint16_t *__restrict__ bias, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int r = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (r >= N) return;
    float acc = 0.f;
    for (int k = lane; k < K; k += 64) {
        float w;
        if constexpr (QW) w = (float)reinterpret_cast<const int8_t *>(Wv)[(size_t)r * K + k];
        else w = h2f(reinterpret_cast<const uint16_t *>(Wv)[(size_t)r * K + k]);
        acc += h2f(x[k]) * w;
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        float v = acc;
        if constexpr (QW) v *= Ws[r];
        if (bias) v += h2f(bias[r]);
        C[r] = f2h(v);
    }
}

typedef void (*GemvFn)(uint16_t *, const uint16_t *, const void *, const float *, const uint16_t *, int,
                       const uint16_t *, const uint16_t *, const uint16_t *);

struct GemvCfg {
    int row_chunks;   // 16-byte chunks per row this kernel is built for
    bool qw;
    int rows_per_wave;
    int waves_per_block;
    GemvFn fn;
    const char *name;
};

#define G2_GV(LPR, CPL, U, QW, WPB) \
    {LPR * CPL, QW, (64 / LPR) * U, WPB, k_gemv<LPR, CPL, U, QW>, "lpr" #LPR "_cpl" #CPL "_u" #U "_" #QW "_wpb" #WPB}

// First match on (row_chunks, qw) is the default; the rest are alternatives for tuning.  INT8 K=3072
// (mlp-proj) takes a whole wave per row: four times the work-groups of 16 lanes per row, so the
// cold launch (weights streamed from HBM) has loads in flight on 192 CUs instead of 48 -- 3.49 against
// 4.42 us per launch, interleaved in one process, the same when the weights are warm.
static const GemvCfg kGv[] = {
    G2_GV(16, 3, 2, true, 1),    // int8 K=768
    G2_GV(16, 3, 1, true, 4),
    G2_GV(64, 3, 1, true, 4),    // int8 K=3072
    G2_GV(16, 6, 1, false, 4),   // fp16 K=768
    G2_GV(64, 6, 1, false, 4),   // fp16 K=3072
    G2_GV(16, 3, 2, true, 4),
    G2_GV(16, 3, 1, true, 1),
    G2_GV(16, 12, 1, true, 4),
    G2_GV(64, 3, 2, true, 4),
    G2_GV(32, 6, 1, true, 4),
    G2_GV(16, 6, 2, false, 4),
    G2_GV(16, 6, 4, false, 4),
    G2_GV(32, 3, 1, false, 4),
    G2_GV(32, 3, 2, false, 4),
    G2_GV(16, 6, 1, false, 1),
    G2_GV(16, 24, 1, false, 4),
};
static const int kNumGv = (int)(sizeof(kGv) / sizeof(kGv[0]));

static int g_force_gv = -2;

static int pick_gemv(int row_chunks, bool qw) {
    if (g_force_gv == -2) {
        const char *e = getenv("GPT2_GEMV_CFG");
        g_force_gv = e ? atoi(e) : -1;
    }
    if (g_force_gv >= 0 && g_force_gv < kNumGv && kGv[g_force_gv].row_chunks == row_chunks && kGv[g_force_gv].qw == qw)
        return g_force_gv;
    for (int i = 0; i < kNumGv; ++i)
        if (kGv[i].row_chunks == row_chunks && kGv[i].qw == qw) return i;
    return -1;
}

void gemv(uint16_t *C, const uint16_t *x, const void *W, const float *Ws, const uint16_t *bias, int N, int K, bool qw,
          int cfg) {
    if (N == 0) return;
    const long row_bytes = qw ? (long)K : 2L * K;
    int c = -1;
    if (K > 0 && row_bytes % 16 == 0 && aligned16(W) && aligned16(x)) {
        const int rc = (int)(row_bytes / 16);
        c = (cfg >= 0 && cfg < kNumGv && kGv[cfg].row_chunks == rc && kGv[cfg].qw == qw) ? cfg : pick_gemv(rc, qw);
    }
    if (c >= 0) {
        const GemvCfg &g = kGv[c];
        const int waves = cdiv(N, g.rows_per_wave);
        const int blocks = cdiv(waves, g.waves_per_block);
        hipLaunchKernelGGL(g.fn, dim3(blocks), dim3(64 * g.waves_per_block), 0, stream(), C, x, W, Ws, bias, N,
                           nullptr, nullptr, nullptr);
        check_launch(qw ? "k_gemv<int8>" : "k_gemv<fp16>");
        return;
    }
    const int blocks = cdiv(N, 4);
    if (qw) hipLaunchKernelGGL(k_gemv_generic<true>, dim3(blocks), dim3(256), 0, stream(), C, x, W, Ws, bias, N, K);
    else hipLaunchKernelGGL(k_gemv_generic<false>, dim3(blocks), dim3(256), 0, stream(), C, x, W, Ws, bias, N, K);
    check_launch("k_gemv_generic");
}

// Fused decode GEMVs: (LayerNorm ->) GEMV (-> gelu | + residual).  Returns false when no fused
// kernel covers the shape (the caller then runs the unfused sequence).
struct FusedGemv {
    int row_chunks;
    bool qw, ln;
    int epi;
    int rows_per_wave;
    GemvFn fn;
};

#define G2_FG(LPR, CPL, QW, LN, EPI) {LPR * CPL, QW, LN, EPI, 64 / LPR, k_gemv<LPR, CPL, 1, QW, LN, EPI>}
static const FusedGemv kFused[] = {
    G2_FG(16, 3, true, true, EPI_NONE),  G2_FG(16, 3, true, true, EPI_GELU),   G2_FG(16, 3, true, false, EPI_RESID),
    G2_FG(64, 3, true, false, EPI_RESID),
    G2_FG(16, 6, false, true, EPI_NONE), G2_FG(16, 6, false, true, EPI_GELU),  G2_FG(16, 6, false, false, EPI_RESID),
    G2_FG(64, 6, false, false, EPI_RESID),
};

bool gemv_fused(uint16_t *C, const uint16_t *x, const void *W, const float *Ws, const uint16_t *bias, int N, int K,
                bool qw, const uint16_t *ln_g, const uint16_t *ln_b, int epi, const uint16_t *resid) {
    const bool ln = ln_g != nullptr;
    const long row_bytes = qw ? (long)K : 2L * K;
    if (N <= 0 || K <= 0 || row_bytes % 16 || !aligned16(W) || !aligned16(x)) return false;
    if (ln && (!aligned16(ln_g) || !aligned16(ln_b))) return false;
    const int rc = (int)(row_bytes / 16);
    for (const FusedGemv &f : kFused) {
        if (f.row_chunks != rc || f.qw != qw || f.ln != ln || f.epi != epi) continue;
        const int blocks = cdiv(cdiv(N, f.rows_per_wave), 4);
        hipLaunchKernelGGL(f.fn, dim3(blocks), dim3(256), 0, stream(), C, x, W, Ws, bias, N, ln_g, ln_b, resid);
        check_launch("k_gemv<fused>");
        return true;
    }
    return false;
}

}  // namespace g2

using namespace g2;

extern "C" void gpt2_gemv_fp16(gpt2_half *C, const gpt2_half *A, const gpt2_half *W, const gpt2_half *bias, int N,
                               int K) {
    if (N < 0 || K < 0 || (N > 0 && (!C || !A || !W))) { arg_fail("gpt2_gemv_fp16: bad shape or null pointer"); return; }
    gemv(C, A, W, nullptr, bias, N, K, false, -1);
}

extern "C" void gpt2_gemv_int8(gpt2_half *C, const gpt2_half *A, const int8_t *Wq, const float *Ws,
                               const gpt2_half *bias, int N, int K) {
    if (N < 0 || K < 0 || (N > 0 && (!C || !A || !Wq || !Ws))) {
        arg_fail("gpt2_gemv_int8: bad shape or null pointer");
        return;
    }
    gemv(C, A, Wq, Ws, bias, N, K, true, -1);
}

extern "C" int gpt2_tune_gemv_count(void) { return kNumGv; }
extern "C" const char *gpt2_tune_gemv_name(int cfg) { return cfg >= 0 && cfg < kNumGv ? kGv[cfg].name : "?"; }
extern "C" int gpt2_tune_gemv_fits(int cfg, int K, int qw) {
    if (cfg < 0 || cfg >= kNumGv) return 0;
    const long rb = qw ? K : 2L * K;
    return rb % 16 == 0 && kGv[cfg].row_chunks == rb / 16 && kGv[cfg].qw == (qw != 0);
}
extern "C" void gpt2_tune_gemv_run(int cfg, gpt2_half *C, const gpt2_half *A, const void *W, const float *Ws,
                                   const gpt2_half *bias, int N, int K) {
    gemv(C, A, W, Ws, bias, N, K, Ws != nullptr, cfg);
}
