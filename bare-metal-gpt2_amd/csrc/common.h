// common.h -- internal helpers shared by the HIP sources of libgpt2amd.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gpt2_kernels.h"
#include "gpt2_kvcache.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

namespace g2 {

// Launch stream for every launcher (set by gpt2_set_stream).
hipStream_t stream();

// Record the first error since the last gpt2_last_error(); later ones are dropped.
void set_error(int code, const char *what);
// Codes >= 1000 are host-side argument errors; below that they are hipError_t values.
enum { E_ARG = 1000, E_ALIGN = 1001, E_FORMAT = 1002, E_CAPACITY = 1003, E_STATE = 1004 };

// Check the launch that was just enqueued.
void check_launch(const char *what);

// Resolves (once per device) the device address of gpt2_forward_noalloc's static scratch on the
// current device; gpt2_set_stream calls it so that a caller who captures the no-allocation forward
// into a graph has it resolved before the capture begins.
void noalloc_prepare();
// Synchronizing calls (gpt2_sync) ask this after the stream drains: nonzero when a persistent
// prefill launched since the last check gave up waiting (its sticky error word, cleared here).
int prefill_persist_take_error();

// A decode step reads (token, pos) from immediates or, under graph replay, from a small
// device-resident state {token, pos}.
struct StepArg {
    int token, pos;
    const int *state;  // nullptr: use the immediates
    __device__ __forceinline__ int tok() const { return state ? state[0] : token; }
    __device__ __forceinline__ int p() const { return state ? state[1] : pos; }
};

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

inline bool arg_fail(const char *what) {
    set_error(E_ARG, what);
    return true;
}

// Wave64 helpers -------------------------------------------------------------------------------
// Sum over the 16 lanes of each DPP row (lanes 16r..16r+15); every lane receives the row sum.
__device__ __forceinline__ float row16_sum(float v) {
    // quad_perm [1,0,3,2] (xor 1), quad_perm [2,3,0,1] (xor 2), row_half_mirror, row_mirror
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, true));
    return v;
}

__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The four row sums of row16_sum combined as (r0 + r1) + (r2 + r3), read as scalars (v_readlane)
// instead of crossing rows through two LDS permutes (xor 16, then xor 32).  Every lane of a row holds
// the same bits after row16_sum, so this is bit for bit what the permutes give every lane.
__device__ __forceinline__ float cross_rows_sum(float v) {
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_sum(float v) { return cross_rows_sum(row16_sum(v)); }

// Wave-uniform sum / max: DPP within each 16-lane row, then the four row results are read as
// scalars (v_readlane) instead of crossing rows through LDS permutes.  Every lane gets the same
// value; the row results are combined in the fixed order 0, 16, 32, 48.
__device__ __forceinline__ float wave_sum_u(float v) {
    v = row16_sum(v);
    return ((lane_f(v, 0) + lane_f(v, 16)) + lane_f(v, 32)) + lane_f(v, 48);
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, true)));
    return v;
}
__device__ __forceinline__ float wave_max_u(float v) {
    v = row16_max(v);
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(f16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (f16)f);   // v_cvt_f16_f32: round to nearest even
}

// LayerNorm of one 768-wide row held by one wave, lane l holding elements 256 i + 4 l + c (i < 3,
// c < 4): the mean, then the mean squared deviation from it, eps inside the square root
// (cuda/kernels_naive.cu:26-41), in fp32.  Every kernel that normalizes rows (the LayerNorm kernel,
// the GEMMs that normalize their own A panel) goes through this function, so they agree bit for
// bit: the fp32 operations are written out (explicit fma) and each output is pinned in fp32 before
// its conversion, so no kernel can fold the conversion into the fma (v_fma_mix: one rounding
// instead of two) where another does not.
__device__ __forceinline__ void ln_row768(const f16x4 (&x)[3], const f16x4 (&g)[3], const f16x4 (&b)[3],
                                          f16x4 (&o)[3]) {
    float v[12];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) v[4 * i + c] = (float)x[i][c];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 12; ++i) s += v[i];
    const float mean = wave_sum(s) / (float)GPT2_N_EMBD;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < 12; ++i) {
        const float d = v[i] - mean;
        q = __builtin_fmaf(d, d, q);
    }
    const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)GPT2_N_EMBD + GPT2_LN_EPS);
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float y = __builtin_fmaf((v[4 * i + c] - mean) * rstd, (float)g[i][c], (float)b[i][c]);
            asm volatile("" : "+v"(y));
            o[i][c] = (f16)y;
        }
}

// ln_row768 on R rows at once (row r in x[r], lane layout as above): each row goes through exactly
// ln_row768's operations, so the bits are those of R calls, but the rows' cross-lane sums are
// issued together, so their latencies (DPP steps and lane reads) overlap instead of
// running one row after another.
template <int R>
__device__ __forceinline__ void ln_rows768(const f16x4 (&x)[R][3], const f16x4 (&g)[3], const f16x4 (&b)[3],
                                           f16x4 (&o)[R][3]) {
    float v[R][12], s[R], q[R], mean[R], rstd[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) v[r][4 * i + c] = (float)x[r][i][c];
        s[r] = 0.f;
#pragma unroll
        for (int i = 0; i < 12; ++i) s[r] += v[r][i];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) s[r] = row16_sum(s[r]);
#pragma unroll
    for (int r = 0; r < R; ++r) s[r] = cross_rows_sum(s[r]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        mean[r] = s[r] / (float)GPT2_N_EMBD;
        q[r] = 0.f;
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            const float d = v[r][i] - mean[r];
            q[r] = __builtin_fmaf(d, d, q[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) q[r] = row16_sum(q[r]);
#pragma unroll
    for (int r = 0; r < R; ++r) q[r] = cross_rows_sum(q[r]);
#pragma unroll
    for (int r = 0; r < R; ++r) rstd[r] = 1.0f / sqrtf(q[r] / (float)GPT2_N_EMBD + GPT2_LN_EPS);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float y = __builtin_fmaf((v[r][4 * i + c] - mean[r]) * rstd[r], (float)g[i][c], (float)b[i][c]);
                asm volatile("" : "+v"(y));
                o[r][i][c] = (f16)y;
            }
}

// gelu_new, the tanh form (model/config.h:41-42): 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))).
// The decode kernels (fused GEMV epilogue, persistent step) use this form.
__device__ __forceinline__ float gelu_tanh(float v) {
    const float z = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    return 0.5f * v * (1.0f + tanhf(z));
}

// gelu_new rounded to fp16 for the prefill, where the elementwise gelu kernel and the fused GEMM
// epilogue must agree bit for bit.  With 1 + tanh(z) = 2 / (1 + e^(-2z)), gelu is v / (1 + e^(-2z)),
// computed as v * rcp(1 + 2^(K * (v + 0.044715 v^3))), K = -2 sqrt(2/pi) log2(e), on the hardware
// exp2 and reciprocal (a few fp32 ulps) with explicit builtins and one explicit fma, so nothing is
// left to contract or reassociate.  The fp32 result is pinned before the conversion: otherwise the
// conversion folds into the last multiply in some kernels (v_fma_mixlo_f16: one rounding) and not in
// others (fp32 product, then convert: two roundings, 1 ulp apart on rare ties).  Large |v|: the
// exponential goes to 0 or +inf and the result to v or -0.
__device__ __forceinline__ uint16_t gelu_f16(float v) {
    constexpr float K = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
    const float inner = __builtin_fmaf(0.044715f, v * v * v, v);
    const float e = __builtin_amdgcn_exp2f(K * inner);
    float y = v * __builtin_amdgcn_rcpf(1.0f + e);
    asm volatile("" : "+v"(y));
    return f2h(y);
}

// Elementwise op fused into a matmul's epilogue: none, gelu_new, or a residual add; and the forms
// of the prefill's LayerNorm fold (LnFold below): the residual add that also emits x * gamma and the
// row statistics, and the matmul over x * gamma that applies the LayerNorm in its epilogue (then
// gelu_new for the fc matmul).
enum { EPI_NONE = 0, EPI_GELU = 1, EPI_RESID = 2, EPI_RESID_LN = 3, EPI_LNF = 4, EPI_LNF_GELU = 5 };

// LayerNorm folded into the matmul that consumes it.  For a row x (768 wide) with mean mu and
// rstd = 1 / sqrt(var + eps),
//   LN(x) . W_n = rstd (sum_k x_k g_k W_nk - mu sum_k g_k W_nk) + sum_k b_k W_nk
// so the consumer multiplies xg = x * gamma (fp16) by W and finishes each output with
//   rstd_m (P_mn - mu_m G_n) + H_n,   G_n = sum_k gamma_k W_nk,  H_n = sum_k beta_k W_nk
// (fp32, per consumer matrix; INT8: W_nk = s_n q_nk).  mu and var come from per-row partial sums
// of the fp16 x (sum, sum of squares), one partial per 16-column slice of the row, each written by
// the one wave that produced those columns: 48 slots per row, summed in a fixed order by the
// consumer, so the result does not depend on which work-group finishes first.  The partials are
// stored slot-major with a slot stride of lnfold_stride(M) rows: an odd number of 128-byte lines
// (from M = 16 up), so the slots of a row block spread over the L2 channels instead of lining up
// on one (a stride of M = 512 rows is 4 KB).
constexpr int LNF_SLOTS = GPT2_N_EMBD / 16;
inline int lnfold_stride(int M) {
    if (M < 16) return M;
    const int r = (M + 15) & ~15;
    return (r / 16) % 2 ? r : r + 16;
}
struct LnFold {
    const uint16_t *gamma;   // RESID_LN: gamma of the LayerNorm the x feeds (fp16, 768)
    uint16_t *xg;            // RESID_LN: x * gamma, fp16, row-major like C
    float2 *stats_out;       // RESID_LN: [LNF_SLOTS][stride] (sum x, sum x^2) of 16 columns each
    const float2 *stats_in;  // LNF: the producer's stats of the A rows
    const float2 *gh;        // LNF: (G_n, H_n) per output column
    int stride;              // rows per slot in the partials: lnfold_stride(M)
};

// A GEMM output after scale and bias, as the unfused sequence would leave it: rounded to fp16, then
// gelu (rounded again) or the residual r added (rounded again) -- the rounding points of a separate
// matmul, gelu and add (cuda/forward_cuda.cu:99-105), so fusing changes no bit.
template <int EPI>
__device__ __forceinline__ uint16_t epi_out(float v, uint16_t r) {
    uint16_t o = f2h(v);
    if constexpr (EPI == EPI_GELU || EPI == EPI_LNF_GELU) o = gelu_f16(h2f(o));
    else if constexpr (EPI == EPI_RESID || EPI == EPI_RESID_LN) o = f2h(h2f(r) + h2f(o));
    return o;
}

// Sign-exact int8 -> fp16 for four packed bytes: (b ^ 0x80) is b + 128 in [1, 255]; the half with
// bits 0x6400 | u is 1024 + u; subtracting 1152 leaves b.
__device__ __forceinline__ void i8x4_to_f16x4_v(uint32_t w, f16x2 &lo, f16x2 &hi) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x07030602u);
    const f16x2 off = {(f16)-1152.0f, (f16)-1152.0f};
    lo = __builtin_bit_cast(f16x2, a) + off;
    hi = __builtin_bit_cast(f16x2, b) + off;
}

// The same widening as two f16x2 words (lo, hi) of 32 bits.
__device__ __forceinline__ void i8x4_to_f16x4(uint32_t w, uint32_t &lo, uint32_t &hi) {
    f16x2 a, b;
    i8x4_to_f16x4_v(w, a, b);
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
}

// Eight int8 codes (two packed words) widened to eight exact fp16 values.
__device__ __forceinline__ f16x8 i8x8_to_f16x8(uint2 w) {
    uint32_t h[4];
    i8x4_to_f16x4(w.x, h[0], h[1]);
    i8x4_to_f16x4(w.y, h[2], h[3]);
    const i32x4 v = {(int)h[0], (int)h[1], (int)h[2], (int)h[3]};
    return __builtin_bit_cast(f16x8, v);
}

// Work-group barrier for LDS traffic: waits for this wave's LDS (and scalar) operations only, not for
// its outstanding global loads and stores, which __syncthreads() also drains.  Loads issued ahead
// (the next tile, the next phase's weights) stay in flight across it; the caller waits for those
// itself before using them.  The "memory" clobber keeps the compiler from moving memory accesses
// across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt immediate for "at most n vector-memory operations outstanding" (gfx9 encoding, expcnt
// and lgkmcnt left unconstrained).
template <int n>
__device__ __forceinline__ void wait_vm() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
}

// Wait until at most `after` k-tiles of this wave's loads (L instructions each) are outstanding
// (after is a run-time value in [0, MAXA]; each case is an immediate s_waitcnt).
template <int L, int MAXA>
__device__ __forceinline__ void wait_tiles(int after) {
    if constexpr (MAXA >= 0) {
        if (after == MAXA) { wait_vm<L * MAXA>(); return; }
        wait_tiles<L, MAXA - 1>(after);
    }
}

}  // namespace g2

// LDS pointer for global_load_lds (device pass only: the address space does not exist on the host).
#define G2_LDS(p) ((__attribute__((address_space(3))) void *)(p))

#define G2_HALF(p) reinterpret_cast<f16 *>(p)
#define G2_CHALF(p) reinterpret_cast<const f16 *>(p)
