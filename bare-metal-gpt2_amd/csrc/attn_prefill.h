// attn_prefill.h -- causal prefill attention on the MFMA units (gfx950): one block of 16 queries
// of one head, as a device function shared by the attention launch (attn_prefill.hip) and the
// persistent prefill (prefill.hip).
//
// Semantics of cpu/forward_cpu.c:83-116 (the reference's fused attention, cuda/kernels_fused.cu:58-140):
// att[i, h*64 + d] = sum_{j<=i} softmax_j(q_i . k_j / 8) v_j[d] over qkv[T, 3*768] (q | k | v, head h
// at columns h*64).
//
// Design, MI355X-first:
//   * A work-group owns 16 queries of one head; its four waves split the keys [0, last query] in
//     32-key chunks (chunk c on wave c % 4), each keeping its own online-softmax state, merged
//     through LDS at the end.
//   * Scores on v_mfma_f32_16x16x32_f16 with the keys as the A operand and the queries as B:
//     S[key][query], so a lane holds four keys of one query (keys 4g..4g+3 of a 16-key tile, lane
//     group g = lane / 16).  K and Q fragments are 16-byte loads straight from qkv (8 consecutive
//     dims of one row per lane), no LDS.
//   * P.V as O^T[d][query] = V^T[d][key] . P[key][query]: the MFMA k-slots 8g..8g+7 of lane group g
//     are mapped to keys {4g..4g+3} of the chunk's first tile and {16+4g..16+4g+3} of its second --
//     exactly the keys the lane already holds P for -- so P is the B operand as it comes out of the
//     softmax, converted to fp16 in registers.  V^T (keys contiguous per dim) is the A operand: each
//     wave stores its chunk's 32 x 64 V block row-major in its own LDS tile (16-byte writes, rows
//     padded to 160 B so that neither the writes nor the reads below meet a bank conflict) and
//     reads each fragment half with gfx950's transposing LDS read, ds_read_b64_tr_b16: within 16
//     lanes, lane 4k+a names 4 dims of key k and lane 4a+b receives dim b of those 4 keys.
//   * Softmax in the log2 domain (p = 2^(s*log2(e)/8 - m) as one FMA and v_exp_f32), the row maximum
//     shared by the lane groups of a query each chunk through the VALU lane swaps (no LDS
//     permutes); the causal mask is applied only to chunks that cross the diagonal.  The
//     denominator sums the fp16-rounded probabilities the MFMA sees, so the output is an exact
//     convex combination of the value rows.
#pragma once

#include <cmath>

#include "common.h"

namespace g2 {

constexpr int AP_QB = 16;                      // queries per work-group
constexpr int AP_CK = 32;                      // keys per chunk
constexpr int AP_W = 4;                        // waves per work-group
constexpr int AP_RV = 160;                     // bytes per V row in LDS (64 dims + 32 B pad)

// 2^x on the hardware exp unit (no denormal-range fix-up: arguments here are <= 0 and a result
// below 2^-126 may flush to zero, which is below anything an fp16 probability can hold).
__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

// Maximum over the four lane groups of a query (lanes l, l^16, l^32, l^48), on the VALU lane
// swaps of gfx950: swapping a value with itself pairs each lane with its partner in either order.
__device__ __forceinline__ float group_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// gfx950's transposing LDS read of 8 bytes (ds_read_b64_tr_b16): within each 16 lanes, lane 4k+a
// supplies the address of 4 consecutive halves, and lane 4a+b receives half b of the addresses of
// lanes a, 4+a, 8+a, 12+a, in that order (layout checked on the GPU).
__device__ __forceinline__ f16x4 tr_read(const char *p) {
#if defined(__HIP_DEVICE_COMPILE__)   // LDS address-space pointers exist only in the device pass
    typedef short i16x4 __attribute__((ext_vector_type(4)));
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4 *)(p));
    return __builtin_bit_cast(f16x4, v);
#else
    (void)p;
    return f16x4{};
#endif
}

// LDS of one attention block (four waves).
struct AttnLds {
    char vt_all[AP_W][AP_CK * AP_RV];
    float mrg_m[AP_W][AP_QB], mrg_l[AP_W][AP_QB];
    f32x4 mrg_o[AP_W][AP_W][64];    // [source wave][dim group][lane]
};

// Queries q0 .. q0+15 of head h over keys [0, last query]; 256 threads.  Kc, Vc (optional): the
// layer's K and V cache planes ([H][maxT][D]), filled with this block's 16 rows.  COHERENT: the
// output rows are stored with device-scope (sc1) stores, for a consumer in the same launch on
// another XCD.  Ends with every wave past the LDS merge (the caller may reuse `lds` after a barrier).
template <bool COHERENT>
__device__ __forceinline__ void attn_block(AttnLds &lds, uint16_t *__restrict__ att, const uint16_t *__restrict__ qkv,
                                           int T, uint16_t *__restrict__ Kc, uint16_t *__restrict__ Vc, int maxT,
                                           int h, int q0) {
    constexpr int E = GPT2_N_EMBD, D = GPT2_HEAD_DIM, S3 = 3 * GPT2_N_EMBD;
    static_assert(D == 64 && AP_QB == 16 && AP_CK == 32, "fragment layout is written for these sizes");
    auto &vt_all = lds.vt_all;
    auto &mrg_m = lds.mrg_m;
    auto &mrg_l = lds.mrg_l;
    auto &mrg_o = lds.mrg_o;

    // wave through readfirstlane: the chunk loop counter and the mask test are then scalar
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int jq = lane & 15, g = lane >> 4;
    // The prefill's K/V cache rows of this block's positions and head, one 16-byte chunk per thread
    // (16 positions x 8 chunks for K, the same for V), into [H][maxT][D] of the layer.  The chunk is
    // loaded here, before the queries and keys (unconditionally, at a clamped row), and stored at
    // the end: storing it right after its load would make the wave wait a memory round trip before
    // issuing any attention load.
    static_assert(2 * AP_QB * (D / 8) == 64 * AP_W, "one chunk per thread");
    const int ft = q0 + ((threadIdx.x >> 3) & (AP_QB - 1)), fd8 = (threadIdx.x & 7) * 8, fv = threadIdx.x >> 7;
    const f16x8 fill = *reinterpret_cast<const f16x8 *>(qkv + (size_t)min(ft, T - 1) * S3 + (fv ? 2 * E : E) + h * D + fd8);
    const int qlast = min(q0 + AP_QB, T) - 1;
    const int nc = qlast / AP_CK + 1;          // chunks over keys [0, qlast]; chunk start <= q0
    const int q = q0 + jq;                     // this lane's query (q >= T: computed, not stored)
    const uint16_t *Qp = qkv + (size_t)min(q, T - 1) * S3 + h * D;
    const f16x8 qf0 = *reinterpret_cast<const f16x8 *>(Qp + 8 * g);
    const f16x8 qf1 = *reinterpret_cast<const f16x8 *>(Qp + 32 + 8 * g);
    const uint16_t *Kb = qkv + E + h * D, *Vb = qkv + 2 * E + h * D;
    char *vt = vt_all[wave];
    const int vk = 4 * (lane >> 3), vd = 8 * (lane & 7);   // V staging: keys vk..vk+3, dims vd..vd+7
    constexpr float SL2 = 0.125f * 1.4426950408889634f;     // 1/sqrt(64) * log2(e)

    struct Chunk {
        f16x8 k[2][2];   // [tile][dim half]: key 16*tile + jq, dims 32*half + 8g .. +7
        f16x8 v[4];      // keys vk + i, dims vd .. vd+7
    };
    auto load = [&](int c, Chunk &R) {
        const int kc = c * AP_CK;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint16_t *kr = Kb + (size_t)min(kc + 16 * t + jq, T - 1) * S3;   // rows past T are masked
            R.k[t][0] = *reinterpret_cast<const f16x8 *>(kr + 8 * g);
            R.k[t][1] = *reinterpret_cast<const f16x8 *>(kr + 32 + 8 * g);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            R.v[i] = *reinterpret_cast<const f16x8 *>(Vb + (size_t)min(kc + vk + i, T - 1) * S3 + vd);
    };

    float m = -INFINITY, lsum = 0.f;
    f32x4 o[4];
#pragma unroll
    for (int dg = 0; dg < 4; ++dg) o[dg] = f32x4{0.f, 0.f, 0.f, 0.f};
    // One chunk: scores, online softmax, V^T through LDS, P.V.  Two register buffers alternate
    // (the next chunk of this wave loads while one is consumed); loads are unconditional, the
    // chunk index clamped to the last one, so no buffer is ever undefined on a compiler-visible path.
    auto step = [&](int c, const Chunk &R) {
        const int kc = c * AP_CK;
        // ---- scores of keys kc + 16t + 4g + r for query q
        f32x4 s[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(R.k[t][0], qf0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(R.k[t][1], qf1, s[t], 0, 0, 0);
        }
        // Causal mask only on a chunk that reaches past the block's first query (wave-uniform test).
        if (kc + AP_CK - 1 > q0) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (kc + 16 * t + 4 * g + r > q) s[t][r] = -INFINITY;
        }
        float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                         fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
        mx = group_max(mx);
        const float mnew = fmaxf(m, mx * SL2);  // finite: key kc <= q0 <= q
        const float corr = exp2_raw(m - mnew);  // 0 on the wave's first chunk
        m = mnew;
        f16x8 pb;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) pb[4 * t + r] = (f16)exp2_raw(fmaf(s[t][r], SL2, -mnew));
        // the denominator sums exactly the fp16 probabilities the MFMA multiplies
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e += 2) ps = __builtin_amdgcn_fdot2(f16x2{pb[e], pb[e + 1]}, f16x2{1, 1}, ps, false);
        lsum = fmaf(lsum, corr, ps);
        // ---- the chunk's V rows into this wave's LDS tile, row-major: key vk + i, dims vd .. vd+7
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<f16x8 *>(vt + (vk + i) * AP_RV + 2 * vd) = R.v[i];
        // The tile is written and read by this wave only: waiting for its own LDS writes is enough
        // (the "memory" clobber keeps the compiler from moving the reads above the writes).
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) {
            // lane jq = 4q + r of group g names dims 16dg + 4r .. +3 of key (base + q); it receives
            // dim 16dg + jq of keys base .. base+3 (base 4g: the lo half, 16 + 4g: the hi half)
            const char *col = vt + 2 * (16 * dg + 4 * (jq & 3));
            const f16x4 lo = tr_read(col + (4 * g + (jq >> 2)) * AP_RV);
            const f16x4 hi = tr_read(col + (16 + 4 * g + (jq >> 2)) * AP_RV);
            const f16x8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[dg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, o[dg] * corr, 0, 0, 0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // reads done before the next chunk's writes
    };
    Chunk A, B;
    load(min(wave, nc - 1), A);
    for (int c = wave; c < nc; c += 2 * AP_W) {
        load(min(c + AP_W, nc - 1), B);
        step(c, A);
        if (c + AP_W >= nc) break;
        load(min(c + 2 * AP_W, nc - 1), A);
        step(c + AP_W, B);
    }
    // ---- merge the four waves' states: wave w finishes dims 16w .. 16w+15
    lsum = group_sum(lsum);
    if (g == 0) {
        mrg_m[wave][jq] = m;
        mrg_l[wave][jq] = lsum;
    }
#pragma unroll
    for (int dg = 0; dg < 4; ++dg) mrg_o[wave][dg][lane] = o[dg];
    __syncthreads();
    float mw[AP_W], lw[AP_W], mmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < AP_W; ++u) {
        mw[u] = mrg_m[u][jq];
        lw[u] = mrg_l[u][jq];
        mmax = (lw[u] != 0.f) ? fmaxf(mmax, mw[u]) : mmax;   // wave 0 always has keys
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
#pragma unroll
    for (int u = 0; u < AP_W; ++u) {
        const float f = (lw[u] != 0.f) ? exp2_raw(mw[u] - mmax) : 0.f;
        L += lw[u] * f;
        acc += mrg_o[u][wave][lane] * f;
    }
    if (Kc && ft < T)   // every wave, including those with no chunk
        *reinterpret_cast<f16x8 *>((fv ? Vc : Kc) + ((size_t)h * maxT + ft) * D + fd8) = fill;
    if (q < T) {
        const float inv = 1.0f / L;
        const uint2 pk = {(uint32_t)f2h(acc[0] * inv) | ((uint32_t)f2h(acc[1] * inv) << 16),
                          (uint32_t)f2h(acc[2] * inv) | ((uint32_t)f2h(acc[3] * inv) << 16)};
        uint2 *dst = reinterpret_cast<uint2 *>(att + (size_t)q * E + h * D + 16 * wave + 4 * g);
        if constexpr (COHERENT)
            __hip_atomic_store(reinterpret_cast<uint64_t *>(dst), __builtin_bit_cast(uint64_t, pk), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        else
            *dst = pk;
    }
}

}  // namespace g2

