// attn_prefill.hip -- causal prefill attention on the MFMA units (gfx950).
//
// Replaces the reference's fused attention (cuda/kernels_fused.cu:58-140; semantics of
// cpu/forward_cpu.c:83-116): att[i, h*64 + d] = sum_{j<=i} softmax_j(q_i . k_j / 8) v_j[d] over
// qkv[T, 3*768] (q | k | v, head h at columns h*64).
//
// Design, MI355X-first:
//   * A work-group owns 16 queries of one head; its four waves split the keys [0, last query] in
//     32-key chunks (chunk c on wave c % 4), each keeping its own online-softmax state, merged
//     through LDS at the end.  The heaviest query blocks (the last ones) are dispatched first.
//   * Scores on v_mfma_f32_16x16x32_f16 with the keys as the A operand and the queries as B:
//     S[key][query], so a lane holds four keys of one query (keys 4g..4g+3 of a 16-key tile, lane
//     group g = lane / 16).  K and Q fragments are 16-byte loads straight from qkv (8 consecutive
//     dims of one row per lane), no LDS.
//   * P.V as O^T[d][query] = V^T[d][key] . P[key][query]: the MFMA k-slots 8g..8g+7 of lane group g
//     are mapped to keys {4g..4g+3} of the chunk's first tile and {16+4g..16+4g+3} of its second --
//     exactly the keys the lane already holds P for -- so P is the B operand as it comes out of the
//     softmax, converted to fp16 in registers.  V^T (keys contiguous per dim) is the A operand: each
//     wave transposes its chunk's 32 x 64 V block through its own LDS tile (a lane packs four keys
//     of one dim into one 8-byte write; a fragment is two 8-byte reads).
//   * Softmax in the log2 domain (scores pre-scaled by log2(e)/8, exp2), the row maximum shared by
//     the lane groups of a query each chunk; the denominator sums the fp16-rounded probabilities
//     the MFMA sees, so the output is an exact convex combination of the value rows.
#include <cmath>

#include "common.h"

namespace g2 {

constexpr int AP_QB = 16;                      // queries per work-group
constexpr int AP_CK = 32;                      // keys per chunk
constexpr int AP_W = 4;                        // waves per work-group
constexpr int AP_RS = 2 * AP_CK + 8;           // bytes per V^T row in LDS (32 keys + 8 B pad)

__global__ __launch_bounds__(64 * AP_W) void k_attn_prefill_mfma(uint16_t *__restrict__ att,
                                                                  const uint16_t *__restrict__ qkv, int T) {
    constexpr int E = GPT2_N_EMBD, D = GPT2_HEAD_DIM, S3 = 3 * GPT2_N_EMBD;
    static_assert(D == 64 && AP_QB == 16 && AP_CK == 32, "fragment layout is written for these sizes");
    __shared__ __attribute__((aligned(16))) char vt_all[AP_W][D * AP_RS];
    __shared__ float mrg_m[AP_W][AP_QB], mrg_l[AP_W][AP_QB];
    __shared__ f32x4 mrg_o[AP_W][AP_W][64];    // [source wave][dim group][lane]

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int jq = lane & 15, g = lane >> 4;
    const int h = blockIdx.y;
    const int q0 = (gridDim.x - 1 - blockIdx.x) * AP_QB;   // heaviest blocks first
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
    // Loads are unconditional (chunk index clamped to the last one): no chunk register is ever
    // left undefined on a path the compiler can see.
    Chunk cur, nxt;
    load(min(wave, nc - 1), cur);
    for (int c = wave; c < nc; c += AP_W) {
        load(min(c + AP_W, nc - 1), nxt);   // the next chunk of this wave (a repeat at the end)
        const int kc = c * AP_CK;
        // ---- scores of keys kc + 16t + 4g + r for query q
        f32x4 s[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[t][0], qf0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[t][1], qf1, s[t], 0, 0, 0);
        }
        float x[8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) x[4 * t + r] = (kc + 16 * t + 4 * g + r <= q) ? s[t][r] * SL2 : -INFINITY;
        float mx = x[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) mx = fmaxf(mx, x[e]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m, mx);        // finite: key kc <= q0 <= q
        const float corr = exp2f(m - mnew);     // 0 on the wave's first chunk
        m = mnew;
        f16x8 pb;
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            pb[e] = (f16)exp2f(x[e] - mnew);
            ps += (float)pb[e];
        }
        lsum = lsum * corr + ps;
        // ---- V^T of the chunk into this wave's LDS tile: row d holds keys 0..31
        {
            uint32_t u[4][4];   // u[i][j]: dims vd+2j (low half), vd+2j+1 (high half) of key vk+i
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 b = __builtin_bit_cast(uint4, cur.v[i]);
                u[i][0] = b.x;
                u[i][1] = b.y;
                u[i][2] = b.z;
                u[i][3] = b.w;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // dim vd+2j: low halves of the four keys; dim vd+2j+1: high halves
                const uint2 lo = {__builtin_amdgcn_perm(u[1][j], u[0][j], 0x05040100u),
                                  __builtin_amdgcn_perm(u[3][j], u[2][j], 0x05040100u)};
                const uint2 hi = {__builtin_amdgcn_perm(u[1][j], u[0][j], 0x07060302u),
                                  __builtin_amdgcn_perm(u[3][j], u[2][j], 0x07060302u)};
                *reinterpret_cast<uint2 *>(vt + (vd + 2 * j) * AP_RS + 2 * vk) = lo;
                *reinterpret_cast<uint2 *>(vt + (vd + 2 * j + 1) * AP_RS + 2 * vk) = hi;
            }
        }
        // The tile is written and read by this wave only: waiting for its own LDS writes is enough
        // (the "memory" clobber keeps the compiler from moving the reads above the writes).
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) {
            const char *row = vt + (16 * dg + jq) * AP_RS;
            const uint2 lo = *reinterpret_cast<const uint2 *>(row + 8 * g);        // keys 4g .. 4g+3
            const uint2 hi = *reinterpret_cast<const uint2 *>(row + 32 + 8 * g);   // keys 16+4g .. 16+4g+3
            const f16x8 va = __builtin_bit_cast(f16x8, uint4{lo.x, lo.y, hi.x, hi.y});
            o[dg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, o[dg] * corr, 0, 0, 0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // reads done before the next chunk's writes
        cur = nxt;
    }
    // ---- merge the four waves' states: wave w finishes dims 16w .. 16w+15
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
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
        const float f = (lw[u] != 0.f) ? exp2f(mw[u] - mmax) : 0.f;
        L += lw[u] * f;
        acc += mrg_o[u][wave][lane] * f;
    }
    if (q < T) {
        const float inv = 1.0f / L;
        const uint2 pk = {(uint32_t)f2h(acc[0] * inv) | ((uint32_t)f2h(acc[1] * inv) << 16),
                          (uint32_t)f2h(acc[2] * inv) | ((uint32_t)f2h(acc[3] * inv) << 16)};
        *reinterpret_cast<uint2 *>(att + (size_t)q * E + h * D + 16 * wave + 4 * g) = pk;
    }
}

void attention_prefill(uint16_t *att, const uint16_t *qkv, int T) {
    hipLaunchKernelGGL(k_attn_prefill_mfma, dim3(cdiv(T, AP_QB), GPT2_N_HEAD), dim3(64 * AP_W), 0, stream(), att, qkv, T);
    check_launch("k_attn_prefill_mfma");
}

}  // namespace g2
