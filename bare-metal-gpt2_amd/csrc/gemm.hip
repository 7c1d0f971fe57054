// gemm.hip -- prefill GEMMs for gfx950: C[M,N] = A[M,K] . W[N,K]^T (+bias), fp16 in, fp32 acc.
//
// Replaces the reference's 16x16 CUDA-core tiled GEMM (cuda/kernels_tiled.cu:24-53) and its INT8
// twin (cuda/kernels_quant.cu:38-67).  Design, MI355X-first:
//   * v_mfma_f32_16x16x32_f16: W rows feed the MFMA "A" operand and activation rows the "B"
//     operand, so the accumulator holds D[n][m] = C[m][n] and each lane owns four consecutive n of
//     one output row m: the epilogue writes 8-byte vectors into row-major C.
//   * Both operands are K-contiguous, so a 16-byte load is 8 consecutive k of one row.  The MFMA
//     k-lane mapping only has to agree between the two operands (a dot product is order free), so
//     each lane group reads 8 consecutive k of its row for both.
//   * Main path k_gemm_dl: tiles go global -> LDS with global_load_lds_dwordx4 through an S-stage
//     ring (no VGPR staging), the 16-byte chunk index XOR-swizzled by row so fragment reads hit
//     distinct banks; one barrier per 64-wide k-tile.
//   * INT8 weights (weight-only scheme) stay int8 in LDS and are widened to exact fp16 as fragments
//     are read: |q| <= 127 is exact in fp16 and int8 x fp16 products are exact in fp32, so the
//     MFMA path is the fp16 one; the per-row scale is applied once in the epilogue, then the bias
//     (cuda/kernels_quant.cu:56-59).
//   * Work-group -> tile mapping is XCD-aware: consecutive work-groups go round robin over the 8
//     XCDs, so each XCD is given one contiguous run of tiles (n-major, m fastest), and the W tiles it
//     reads stay in its own L2.
//   * k_gemm_mfma (register-ring pipeline) takes INT8 weights at the GPT-2 prefill shapes (its
//     widening of each W fragment overlaps the next k-tiles' loads better than the LDS ring's) and
//     K % 64 != 0 shapes in its predicated form; shapes or pointers no MFMA path can take
//     (K % 8 != 0, unaligned rows) run k_gemm_generic.
#include <cstdlib>
#include <cstring>

#include "common.h"

namespace g2 {
void gemv(uint16_t *C, const uint16_t *x, const void *W, const float *Ws, const uint16_t *bias, int N, int K, bool qw,
          int cfg);   // gemv.hip

// 16-byte chunk swizzle inside an LDS row of CH chunks.  Eight consecutive rows read at one
// logical chunk land on eight distinct 16-byte bank groups (measured: zero SQ_LDS_BANK_CONFLICT).
template <int CH>
__device__ __forceinline__ int swz(int row, int c) {
    if constexpr (CH >= 8) return c ^ (row & 7);
    else return c ^ ((row >> 1) & 3);
}

// Map the linear work-group id onto a tile id so that each XCD owns a contiguous tile range.
__device__ __forceinline__ int xcd_tile(int bid, int ntiles) {
    const int xcd = bid & 7, slot = bid >> 3;
    const int per = ntiles >> 3, rem = ntiles & 7;
    return xcd * per + (xcd < rem ? xcd : rem) + slot;
}

// GUARD: any K % 8 == 0 (predicated, zero-filled loads); otherwise K % (BK * DEPTH) == 0.
template <int BN, int BM, int BK, int WN, int WM, bool QW, int DEPTH, bool GUARD = false>
__global__ __launch_bounds__(256) void k_gemm_mfma(uint16_t *__restrict__ C, const uint16_t *__restrict__ A,
                                                   const void *__restrict__ Wv, const float *__restrict__ Ws,
                                                   const uint16_t *__restrict__ bias, int M, int N, int K,
                                                   int tiles_m, int ntiles, int vec_store,
                                                   const uint16_t *resid) {
    (void)resid;   // the fused epilogues live in k_gemm_dl
    static_assert(WN * WM == 4, "four waves per work-group");
    constexpr int CH = BK / 8;               // 16-byte chunks per LDS row
    constexpr int WTN = BN / WN, WTM = BM / WM;  // wave tile
    constexpr int TN = WTN / 16, TM = WTM / 16;
    constexpr int GA = BM * CH;                    // 16-byte A chunks per k-tile
    constexpr int GW = QW ? BN * CH / 2 : BN * CH; // 16-byte W chunks per k-tile (int8: 16 k each)
    constexpr int NLA = (GA + 255) / 256, NLW = (GW + 255) / 256;

    __shared__ __attribute__((aligned(16))) f16x8 sW[2][BN * CH];
    __shared__ __attribute__((aligned(16))) f16x8 sA[2][BM * CH];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = xcd_tile(blockIdx.x, ntiles);
    const int n0 = (tile / tiles_m) * BN, m0 = (tile % tiles_m) * BM;
    const int wn0 = (wave / WM) * WTN, wm0 = (wave % WM) * WTM;
    const int nk = (K + BK - 1) / BK;

    const f16x8 zero8 = {};
    // Register ring: DEPTH k-tiles of global loads are in flight while one is consumed.
    f16x8 rra[DEPTH][NLA];
    i32x4 rrw[DEPTH][NLW];

    // Without GUARD, loads are never predicated: rows past M or N read the last valid row (their
    // results are not stored) and K is a multiple of BK*DEPTH, so every tile issues the same number of
    // loads and the compiler can count them (s_waitcnt vmcnt(n) on the oldest ring slot only).
    auto gload = [&](int kt, f16x8 (&ra)[NLA], i32x4 (&rw)[NLW]) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < NLA; ++i) {
            const int id = tid + 256 * i, row = id / CH, c = id % CH;
            if (GA % 256 != 0 && id >= GA) break;
            if constexpr (GUARD) {
                const int m = m0 + row, k = k0 + c * 8;
                ra[i] = (m < M && k < K) ? *reinterpret_cast<const f16x8 *>(A + (size_t)m * K + k) : zero8;
            } else {
                const int m = min(m0 + row, M - 1);
                ra[i] = *reinterpret_cast<const f16x8 *>(A + (size_t)m * K + k0 + c * 8);
            }
        }
#pragma unroll
        for (int i = 0; i < NLW; ++i) {
            const int id = tid + 256 * i;
            if (GW % 256 != 0 && id >= GW) break;
            if constexpr (QW) {
                constexpr int CQ = CH / 2;   // 16-byte int8 chunks per row
                const int row = id / CQ, c = id % CQ;
                const int8_t *src = reinterpret_cast<const int8_t *>(Wv);
                if constexpr (GUARD) {
                    const int n = n0 + row, k = k0 + c * 16;
                    rw[i] = (n < N && k < K) ? *reinterpret_cast<const i32x4 *>(src + (size_t)n * K + k) : i32x4{0, 0, 0, 0};
                } else {
                    const int n = min(n0 + row, N - 1);
                    rw[i] = *reinterpret_cast<const i32x4 *>(src + (size_t)n * K + k0 + c * 16);
                }
            } else {
                const int row = id / CH, c = id % CH;
                const uint16_t *src = reinterpret_cast<const uint16_t *>(Wv);
                if constexpr (GUARD) {
                    const int n = n0 + row, k = k0 + c * 8;
                    rw[i] = (n < N && k < K) ? *reinterpret_cast<const i32x4 *>(src + (size_t)n * K + k) : i32x4{0, 0, 0, 0};
                } else {
                    const int n = min(n0 + row, N - 1);
                    rw[i] = *reinterpret_cast<const i32x4 *>(src + (size_t)n * K + k0 + c * 8);
                }
            }
        }
    };
    auto lstore = [&](int buf, const f16x8 (&ra)[NLA], const i32x4 (&rw)[NLW]) {
#pragma unroll
        for (int i = 0; i < NLA; ++i) {
            const int id = tid + 256 * i, row = id / CH, c = id % CH;
            if (GA % 256 != 0 && id >= GA) break;
            sA[buf][row * CH + swz<CH>(row, c)] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < NLW; ++i) {
            const int id = tid + 256 * i;
            if (GW % 256 != 0 && id >= GW) break;
            if constexpr (QW) {
                constexpr int CQ = CH / 2;
                const int row = id / CQ, c = id % CQ;
                uint32_t h[8];
                i8x4_to_f16x4((uint32_t)rw[i].x, h[0], h[1]);
                i8x4_to_f16x4((uint32_t)rw[i].y, h[2], h[3]);
                i8x4_to_f16x4((uint32_t)rw[i].z, h[4], h[5]);
                i8x4_to_f16x4((uint32_t)rw[i].w, h[6], h[7]);
                const i32x4 lo = {(int)h[0], (int)h[1], (int)h[2], (int)h[3]};
                const i32x4 hi = {(int)h[4], (int)h[5], (int)h[6], (int)h[7]};
                sW[buf][row * CH + swz<CH>(row, 2 * c)] = __builtin_bit_cast(f16x8, lo);
                sW[buf][row * CH + swz<CH>(row, 2 * c + 1)] = __builtin_bit_cast(f16x8, hi);
            } else {
                const int row = id / CH, c = id % CH;
                sW[buf][row * CH + swz<CH>(row, c)] = __builtin_bit_cast(f16x8, rw[i]);
            }
        }
    };

    f32x4 acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int lrow = lane & 15, lgrp = lane >> 4;

    // Software pipeline, one barrier per k-tile.  At the top of iteration kt, LDS buffer kt&1 holds
    // tile kt and ring slot t % DEPTH holds (or is loading) tile t for t in kt+1 .. kt+DEPTH.  The
    // iteration reads tile kt's fragments, then stores tile kt+1 into the other LDS buffer and
    // refills its ring slot with tile kt+1+DEPTH, then runs the MFMAs: LDS writes, global loads and
    // MFMAs of one wave are in flight together.  The buffer written at kt was last read at kt-1,
    // before that iteration's closing barrier.  The body has no branches, so the compiler's vmcnt
    // waits stay exact (they wait for the oldest ring slot only): past the last tile the refill
    // re-reads tile nk-1 (a cache hit), and the last iteration's store fills the idle buffer.
    // DEPTH divides nk (the config table only offers a config when K % (BK*DEPTH) == 0).
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) gload(min(d, nk - 1), rra[d], rrw[d]);
    lstore(0, rra[0], rrw[0]);
    gload(min(DEPTH, nk - 1), rra[0], rrw[0]);
    __syncthreads();
    for (int kt0 = 0; kt0 < nk; kt0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int kt = kt0 + d;
            {
                constexpr int KS = BK / 32;
                f16x8 fw[KS][TN], fa[KS][TM];
                const int cur = kt & 1;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int c = ks * 4 + lgrp;
#pragma unroll
                    for (int a = 0; a < TN; ++a) {
                        const int r = wn0 + a * 16 + lrow;
                        fw[ks][a] = sW[cur][r * CH + swz<CH>(r, c)];
                    }
#pragma unroll
                    for (int b = 0; b < TM; ++b) {
                        const int r = wm0 + b * 16 + lrow;
                        fa[ks][b] = sA[cur][r * CH + swz<CH>(r, c)];
                    }
                }
                const int nxt = (d + 1) % DEPTH;   // a constant once the d-loop is unrolled
                lstore(cur ^ 1, rra[nxt], rrw[nxt]);
                gload(min(kt + 1 + DEPTH, nk - 1), rra[nxt], rrw[nxt]);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int a = 0; a < TN; ++a)
#pragma unroll
                        for (int b = 0; b < TM; ++b)
                            acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fw[ks][a], fa[ks][b], acc[a][b], 0, 0, 0);
                __syncthreads();
            }
        }
    }

    // Epilogue: lane holds D[n][m] for n = nb..nb+3, m = mrow.
#pragma unroll
    for (int a = 0; a < TN; ++a) {
        const int nb = n0 + wn0 + a * 16 + lgrp * 4;
        float sc[4] = {1.f, 1.f, 1.f, 1.f}, bs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (nb + i < N) {
                if constexpr (QW) sc[i] = Ws[nb + i];
                if (bias) bs[i] = h2f(bias[nb + i]);
            }
        }
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const int m = m0 + wm0 + b * 16 + lrow;
            if (m >= M) continue;
            uint16_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = acc[a][b][i];
                if constexpr (QW) v = v * sc[i];
                o[i] = f2h(v + bs[i]);
            }
            uint16_t *dst = C + (size_t)m * N + nb;
            if ((vec_store & 1) && nb + 3 < N) {
                const uint2 pk = {(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
                *reinterpret_cast<uint2 *>(dst) = pk;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (nb + i < N) dst[i] = o[i];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Direct-to-LDS pipeline (k_gemm_dl).  The per-CU data paths measured on MI355X set the design:
// global (L1/L2 hit) -> CU 64 B/clk, LDS reads 126 B/clk with 4 waves per CU and 234 B/clk with 8,
// fp16 MFMA 4096 FLOP/clk.  So:
//   * tiles are fetched with global_load_lds_dwordx4: each wave instruction moves 1 KB straight
//     into LDS, with no VGPR staging, no ds_write and no register ring;
//   * S LDS stages are in flight (S-1 k-tiles of loads outstanding while one is consumed), and the
//     pipeline drains exactly: no k-tile is fetched twice;
//   * the 16-byte chunk swizzle of the LDS rows is made by choosing which global chunk each lane
//     fetches (lane i of an instruction always lands at byte 16*i of its 1 KB);
//   * INT8 weights stay int8 in LDS (half the bytes) and are widened to exact fp16 as fragments
//     are read;
//   * one barrier per k-tile: the buffer refilled at step kt was last read at step kt-1.


// Split-K across work-groups (k_gemm_sk), one copy per GPU: an arrival counter per output tile
// (zero between launches: the last split of a tile resets it) and the splits' fp32 partial tiles.
// Launches that use them must not overlap on one GPU; the library enqueues every kernel on one stream.
constexpr int SK_TILES = 2048;
constexpr size_t SK_WS_WORDS = (size_t)1 << 20;   // 64-bit words: 8 MiB (larger calls take another config)
__device__ uint32_t g_sk_cnt[SK_TILES];
__device__ uint64_t g_sk_ws[SK_WS_WORDS];

// KS > 1 splits the k-tiles inside the work-group: KS groups of WN x WM waves, each with its own LDS
// ring, run the same pipeline over consecutive 1/KS shares of K (so their barriers line up), and
// groups 1.. add their accumulators into group 0's through LDS before the epilogue.
// U > 1 covers U consecutive k-tiles per barrier: their fragments are read back to back (one LDS
// round trip) and then multiplied, and U tiles are refilled at a time (S % U == 0, S >= 2U).
// EPI: the elementwise op fused into the epilogue (EPI_GELU; EPI_RESID adds resid, which may be C).
// LNP (k_gemm_dl_ln): A is the LayerNorm of X[m0 .. m0+BM) (K = 768, gamma ln_g, beta ln_b), built
// once per work-group into an LDS panel that holds all of the tile's A; the ring then carries W only.
// SK > 1 (k_gemm_sk) splits K across SK work-groups per tile (see the split-K state below).
template <int BN, int BM, int WN, int WM, int S, bool QW, int KS, int U, int EPI, bool LNP, int SK = 1>
__device__ __forceinline__ void gemm_dl(uint16_t *__restrict__ C, const uint16_t *__restrict__ A,
                                        const void *__restrict__ Wv, const float *__restrict__ Ws,
                                        const uint16_t *__restrict__ bias, int M, int N, int K, int tiles_m,
                                        int ntiles, int flags, const uint16_t *resid,
                                        const uint16_t *__restrict__ ln_g, const uint16_t *__restrict__ ln_b,
                                        const LnFold &lf) {
#if defined(__HIP_DEVICE_COMPILE__)   // LDS address-space pointers exist only in the device pass
    // flags: bit 0 = C rows are 8-byte aligned (vector stores); bits 4-7 = gn, the XCD block grid
    // (see below; 0 = contiguous runs of tiles per XCD).
    const int vec_store = flags & 1, gn = (flags >> 4) & 15;
    constexpr int NW = WN * WM;
    constexpr int BK = 64;
    constexpr int A_BYTES = BM * BK * 2;        // fp16 A tile: rows of 128 B (8 chunks)
    constexpr int RA = LNP ? 0 : A_BYTES;       // A bytes per ring stage (the LN panel holds all of A)
    constexpr int W_ROWB = QW ? BK : BK * 2;    // W tile rows: 64 B int8 (4 chunks) or 128 B fp16
    constexpr int W_BYTES = BN * W_ROWB;
    constexpr int STAGE = RA + W_BYTES;
    constexpr int PANEL = LNP ? BM * GPT2_N_EMBD * 2 : 0;
    constexpr int A_INS = RA / 1024, W_INS = W_BYTES / 1024;
    static_assert(A_BYTES % 1024 == 0 && W_BYTES % 1024 == 0, "1 KB load granules");
    static_assert(!LNP || (KS == 1 && EPI != EPI_RESID), "the LN panel form has one k group, no residual");
    static_assert(SK == 1 || (KS == 1 && !LNP), "split-K across work-groups: one k group, no LN panel");
    constexpr int TOT = A_INS + W_INS, LO = TOT / NW, REM = TOT % NW, LMAX = LO + (REM ? 1 : 0);
    constexpr int WTN = BN / WN, WTM = BM / WM, TN = WTN / 16, TM = WTM / 16;
    static_assert(TN * 16 == WTN && TM * 16 == WTM, "wave tile is whole 16x16 blocks");
    static_assert(S >= 2 && (S - 2) * LMAX < 64, "stages");
    static_assert(U >= 1 && S % U == 0 && S >= 2 * U, "k-tiles per barrier");

    // LayerNorm fold (LnFold): EPI_RESID_LN writes x*gamma of the next LayerNorm and each row's
    // partial sums; EPI_LNF / EPI_LNF_GELU finish the LayerNorm of A = x*gamma in the epilogue.  The
    // FG waves that share a block of rows (the WN column waves of every k group) split the 48 row
    // partials FSL apiece and meet in a small LDS area after the panel (part of the one LDS object).
    constexpr bool RLN = EPI == EPI_RESID_LN, LNF = EPI == EPI_LNF || EPI == EPI_LNF_GELU;
    static_assert(!(RLN || LNF) || (!LNP && SK == 1), "the LayerNorm fold is a plain direct-to-LDS form");
    constexpr int FG = WN * KS, FSL = LNF_SLOTS / FG;
    static_assert(!LNF || (FSL * FG == LNF_SLOTS && FSL % 4 == 0), "row partials split evenly, 4 lane groups");
    constexpr int FOLD_LDS = LNF ? FG * BM * 8 : 0;

    __shared__ __attribute__((aligned(1024))) char smem_all[KS * S * STAGE + PANEL + FOLD_LDS];
    char *const panel = smem_all + KS * S * STAGE;   // LNP: 12 k-tile blocks of A, as a ring stage lays them out
    float2 *const fold_red = reinterpret_cast<float2 *>(smem_all + KS * S * STAGE + PANEL);   // [FG][BM]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave_all / NW, wave = wave_all % NW;   // k group; wave inside the group
    char *smem = smem_all + kg * S * STAGE;
    const int nk = K / BK / KS / SK;                      // k-tiles per group
    const size_t welt = QW ? 1 : 2;
    // SK > 1: work-group b is split (vt % SK) of tile (vt / SK); the splits of a tile are consecutive
    // in the XCD-aware order, so they run on one XCD
    const int vt = xcd_tile(blockIdx.x, ntiles * SK);
    int tile = vt / SK;
    const int split = vt - tile * SK;
    if (SK == 1 && gn) {
        // 2-D XCD blocks: the tile grid (tiles_n x tiles_m) is cut into gn x (8 / gn) blocks and XCD x
        // (work-group b runs on XCD b % 8) takes block (x % gn, x / gn), m fastest inside it, so its L2
        // fetches W rows for tiles_n / gn n-tiles and A rows for 8 tiles_m / gn m-tiles instead of all
        // of A (the host sets gn only where both divide and ntiles % 8 == 0).
        const int xcd = blockIdx.x & 7, i = blockIdx.x >> 3;
        const int bn_ = ntiles / tiles_m / gn, bm_ = tiles_m * gn / 8;
        tile = ((xcd % gn) * bn_ + i / bm_) * tiles_m + (xcd / gn) * bm_ + i % bm_;
    }
    const int n0 = (tile / tiles_m) * BN, m0 = (tile % tiles_m) * BM;
    const int wn0 = (wave / WM) * WTN, wm0 = (wave % WM) * WTM;

    // This wave's load instructions: global source (at k = 0) and LDS offset inside a stage.
    const char *gsrc[LMAX];
    int ldst[LMAX], kstep[LMAX];
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        const int q = wave + NW * j;
        if (q < A_INS) {
            const int row = 8 * q + (lane >> 3), c = (lane & 7) ^ (row & 7);
            const int m = min(m0 + row, M - 1);
            gsrc[j] = reinterpret_cast<const char *>(A + (size_t)m * K + c * 8);
            ldst[j] = q * 1024;
            kstep[j] = BK * 2;
        } else {
            const int qw = min(q, TOT - 1) - A_INS;
            int row, c;
            if constexpr (QW) { row = 16 * qw + (lane >> 2); c = (lane & 3) ^ ((row >> 2) & 3); }
            else { row = 8 * qw + (lane >> 3); c = (lane & 7) ^ (row & 7); }
            const int n = min(n0 + row, N - 1);
            gsrc[j] = reinterpret_cast<const char *>(Wv) + (size_t)n * K * welt + c * 16;
            ldst[j] = RA + qw * 1024;
            kstep[j] = BK * (int)welt;
        }
    }
#pragma unroll
    for (int j = 0; j < LMAX; ++j) gsrc[j] += (size_t)(split * KS + kg) * nk * kstep[j];   // this group's share of K
    const int nld = (REM == 0 || wave < REM) ? LMAX : LO;   // wave-uniform
    auto issue = [&](int kt) {
        char *st = smem + (kt % S) * STAGE;
#pragma unroll
        for (int j = 0; j < LMAX; ++j)
            if (j < nld)
                __builtin_amdgcn_global_load_lds(gsrc[j] + (size_t)kt * kstep[j], G2_LDS(st + ldst[j]), 16, 0, 0);
    };
    auto wait_for = [&](int after) {
        if constexpr (REM == 0) wait_tiles<LO, S - 2>(after);
        else {
            if (wave < REM) wait_tiles<LO + 1, S - 2>(after);
            else wait_tiles<LO, S - 2>(after);
        }
    };

    f32x4 acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int lrow = lane & 15, lgrp = lane >> 4;

    // Fragments of one k-tile (2 MFMA k-steps of 32): A rows as the MFMA B operand, W rows as the
    // A operand (int8 W kept as raw codes until the MFMA phase).
    struct Frag {
        f16x8 fa[2][TM];
        f16x8 fw[2][TN];
        uint2 wq[2][TN];
    };
    auto load_frags = [&](int kt, Frag &F) {
        const char *st = smem + (kt % S) * STAGE;
        const char *sa = LNP ? panel + kt * A_BYTES : st;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int c = ks * 4 + lgrp;
#pragma unroll
            for (int b = 0; b < TM; ++b) {
                const int r = wm0 + b * 16 + lrow;
                F.fa[ks][b] = *reinterpret_cast<const f16x8 *>(sa + r * 128 + ((c ^ (r & 7)) << 4));
            }
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                const int r = wn0 + a * 16 + lrow;
                if constexpr (QW) {
                    const int cq = (ks * 2 + (lgrp >> 1)) ^ ((r >> 2) & 3);
                    F.wq[ks][a] = *reinterpret_cast<const uint2 *>(st + RA + r * 64 + (cq << 4) + ((lgrp & 1) << 3));
                } else {
                    F.fw[ks][a] = *reinterpret_cast<const f16x8 *>(st + RA + r * 128 + ((c ^ (r & 7)) << 4));
                }
            }
        }
    };
    auto mfmas = [&](const Frag &F) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                f16x8 w;
                if constexpr (QW) w = i8x8_to_f16x8(F.wq[ks][a]);
                else w = F.fw[ks][a];
#pragma unroll
                for (int b = 0; b < TM; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, F.fa[ks][b], acc[a][b], 0, 0, 0);
            }
    };

    // Epilogue operands (per-channel scales, bias, residual) are loaded here, ahead of the first
    // k-tiles: they land long before the last MFMA instead of costing the epilogue a memory round
    // trip after it.  The loads are unconditional, one element per register, at clamped indices
    // (out-of-range columns and rows are dropped in the epilogue; without a bias, A[0] stands in and
    // is not used): a branch around a load, or converting or packing the value before the
    // epilogue, would make the wave wait for the load right here.  The residual (fused only where C
    // rows are 8-byte aligned) is one 8-byte load of the lane's 4 columns per output block, by the
    // k group that stores (4 scattered 2-byte loads per block, in every k group, cost 0.8-2.3 us per
    // launch in request traffic).  (The residual may alias C: this lane is the only one that writes
    // these elements, in the epilogue.)
    // The LayerNorm fold's operands the same way: RESID_LN the next LayerNorm's gamma of the lane's
    // columns; LNF each column's (G, H) and, per row, the lane's share of the producer's row partials
    // (stored slot-major, [slot][row]: 16 lanes of a lane group read 16 consecutive rows of one slot;
    // fold member fgi takes slots fgi * FSL + lgrp + 4 j), summed below before the k-loop.
    uint32_t bs_e[TN][4];            // fp16 bias bits, zero-extended
    float sc_e[TN][4];
    uint2 rs2[TN][TM];               // fp16 residual bits, 4 columns packed
    uint32_t gm_e[RLN ? TN : 1][4];  // fp16 gamma bits
    float2 gh_e[LNF ? TN : 1][4];
    constexpr int QSLOT = LNF ? FSL / 4 : 1;
    const int fgi = wave / WM + WN * kg;
    float2 st_e[LNF ? TM : 1][QSLOT];
#pragma unroll
    for (int a = 0; a < TN; ++a) {
        const int nb = n0 + wn0 + a * 16 + lgrp * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = min(nb + i, N - 1);
            sc_e[a][i] = 1.f;
            if constexpr (QW) sc_e[a][i] = Ws[n];
            bs_e[a][i] = *(bias ? bias + n : A);
            if constexpr (RLN) gm_e[a][i] = lf.gamma[n];
            if constexpr (LNF) gh_e[a][i] = lf.gh[n];
        }
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            rs2[a][b] = uint2{0u, 0u};
            if constexpr (EPI == EPI_RESID || RLN)
                if (KS == 1 || kg == 0)
                    rs2[a][b] = *reinterpret_cast<const uint2 *>(
                        resid + (size_t)min(m0 + wm0 + b * 16 + lrow, M - 1) * N + min(nb, N - 4));
        }
    }
    if constexpr (LNF) {
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const float2 *sr =
                lf.stats_in + (size_t)(fgi * FSL + lgrp) * lf.stride + min(m0 + wm0 + b * 16 + lrow, M - 1);
#pragma unroll
            for (int j = 0; j < QSLOT; ++j) st_e[b][j] = sr[(size_t)4 * j * lf.stride];
        }
    }
    auto rs_at = [&](int a, int b, int i) -> uint16_t {
        return (uint16_t)((i < 2 ? rs2[a][b].x : rs2[a][b].y) >> (16 * (i & 1)));
    };

    // LNP: the tile's rows of X and gamma/beta are loaded first, the ring's first W tiles go out right
    // behind them, and the LayerNorm runs while those are in flight.  Wave w normalizes rows w,
    // w + NW, ...; where NW does not divide BM a wave repeats row BM-1 (the same bits to the same
    // LDS bytes).  Rows past M normalize row M-1 (never stored).  The first barrier of the k-loop
    // orders the panel writes before any fragment read.
    constexpr int RPW = LNP ? (BM + NW - 1) / NW : 1;
    f16x4 lx[RPW][3], lg[3], lb[3];
    if constexpr (LNP) {
        const int lane4 = 4 * lane;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            lg[i] = *reinterpret_cast<const f16x4 *>(ln_g + 256 * i + lane4);
            lb[i] = *reinterpret_cast<const f16x4 *>(ln_b + 256 * i + lane4);
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = min(wave + NW * r, BM - 1);
            const uint16_t *xr = A + (size_t)min(m0 + row, M - 1) * GPT2_N_EMBD;
#pragma unroll
            for (int i = 0; i < 3; ++i) lx[r][i] = *reinterpret_cast<const f16x4 *>(xr + 256 * i + lane4);
        }
    }
    // Prologue: tiles 0 .. S-U-1 in flight (the config table requires nk >= S - U, nk % U == 0).
#pragma unroll
    for (int s = 0; s < S - U; ++s) issue(s);
    // LNF: this wave's FSL partials of each row (loaded before the tiles): each lane sums its
    // slots, lanes lrow + 16 g exchange (a fixed pairing: the four lanes of the row end with the same
    // bits), and lane group 0 leaves the sum in the fold area; the k-loop's barriers (it runs at least
    // once) publish it to the epilogue.
    if constexpr (LNF) {
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int j = 0; j < QSLOT; ++j) {
                s1 += st_e[b][j].x;
                s2 += st_e[b][j].y;
            }
            s1 += __shfl_xor(s1, 16);
            s2 += __shfl_xor(s2, 16);
            s1 += __shfl_xor(s1, 32);
            s2 += __shfl_xor(s2, 32);
            if (lgrp == 0) fold_red[fgi * BM + wm0 + b * 16 + lrow] = float2{s1, s2};
        }
    }
    if constexpr (LNP) {
        const int chunk = (lane & 15) >> 1;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = min(wave + NW * r, BM - 1);
            f16x4 o[3];
            ln_row768(lx[r], lg, lb, o);
#pragma unroll
            for (int i = 0; i < 3; ++i)   // elements 256 i + 4 lane .. +3: k-tile 4 i + lane / 16
                *reinterpret_cast<f16x4 *>(panel + (4 * i + (lane >> 4)) * A_BYTES + row * 128 +
                                           ((chunk ^ (row & 7)) << 4) + (lane & 1) * 8) = o[i];
        }
    }
    int kt = 0;
    for (; kt + S - U < nk; kt += U) {
        wait_for(S - 2 * U);   // tiles kt .. kt+U-1 have landed (this wave's part; the barrier: all)
        lds_barrier();
#pragma unroll
        for (int u = 0; u < U; ++u) issue(kt + S - U + u);   // into the buffers of tiles kt-U .. kt-1
        Frag F[U];
#pragma unroll
        for (int u = 0; u < U; ++u) load_frags(kt + u, F[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) mfmas(F[u]);
    }
    for (; kt < nk; kt += U) {
        wait_for(nk - U - kt);
        lds_barrier();
        Frag F[U];
#pragma unroll
        for (int u = 0; u < U; ++u) load_frags(kt + u, F[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) mfmas(F[u]);
    }

    if constexpr (KS > 1) {
        // Groups 1.. hand their partial sums to group 0 through the (now idle) LDS rings.
        constexpr int NACC = TN * TM * 4;
        static_assert((KS - 1) * NW * NACC * 64 * 4 <= KS * S * STAGE, "reduction buffer fits the rings");
        float *red = reinterpret_cast<float *>(smem_all);
        lds_barrier();   // every group is done with its ring
        if (kg > 0) {
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int b = 0; b < TM; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        red[(((kg - 1) * NW + wave) * NACC + (a * TM + b) * 4 + i) * 64 + lane] = acc[a][b][i];
        }
        lds_barrier();
        if (kg == 0) {
#pragma unroll
            for (int g = 1; g < KS; ++g)
#pragma unroll
                for (int a = 0; a < TN; ++a)
#pragma unroll
                    for (int b = 0; b < TM; ++b)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[a][b][i] += red[(((g - 1) * NW + wave) * NACC + (a * TM + b) * 4 + i) * 64 + lane];
        }
    }
    if constexpr (SK > 1) {
        // Each split stores its fp32 accumulators into its slot of the workspace with device-scope
        // stores (they reach memory shared by every XCD), waits for them, and bumps the tile's
        // counter.  The split that arrives last sums all SK partial tiles in split order 0, 1, ..
        // (the same order whichever split is last, so the result is deterministic), resets the
        // counter for the next launch and runs the epilogue; the others are done.  Nothing waits on
        // another work-group.
        constexpr int NP = TN * TM * 2;                 // 64-bit accumulator pairs per lane
        constexpr size_t SLOT = (size_t)NW * NP * 64;   // 64-bit words per split's partial tile
        // the arrival count is broadcast through the ring, idle after the first barrier below (a
        // second LDS object would cost the k-loop its alias information, see tests/test_asm_lds_dma.py)
        uint32_t *s_arrived = reinterpret_cast<uint32_t *>(smem_all);
        uint64_t *ws = g_sk_ws + (size_t)tile * SK * SLOT + (size_t)wave * NP * 64 + lane;
        auto pack = [](float x, float y) { return (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32); };
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    __hip_atomic_store(ws + split * SLOT + ((a * TM + b) * 2 + h) * 64,
                                       pack(acc[a][b][2 * h], acc[a][b][2 * h + 1]), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        wait_vm<0>();
        __syncthreads();
        // One thread adds 1, so the count is exact whatever the compiler does with atomics of many
        // lanes (a straight-line branch: no loop runs through this barrier).
        if (tid == 0) *s_arrived = __hip_atomic_fetch_add(g_sk_cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (__builtin_amdgcn_readfirstlane(*s_arrived) != SK - 1) return;
        if (tid == 0) __hip_atomic_store(g_sk_cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint64_t part[SK][NP];
#pragma unroll
        for (int sp = 0; sp < SK; ++sp)
#pragma unroll
            for (int j = 0; j < NP; ++j)
                part[sp][j] = sp == split ? 0 : __hip_atomic_load(ws + sp * SLOT + j * 64, __ATOMIC_RELAXED,
                                                                  __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b) {
                f32x4 sum;
#pragma unroll
                for (int sp = 0; sp < SK; ++sp) {
                    f32x4 p = acc[a][b];
                    if (sp != split) {
                        const uint64_t lo = part[sp][(a * TM + b) * 2], hi = part[sp][(a * TM + b) * 2 + 1];
                        p = f32x4{__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                                  __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32))};
                    }
                    sum = sp == 0 ? p : sum + p;
                }
                acc[a][b] = sum;
            }
    }
    // LNF: each row's mean and rstd from the FG member sums, added in member order (every wave of
    // the row block gets the same bits).
    float mu_e[LNF ? TM : 1], rsd_e[LNF ? TM : 1];
    if constexpr (LNF) {
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int g = 0; g < FG; ++g) {
                const float2 p = fold_red[g * BM + wm0 + b * 16 + lrow];
                s1 += p.x;
                s2 += p.y;
            }
            const float mean = s1 * (1.0f / GPT2_N_EMBD);
            const float var = fmaxf(s2 * (1.0f / GPT2_N_EMBD) - mean * mean, 0.f);
            mu_e[b] = mean;
            rsd_e[b] = 1.0f / sqrtf(var + GPT2_LN_EPS);
        }
    }
    // Epilogue: lane holds D[n][m] for n = nb..nb+3, m = mrow.
    if (!vec_store) {
        if constexpr (RLN || LNF) return;   // the host runs the fold only where C rows are 8-byte aligned
        else {
        // Rows of C that are not 8-byte aligned (odd N: the tied head's 50257 columns): the tile
        // is staged in the now idle LDS ring and leaves row by row, a wave writing 64 consecutive
        // column pairs per store (dword-aligned in C; a lone first or last column as a 2-byte
        // store), instead of 2-byte stores scattered over 16 rows per instruction.
        constexpr int CS = BN + 4;   // staged row stride (halves): rows 8 bytes apart in banks
        static_assert(BM * CS * 2 <= KS * S * STAGE, "staged C tile fits the LDS ring");
        uint16_t *ct = reinterpret_cast<uint16_t *>(smem_all);
        lds_barrier();   // every wave is done with the last k-tile's fragments (and the k-group sums)
#pragma unroll
        for (int a = 0; a < TN && kg == 0; ++a) {
            const int nl = wn0 + a * 16 + lgrp * 4;
#pragma unroll
            for (int b = 0; b < TM; ++b) {
                const int ml = wm0 + b * 16 + lrow;
                uint16_t o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = acc[a][b][i];
                    if constexpr (QW) v = v * sc_e[a][i];
                    o[i] = epi_out<EPI>(v + (bias ? h2f((uint16_t)bs_e[a][i]) : 0.f), rs_at(a, b, i));
                }
                *reinterpret_cast<uint2 *>(ct + ml * CS + nl) =
                    uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
            }
        }
        lds_barrier();
        const int ncols = min(BN, N - n0);
        for (int r = wave_all; r < BM && m0 + r < M; r += NW * KS) {
            const uint16_t *src = ct + r * CS;
            uint16_t *dst = C + (size_t)(m0 + r) * N + n0;
            const int head = (int)(((uintptr_t)dst >> 1) & 1);   // column 0 is not 4-byte aligned
            for (int c = head + 2 * lane; c + 1 < ncols; c += 128)
                *reinterpret_cast<uint32_t *>(dst + c) = (uint32_t)src[c] | ((uint32_t)src[c + 1] << 16);
            if (lane == 0 && head) dst[0] = src[0];
            if (lane == 1 && ((ncols - head) & 1)) dst[ncols - 1] = src[ncols - 1];
        }
        return;
        }
    }
    if (kg != 0) return;
#pragma unroll
    for (int a = 0; a < TN; ++a) {
        const int nb = n0 + wn0 + a * 16 + lgrp * 4;
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const int m = m0 + wm0 + b * 16 + lrow;
            uint16_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = acc[a][b][i];
                if constexpr (QW) v = v * sc_e[a][i];
                // LNF: v is x*gamma . W_n; the row's LayerNorm finishes it (then the bias, gelu)
                if constexpr (LNF) v = __builtin_fmaf(rsd_e[b], v - mu_e[b] * gh_e[a][i].x, gh_e[a][i].y);
                o[i] = epi_out<EPI>(v + (bias ? h2f((uint16_t)bs_e[a][i]) : 0.f), rs_at(a, b, i));
            }
            if constexpr (RLN) {
                // x * gamma for the consumer, and the row's sums over these 16 columns: the lane's 4,
                // then the four lane groups of the row (every lane joins the exchange; rows past M
                // store nothing)
                float s1 = 0.f, s2 = 0.f;
                uint16_t g4[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float xv = h2f(o[i]);
                    s1 += xv;
                    s2 = __builtin_fmaf(xv, xv, s2);
                    g4[i] = f2h(xv * h2f((uint16_t)gm_e[a][i]));
                }
                s1 += __shfl_xor(s1, 16);
                s2 += __shfl_xor(s2, 16);
                s1 += __shfl_xor(s1, 32);
                s2 += __shfl_xor(s2, 32);
                if (m < M) {
                    *reinterpret_cast<uint2 *>(lf.xg + (size_t)m * N + nb) =
                        uint2{(uint32_t)g4[0] | ((uint32_t)g4[1] << 16), (uint32_t)g4[2] | ((uint32_t)g4[3] << 16)};
                    if (lgrp == 0) lf.stats_out[(size_t)((n0 + wn0 + a * 16) / 16) * lf.stride + m] = float2{s1, s2};
                }
            }
            if (m >= M) continue;
            uint16_t *dst = C + (size_t)m * N + nb;
            if (vec_store && nb + 3 < N) {
                const uint2 pk = {(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
                *reinterpret_cast<uint2 *>(dst) = pk;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (nb + i < N) dst[i] = o[i];
            }
        }
    }
#endif
}

template <int BN, int BM, int WN, int WM, int S, bool QW, int KS = 1, int U = 1, int EPI = EPI_NONE>
__global__ __launch_bounds__(WN *WM * KS * 64) void k_gemm_dl(uint16_t *__restrict__ C, const uint16_t *__restrict__ A,
                                                         const void *__restrict__ Wv, const float *__restrict__ Ws,
                                                         const uint16_t *__restrict__ bias, int M, int N, int K,
                                                         int tiles_m, int ntiles, int vec_store,
                                                         const uint16_t *resid) {
    gemm_dl<BN, BM, WN, WM, S, QW, KS, U, EPI, false>(C, A, Wv, Ws, bias, M, N, K, tiles_m, ntiles, vec_store, resid,
                                                      nullptr, nullptr, LnFold{});
}

// k_gemm_dl with K split over SK work-groups per tile (grid = tiles x SK): for tiles large enough
// to read few bytes per FLOP, which alone would leave CUs idle.
template <int BN, int BM, int WN, int WM, int S, bool QW, int U, int EPI, int SK>
__global__ __launch_bounds__(WN *WM * 64) void k_gemm_sk(uint16_t *__restrict__ C, const uint16_t *__restrict__ A,
                                                    const void *__restrict__ Wv, const float *__restrict__ Ws,
                                                    const uint16_t *__restrict__ bias, int M, int N, int K,
                                                    int tiles_m, int ntiles, int vec_store, const uint16_t *resid) {
    gemm_dl<BN, BM, WN, WM, S, QW, 1, U, EPI, false, SK>(C, A, Wv, Ws, bias, M, N, K, tiles_m, ntiles, vec_store,
                                                         resid, nullptr, nullptr, LnFold{});
}

// k_gemm_dl with the prefill's LayerNorm fold (EPI_RESID_LN, EPI_LNF, EPI_LNF_GELU; LnFold).
template <int BN, int BM, int WN, int WM, int S, bool QW, int KS, int U, int EPI>
__global__ __launch_bounds__(WN *WM * KS * 64) void k_gemm_dl_lnf(uint16_t *__restrict__ C,
                                                             const uint16_t *__restrict__ A,
                                                             const void *__restrict__ Wv, const float *__restrict__ Ws,
                                                             const uint16_t *__restrict__ bias, int M, int N, int K,
                                                             int tiles_m, int ntiles, int vec_store,
                                                             const uint16_t *resid, LnFold lf) {
    gemm_dl<BN, BM, WN, WM, S, QW, KS, U, EPI, false>(C, A, Wv, Ws, bias, M, N, K, tiles_m, ntiles, vec_store, resid,
                                                      nullptr, nullptr, lf);
}

// C = LayerNorm(X; ln_g, ln_b) . W^T (+ bias) (then gelu for EPI_GELU), K = 768: the prefill's
// LN1 -> QKV and LN2 -> fc without the LayerNorm launch and its round trip through memory.  Each
// work-group normalizes its BM rows of X itself (the rows are recomputed by every work-group of the
// same rows: N / BN times the LayerNorm's arithmetic, its reads served by L2), with the LayerNorm
// kernel's arithmetic (ln_row768), so C is bit-identical to the LayerNorm kernel followed by the
// plain GEMM on any one-k-group config.
template <int BN, int BM, int WN, int WM, int S, bool QW, int U, int EPI>
__global__ __launch_bounds__(WN *WM * 64) void k_gemm_dl_ln(uint16_t *__restrict__ C, const uint16_t *__restrict__ X,
                                                       const void *__restrict__ Wv, const float *__restrict__ Ws,
                                                       const uint16_t *__restrict__ bias, int M, int N, int K,
                                                       int tiles_m, int ntiles, int vec_store,
                                                       const uint16_t *__restrict__ ln_g,
                                                       const uint16_t *__restrict__ ln_b) {
    gemm_dl<BN, BM, WN, WM, S, QW, 1, U, EPI, true>(C, X, Wv, Ws, bias, M, N, K, tiles_m, ntiles, vec_store, nullptr,
                                                    ln_g, ln_b, LnFold{});
}

// Any shape, any alignment: 16x16 outputs per work-group, k staged through LDS as fp32.
template <bool QW>
__global__ __launch_bounds__(256) void k_gemm_generic(uint16_t *__restrict__ C, const uint16_t *__restrict__ A,
                                                      const void *__restrict__ Wv, const float *__restrict__ Ws,
                                                      const uint16_t *__restrict__ bias, int M, int N, int K) {
    __shared__ float sa[16][17], sw[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m = blockIdx.y * 16 + ty, n = blockIdx.x * 16 + tx, nw = blockIdx.x * 16 + ty;
    float acc = 0.f;
    for (int k0 = 0; k0 < K; k0 += 16) {
        const int k = k0 + tx;
        sa[ty][tx] = (m < M && k < K) ? h2f(A[(size_t)m * K + k]) : 0.f;
        float wv = 0.f;
        if (nw < N && k < K) {
            if constexpr (QW) wv = (float)reinterpret_cast<const int8_t *>(Wv)[(size_t)nw * K + k];
            else wv = h2f(reinterpret_cast<const uint16_t *>(Wv)[(size_t)nw * K + k]);
        }
        sw[ty][tx] = wv;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) acc += sa[ty][kk] * sw[tx][kk];
        __syncthreads();
    }
    if (m < M && n < N) {
        float v = acc;
        if constexpr (QW) v *= Ws[n];
        if (bias) v += h2f(bias[n]);
        C[(size_t)m * N + n] = f2h(v);
    }
}

// One thread per output, bias first, k ascending (the reference's baseline, kernels_naive.cu:44-53).
__global__ void k_gemm_naive(uint16_t *__restrict__ C, const uint16_t *__restrict__ A, const uint16_t *__restrict__ W,
                             const uint16_t *__restrict__ bias, int M, int N, int K) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)M * N) return;
    const int m = (int)(idx / N), n = (int)(idx - (long)m * N);
    float acc = bias ? h2f(bias[n]) : 0.f;
    for (int k = 0; k < K; ++k) acc += h2f(A[(size_t)m * K + k]) * h2f(W[(size_t)n * K + k]);
    C[idx] = f2h(acc);
}

// ---------------------------------------------------------------------------- tile table
typedef void (*GemmFn)(uint16_t *, const uint16_t *, const void *, const float *, const uint16_t *, int, int, int, int,
                       int, int, const uint16_t *);
struct GemmCfg {
    int bn, bm, kmul;    // K must be a multiple of kmul (BK * DEPTH, or 8 for the guarded kernel)
    int kmin, threads;   // and at least kmin; work-group size
    GemmFn fp16, int8;
    GemmFn fused[2][2];  // [int8][gelu, residual]: fused-epilogue kernels, on the configs the prefill picks
    bool dl;             // direct-to-LDS pipeline
    const char *name;
    int sk;              // > 1: K split over sk work-groups per tile (k_gemm_sk; grid = tiles x sk)
};

#define G2_NOFUSE {{nullptr, nullptr}, {nullptr, nullptr}}
#define G2_FUSE(BN, BM, WN, WM, S, KS, U) \
    {{k_gemm_dl<BN, BM, WN, WM, S, false, KS, U, EPI_GELU>, k_gemm_dl<BN, BM, WN, WM, S, false, KS, U, EPI_RESID>}, \
     {k_gemm_dl<BN, BM, WN, WM, S, true, KS, U, EPI_GELU>, k_gemm_dl<BN, BM, WN, WM, S, true, KS, U, EPI_RESID>}}
#define G2_CFG(BN, BM, BK, WN, WM, D) \
    {BN, BM, BK * D, 0, 256, k_gemm_mfma<BN, BM, BK, WN, WM, false, D>, k_gemm_mfma<BN, BM, BK, WN, WM, true, D>, \
     G2_NOFUSE, false, "bn" #BN "_bm" #BM "_bk" #BK "_w" #WN "x" #WM "_d" #D}
// Direct-to-LDS pipeline: K % 64 == 0 and at least S-1 k-tiles (per k group: K % (64 KS) == 0);
// the ...F forms also carry the fused-epilogue kernels.
#define G2_DCFG_(BN, BM, WN, WM, S, FUSE) \
    {BN, BM, 64, 64 * (S - 1), 64 * WN * WM, k_gemm_dl<BN, BM, WN, WM, S, false>, k_gemm_dl<BN, BM, WN, WM, S, true>, \
     FUSE, true, "dl_bn" #BN "_bm" #BM "_w" #WN "x" #WM "_s" #S}
#define G2_DCFG(BN, BM, WN, WM, S) G2_DCFG_(BN, BM, WN, WM, S, G2_NOFUSE)
#define G2_DCFGF(BN, BM, WN, WM, S) G2_DCFG_(BN, BM, WN, WM, S, G2_FUSE(BN, BM, WN, WM, S, 1, 1))
#define G2_DCFGK(BN, BM, WN, WM, S, KS) \
    {BN, BM, 64 * KS, 64 * KS * (S - 1), 64 * WN * WM * KS, k_gemm_dl<BN, BM, WN, WM, S, false, KS>, \
     k_gemm_dl<BN, BM, WN, WM, S, true, KS>, G2_NOFUSE, true, "dl_bn" #BN "_bm" #BM "_w" #WN "x" #WM "_s" #S "_k" #KS}
// ... and U k-tiles per barrier: K % (64 KS U) == 0, at least S-U k-tiles per group.
#define G2_DCFGU_(BN, BM, WN, WM, S, KS, U, FUSE) \
    {BN, BM, 64 * KS * U, 64 * KS * (S - U), 64 * WN * WM * KS, k_gemm_dl<BN, BM, WN, WM, S, false, KS, U>, \
     k_gemm_dl<BN, BM, WN, WM, S, true, KS, U>, FUSE, true, \
     "dl_bn" #BN "_bm" #BM "_w" #WN "x" #WM "_s" #S "_k" #KS "_u" #U}
#define G2_DCFGU(BN, BM, WN, WM, S, KS, U) G2_DCFGU_(BN, BM, WN, WM, S, KS, U, G2_NOFUSE)
#define G2_DCFGUF(BN, BM, WN, WM, S, KS, U) G2_DCFGU_(BN, BM, WN, WM, S, KS, U, G2_FUSE(BN, BM, WN, WM, S, KS, U))
// ... and K split over SK work-groups per tile: K % (64 U SK) == 0, at least S-U k-tiles per split.
#define G2_SKCFG(BN, BM, WN, WM, S, U, SK)                                                                          \
    {BN, BM, 64 * U * SK, 64 * SK * (S - U), 64 * WN * WM, k_gemm_sk<BN, BM, WN, WM, S, false, U, EPI_NONE, SK>,     \
     k_gemm_sk<BN, BM, WN, WM, S, true, U, EPI_NONE, SK>,                                                          \
     {{k_gemm_sk<BN, BM, WN, WM, S, false, U, EPI_GELU, SK>, k_gemm_sk<BN, BM, WN, WM, S, false, U, EPI_RESID, SK>}, \
      {k_gemm_sk<BN, BM, WN, WM, S, true, U, EPI_GELU, SK>, k_gemm_sk<BN, BM, WN, WM, S, true, U, EPI_RESID, SK>}},  \
     true, "sk_bn" #BN "_bm" #BM "_w" #WN "x" #WM "_s" #S "_u" #U "_x" #SK, SK}
static const GemmCfg kCfgs[] = {
    G2_DCFGF(96, 64, 2, 4, 4),      // 0: 8 waves, wave tile 48x16
    G2_DCFGF(128, 64, 4, 2, 3),     // 1: 8 waves, wave tile 32x32 (vocabulary-sized N; INT8 fc at M=1024)
    G2_DCFGF(32, 64, 1, 4, 4),      // 2: 4 waves, wave tile 32x16
    G2_DCFGF(64, 32, 2, 2, 4),      // 3: 4 waves, wave tile 32x16
    G2_DCFG(96, 64, 2, 2, 6),       // 4: 4 waves, wave tile 48x32
    G2_DCFGF(64, 64, 2, 4, 4),      // 5: 8 waves, wave tile 32x16
    G2_DCFGF(128, 128, 2, 4, 4),    // 6: 8 waves, wave tile 64x32
    G2_DCFG(256, 128, 4, 2, 3),     // 7: 8 waves, wave tile 64x64
    G2_DCFGF(32, 32, 1, 2, 4),      // 8: 2 waves, wave tile 32x16
    G2_DCFG(48, 32, 3, 2, 4),       // 9: 6 waves, wave tile 16x16
    G2_DCFG(48, 32, 1, 2, 4),       // 10: 2 waves, wave tile 48x16
    G2_DCFG(48, 32, 3, 2, 6),       // 11: 6 waves, wave tile 16x16, 6 stages
    G2_DCFGK(32, 64, 1, 4, 4, 2),   // 12: two k groups of 4 waves (K=3072: 24 k-tiles each)
    G2_DCFGK(32, 32, 1, 2, 4, 2),   // 13: two k groups of 2 waves
    G2_DCFGK(32, 32, 1, 2, 4, 4),   // 14: four k groups of 2 waves
    G2_DCFGK(48, 32, 3, 2, 4, 2),   // 15: two k groups of 6 waves
    G2_DCFGK(32, 64, 1, 4, 4, 3),   // 16: three k groups of 4 waves
    G2_DCFGK(64, 32, 2, 2, 4, 2),   // 17: two k groups of 4 waves
    G2_DCFGK(32, 64, 1, 4, 3, 2),   // 18: two k groups of 4 waves, 3 stages
    G2_DCFG(96, 32, 3, 2, 4),       // 19: 6 waves, wave tile 32x16
    G2_DCFG(48, 64, 3, 4, 4),       // 20: 12 waves, wave tile 16x16
    G2_DCFGK(128, 64, 4, 2, 3, 2),  // 21: two k groups of 8 waves
    G2_DCFGU(48, 32, 3, 2, 4, 2, 2),  // 22: as 15, two k-tiles per barrier
    G2_DCFGUF(48, 32, 3, 2, 6, 2, 2), // 23: as 15, two k-tiles per barrier, 6 stages (mlp-proj)
    G2_DCFGU(48, 32, 3, 2, 4, 1, 2),  // 24: as 9, two k-tiles per barrier (QKV)
    G2_DCFGUF(48, 32, 3, 2, 6, 1, 2), // 25: as 9, two k-tiles per barrier, 6 stages (attn-proj)
    G2_DCFGUF(48, 64, 3, 4, 4, 1, 2), // 26: as 20, two k-tiles per barrier (fc)
    G2_DCFGU(48, 64, 3, 4, 6, 1, 2),  // 27: as 20, two k-tiles per barrier, 6 stages
    G2_DCFGU(48, 32, 3, 2, 6, 1, 3),  // 28: as 9, three k-tiles per barrier
    G2_DCFGU(48, 64, 3, 4, 6, 1, 3),  // 29: as 20, three k-tiles per barrier
    G2_DCFGU(48, 32, 3, 2, 6, 2, 3),  // 30: as 15, three k-tiles per barrier
    G2_DCFGUF(48, 32, 3, 2, 8, 1, 4), // 31: as 9, four k-tiles per barrier (INT8 attn-proj)
    G2_DCFGU(48, 64, 3, 4, 8, 1, 4),  // 32: as 20, four k-tiles per barrier
    G2_DCFGUF(48, 32, 3, 2, 8, 2, 4), // 33: as 15, four k-tiles per barrier (160 KB of LDS; INT8 mlp-proj)
    G2_DCFGUF(48, 64, 3, 2, 4, 1, 2),   // 34: 6 waves, wave tile 16x32 (each widened INT8 fragment feeds 2 MFMAs)
    G2_DCFGUF(48, 32, 3, 1, 4, 1, 2),   // 35: 3 waves, wave tile 16x32 (INT8 QKV, fc)
    G2_DCFGUF(48, 64, 3, 2, 4, 2, 2),   // 36: two k groups of 6 waves, wave tile 16x32
    G2_DCFGU(96, 64, 3, 2, 4, 1, 2),    // 37: 6 waves, wave tile 32x32
    G2_DCFGUF(48, 32, 3, 1, 8, 2, 4),   // 38: two k groups of 3 waves, 8 stages, 4 k-tiles per barrier
    G2_DCFGUF(48, 32, 3, 1, 6, 2, 2),   // 39: two k groups of 3 waves, 6 stages
    G2_DCFGUF(48, 32, 3, 1, 8, 1, 4),   // 40: 3 waves, 8 stages, 4 k-tiles per barrier
    // register-ring pipeline (k_gemm_mfma): reference points for tuning
    G2_CFG(96, 64, 64, 2, 2, 6),    // 41: wave tile 48x32
    G2_CFG(64, 32, 64, 2, 2, 6),    // 42: wave tile 32x16
    G2_CFG(32, 64, 64, 1, 4, 6),    // 43: wave tile 32x16
    G2_CFG(128, 128, 64, 2, 2, 2),  // 44: wave tile 64x64
    G2_DCFGUF(48, 32, 3, 1, 4, 4, 2),   // 45: four k groups of 3 waves, 16x32 wave tiles (INT8 mlp-proj)
    G2_DCFG(128, 64, 4, 2, 2),          // 46: as 1, double-buffered (49 KB of LDS: three work-groups per CU)
    G2_DCFGUF(32, 32, 1, 2, 4, 4, 1),   // 47: as 14 (four k groups of 2 waves), with the fused epilogues
    // split K over work-groups (k_gemm_sk): large tiles (half the L2 bytes per FLOP of the 48x32 tiles)
    // and still 256+ work-groups.  Measured 30-50% slower than the picks above at P=512: the partial
    // tiles cross XCDs through memory (the stores' drain, then the last split's loads: ~3 us of a
    // 5-10 us launch), so no pick uses them.
    G2_SKCFG(96, 64, 3, 2, 4, 2, 2),    // 48: 6 waves, wave tile 32x32, 2 splits
    G2_SKCFG(96, 64, 6, 2, 4, 2, 2),    // 49: 12 waves, wave tile 16x32, 2 splits
    G2_SKCFG(96, 64, 6, 2, 4, 2, 4),    // 50: as 49, 4 splits
    G2_SKCFG(64, 64, 2, 2, 4, 2, 2),    // 51: 4 waves, wave tile 32x32, 2 splits
};
static const int kNumCfgs = (int)(sizeof(kCfgs) / sizeof(kCfgs[0]));
static_assert(sizeof(kCfgs) / sizeof(kCfgs[0]) == 52, "the pick table names configs by index");

// Any K % 8 == 0 (int8: K % 16 == 0): predicated loads, one k-tile of prefetch.
#define G2_GCFG(BN, BM, WN, WM) \
    {BN, BM, 8, 0, 256, k_gemm_mfma<BN, BM, 64, WN, WM, false, 1, true>, k_gemm_mfma<BN, BM, 64, WN, WM, true, 1, true>, \
     G2_NOFUSE, false, "guard_bn" #BN "_bm" #BM}
static const GemmCfg kGuardCfgs[] = {
    G2_GCFG(64, 64, 2, 2),
    G2_GCFG(64, 32, 2, 2),
};

// LayerNorm-panel GEMMs (k_gemm_dl_ln): K = 768, BM = 32, one k group.
typedef void (*GemmLnFn)(uint16_t *, const uint16_t *, const void *, const float *, const uint16_t *, int, int, int,
                         int, int, int, const uint16_t *, const uint16_t *);
struct GemmLnCfg {
    int bn, bm, threads;
    GemmLnFn fn[2][2];   // [int8][EPI_NONE, EPI_GELU]
    const char *name;
};
#define G2_LNCFG(BN, BM, WN, WM, S, U)                                                                         \
    {BN, BM, 64 * WN * WM,                                                                                     \
     {{k_gemm_dl_ln<BN, BM, WN, WM, S, false, U, EPI_NONE>, k_gemm_dl_ln<BN, BM, WN, WM, S, false, U, EPI_GELU>}, \
      {k_gemm_dl_ln<BN, BM, WN, WM, S, true, U, EPI_NONE>, k_gemm_dl_ln<BN, BM, WN, WM, S, true, U, EPI_GELU>}},  \
     "ln_bn" #BN "_bm" #BM "_w" #WN "x" #WM "_s" #S "_u" #U}
static const GemmLnCfg kLnCfgs[] = {
    G2_LNCFG(64, 32, 2, 2, 4, 2),   // 0: 4 waves, wave tile 32x16
    G2_LNCFG(96, 32, 6, 1, 4, 2),   // 1: 6 waves, wave tile 16x32
    G2_LNCFG(96, 32, 3, 1, 4, 2),   // 2: 3 waves, wave tile 32x32
};
static const int kNumLnCfgs = (int)(sizeof(kLnCfgs) / sizeof(kLnCfgs[0]));

// The LayerNorm fold's kernels, on the configs the pick table gives each role: the residual GEMMs
// (attn-proj, mlp-proj: EPI_RESID_LN) and the GEMMs after a LayerNorm (QKV: EPI_LNF, fc:
// EPI_LNF_GELU), fp16 and INT8 weights, every M bucket.  A call whose picked config has no entry
// here (a forced config) runs the LayerNorm launch and the plain GEMM instead.
typedef void (*GemmLnfFn)(uint16_t *, const uint16_t *, const void *, const float *, const uint16_t *, int, int, int,
                          int, int, int, const uint16_t *, LnFold);
struct GemmLnfEntry {
    int cfg;
    bool qw;
    int epi;
    GemmLnfFn fn;
};
#define G2_LNF(CFG, QW, EPI, BN, BM, WN, WM, S, KS, U) {CFG, QW, EPI, k_gemm_dl_lnf<BN, BM, WN, WM, S, QW, KS, U, EPI>}
static const GemmLnfEntry kLnfKernels[] = {
    // residual GEMMs: fp16 attn-proj 8, 25, 36 / mlp-proj 47, 23, 5; INT8 attn-proj 47, 31, 36 / mlp-proj 45, 36
    G2_LNF(5, false, EPI_RESID_LN, 64, 64, 2, 4, 4, 1, 1),
    G2_LNF(8, false, EPI_RESID_LN, 32, 32, 1, 2, 4, 1, 1),
    G2_LNF(23, false, EPI_RESID_LN, 48, 32, 3, 2, 6, 2, 2),
    G2_LNF(25, false, EPI_RESID_LN, 48, 32, 3, 2, 6, 1, 2),
    G2_LNF(36, false, EPI_RESID_LN, 48, 64, 3, 2, 4, 2, 2),
    G2_LNF(47, false, EPI_RESID_LN, 32, 32, 1, 2, 4, 4, 1),
    G2_LNF(31, true, EPI_RESID_LN, 48, 32, 3, 2, 8, 1, 4),
    G2_LNF(36, true, EPI_RESID_LN, 48, 64, 3, 2, 4, 2, 2),
    G2_LNF(45, true, EPI_RESID_LN, 48, 32, 3, 1, 4, 4, 2),
    G2_LNF(47, true, EPI_RESID_LN, 32, 32, 1, 2, 4, 4, 1),
    // QKV: fp16 8, 29, 35, 0; INT8 47, 39, 36, 35
    G2_LNF(0, false, EPI_LNF, 96, 64, 2, 4, 4, 1, 1),
    G2_LNF(8, false, EPI_LNF, 32, 32, 1, 2, 4, 1, 1),
    G2_LNF(29, false, EPI_LNF, 48, 64, 3, 4, 6, 1, 3),
    G2_LNF(35, false, EPI_LNF, 48, 32, 3, 1, 4, 1, 2),
    G2_LNF(35, true, EPI_LNF, 48, 32, 3, 1, 4, 1, 2),
    G2_LNF(36, true, EPI_LNF, 48, 64, 3, 2, 4, 2, 2),
    G2_LNF(39, true, EPI_LNF, 48, 32, 3, 1, 6, 2, 2),
    G2_LNF(47, true, EPI_LNF, 32, 32, 1, 2, 4, 4, 1),
    // fc: fp16 8, 40, 26, 6; INT8 47, 39, 36, 35, 1
    G2_LNF(6, false, EPI_LNF_GELU, 128, 128, 2, 4, 4, 1, 1),
    G2_LNF(8, false, EPI_LNF_GELU, 32, 32, 1, 2, 4, 1, 1),
    G2_LNF(26, false, EPI_LNF_GELU, 48, 64, 3, 4, 4, 1, 2),
    G2_LNF(40, false, EPI_LNF_GELU, 48, 32, 3, 1, 8, 1, 4),
    G2_LNF(1, true, EPI_LNF_GELU, 128, 64, 4, 2, 3, 1, 1),
    G2_LNF(35, true, EPI_LNF_GELU, 48, 32, 3, 1, 4, 1, 2),
    G2_LNF(36, true, EPI_LNF_GELU, 48, 64, 3, 2, 4, 2, 2),
    G2_LNF(39, true, EPI_LNF_GELU, 48, 32, 3, 1, 6, 2, 2),
    G2_LNF(47, true, EPI_LNF_GELU, 32, 32, 1, 2, 4, 4, 1),
};

static int g_force_cfg = -2;  // -2: not read yet; -1: table

static bool cfg_fits(int c, int K) { return K % kCfgs[c].kmul == 0 && K >= kCfgs[c].kmin; }

// A split-K config also needs its tiles within the counters and its partial tiles within the workspace.
static bool sk_room(const GemmCfg &g, int M, int N) {
    if (g.sk <= 1) return true;
    const long tiles = (long)cdiv(M, g.bm) * cdiv(N, g.bn);
    return tiles <= SK_TILES && tiles * g.sk * g.bn * g.bm / 2 <= (long)SK_WS_WORDS;
}
static bool cfg_usable(int c, int M, int N, int K) { return cfg_fits(c, K) && sk_room(kCfgs[c], M, N); }

// The config forced by gpt2_tune_gemm_force or the GPT2_GEMM_CFG environment variable, or -1.
static int forced_cfg() {
    if (g_force_cfg == -2) {
        const char *e = getenv("GPT2_GEMM_CFG");
        g_force_cfg = e ? atoi(e) : -1;
        if (g_force_cfg >= kNumCfgs) g_force_cfg = -1;
    }
    return g_force_cfg;
}

// Measured picks for the GPT-2 trunk shapes, by prompt length: each shape's 12 layer GEMMs
// (distinct weights) back to back on MI355X, every config of the table timed per M bucket (fp16 and
// INT8 weights), then for M in (256, 512] the whole step (12 layers x {QKV, attn-proj, fc, mlp-proj})
// timed over per-shape candidates, because a kernel's best config alone and inside the step differ
// (attn-proj most).  Buckets: M <= 64, <= 128, <= 256, <= 512, <= 1024; shapes QKV, attn-proj, fc,
// mlp-proj; {fp16, INT8}.  Every config the prefill picks for attn-proj, fc and mlp-proj carries the
// fused-epilogue kernels (gelu, residual).
//   * short prompts take small tiles with k groups: 32x32 tiles with four k groups (47) keep 256+
//     waves busy on mlp-proj's K=3072 (M=128: 6.6 us against 10.1 with one group) and on every INT8
//     shape up to M=256 (M=64 QKV: 3.95 against 6.3 us), where each wave widens fewer W rows;
//   * M in (256, 512] (the P=512 headline): 48-row W tiles, chosen inside the step;
//   * M up to 1024: 96x64 / 128x128 tiles for fp16 QKV and fc (10.4 / 10.9 us), 64x64 for mlp-proj
//     (12.9 against 16.5 us), 48x64 with two k groups (36) for attn-proj and the INT8 GEMMs, 128x64
//     for INT8 fc (12.0 against 13.4 us for 48x32, isolated).
static const int kPick[5][4][2] = {
    /* M <= 64   */ {{8, 47}, {8, 47}, {8, 47}, {47, 47}},
    /* M <= 128  */ {{8, 39}, {8, 47}, {8, 39}, {47, 47}},
    /* M <= 256  */ {{29, 36}, {8, 47}, {40, 36}, {47, 45}},
    /* M <= 512  */ {{35, 35}, {25, 31}, {26, 35}, {23, 45}},
    /* M <= 1024 */ {{0, 35}, {36, 36}, {6, 1}, {5, 36}},
};

static int pick_cfg(int M, int N, int K, bool qw = false) {
    if (forced_cfg() >= 0 && cfg_usable(g_force_cfg, M, N, K)) return g_force_cfg;
    int shape = -1;
    if (N == 2304 && K == 768) shape = 0;            // QKV
    else if (N == 768 && K == 768) shape = 1;        // attn-proj
    else if (N == 3072 && K == 768) shape = 2;       // fc
    else if (N == 768 && K == 3072) shape = 3;       // mlp-proj
    if (shape >= 0 && M >= 2 && M <= 1024) {
        const int bucket = M <= 64 ? 0 : M <= 128 ? 1 : M <= 256 ? 2 : M <= 512 ? 3 : 4;
        const int c = kPick[bucket][shape][qw ? 1 : 0];
        if (cfg_usable(c, M, N, K)) return c;
    }
    // Other shapes: vocabulary-sized N (the tied head, 50257 rows of W) has many tiles per CU, where
    // large tiles win on L2 bytes per FLOP (M=512: 128x64 83 us, 256x128 88, 128x128 94, 48-row
    // tiles >= 135) and the 128x64 tile double-buffered (three work-groups per CU) beats its 3-stage
    // form (64 vs 74 us).  Few rows and a long K: four k groups per tile keep more waves busy.
    // Otherwise the largest tile that still gives about one work-group per CU (256 CUs), among the
    // configs whose K constraint holds; -1 when none does (the guarded kernel runs).
    if (M <= 64 && K >= 2048 && N <= 4096 && cfg_fits(47, K)) return 47;
    if (N >= 16384 && M > 32 && cfg_fits(46, K)) return 46;
    if (N >= 16384 && M > 32 && cfg_fits(1, K)) return 1;
    const int order[] = {6, 0, 5, 2, 3, 8};
    int last = -1;
    for (int c : order) {
        if (!cfg_fits(c, K)) continue;
        last = c;
        const long t = (long)cdiv(N, kCfgs[c].bn) * cdiv(M, kCfgs[c].bm);
        if (t >= 256) return c;
    }
    return last;
}

bool gemm_skinny(uint16_t *C, const uint16_t *A, const void *W, const float *Ws, const uint16_t *bias, int M, int N,
                 int K, bool qw, int epi, const uint16_t *resid, const uint16_t *ln_g, const uint16_t *ln_b);

static bool mfma_ok(const void *A, const void *W, int K, bool qw) {
    if (qw) return (K % 16) == 0 && aligned16(A) && aligned16(W);
    return (K % 8) == 0 && aligned16(A) && aligned16(W);
}

// The XCD block grid gn for a direct-to-LDS launch (0: contiguous runs of tiles per XCD).  Each XCD's
// L2 fetches the W rows of its n-tiles and the A rows of its m-tiles once; with contiguous runs every
// XCD covers all m-tiles, so A (at K = 3072 the 3 MB activation of mlp-proj) is fetched by all eight.
// gn x (8 / gn) blocks minimize those bytes.  Measured on MI355X at P=512: mlp-proj (K = 3072) moves
// 26% fewer bytes past its L2s at the same speed; attn-proj (K = 768) ran 4.5% slower, so shorter K
// keeps the contiguous runs.
static int xcd_blocks(const GemmCfg &g, int tiles_m, int tiles_n, int K, bool qw) {
    if (!g.dl || g.sk > 1 || K < 2048 || (tiles_m * tiles_n) % 8) return 0;
    const long wrow = (long)g.bn * (qw ? 1 : 2), arow = (long)g.bm * 2;   // bytes per k of one n-tile / m-tile
    int best = 0;
    long best_cost = 0;
    for (int gn = 8; gn >= 1; gn /= 2) {
        const int gm = 8 / gn;
        if (tiles_n % gn || tiles_m % gm) continue;
        const long cost = tiles_n / gn * wrow + tiles_m / gm * arow;
        if (!best || cost < best_cost) { best = gn; best_cost = cost; }
    }
    // gn = 8 is what contiguous runs already give when 8 divides tiles_n
    return (best == 8 && tiles_n % 8 == 0) ? 0 : best;
}

static void launch_gemm(const GemmCfg &g, GemmFn fn, uint16_t *C, const uint16_t *A, const void *W, const float *Ws,
                        const uint16_t *bias, int M, int N, int K, const uint16_t *resid = nullptr) {
    const int tiles_m = cdiv(M, g.bm), tiles_n = cdiv(N, g.bn);
    const int ntiles = tiles_m * tiles_n;
    const int vec = (N % 4 == 0) && (((uintptr_t)C & 7u) == 0);
    hipLaunchKernelGGL(fn, dim3(ntiles * (g.sk > 1 ? g.sk : 1)), dim3(g.threads), 0, stream(), C, A, W, Ws, bias, M, N,
                       K, tiles_m, ntiles, vec | (xcd_blocks(g, tiles_m, tiles_n, K, Ws != nullptr) << 4), resid);
}

static bool gemm_args(const char *who, const void *C, const void *A, const void *W, int M, int N, int K) {
    if (M < 0 || N < 0 || K < 0) return arg_fail(who);
    if ((long)M * N > 0 && (!C || !A || !W)) return arg_fail(who);
    return false;
}

void gemm(uint16_t *C, const uint16_t *A, const void *W, const float *Ws, const uint16_t *bias, int M, int N, int K,
          bool qw, int cfg) {
    if ((long)M * N == 0) return;
    // M = 1 (the prefill's last-row head, a decode-shaped call) is a GEMV: the tiles would compute
    // 128 rows and keep one.  Tuning runs that force a tile config keep the GEMM.
    if (M == 1 && K > 0 && cfg < 0 && forced_cfg() < 0) {
        gemv(C, A, W, Ws, bias, N, K, qw, -1);
        return;
    }
    // A few rows of A (short prompts): the product is a weight stream, taken by the skinny kernel
    // (gemm_skinny.hip) where its shapes allow.  Tuning runs that force a tile config keep the tiles.
    if (cfg < 0 && forced_cfg() < 0 && gemm_skinny(C, A, W, Ws, bias, M, N, K, qw, EPI_NONE, nullptr, nullptr, nullptr))
        return;
    // K == 0 (an empty sum, C = bias or 0) falls through to the generic kernel.
    if (K > 0 && mfma_ok(A, W, K, qw)) {
        const int c = (cfg >= 0 && cfg < kNumCfgs && cfg_usable(cfg, M, N, K)) ? cfg : pick_cfg(M, N, K, qw);
        const GemmCfg &g = c >= 0 ? kCfgs[c] : kGuardCfgs[(long)cdiv(N, 64) * cdiv(M, 64) >= 256 ? 0 : 1];
        launch_gemm(g, qw ? g.int8 : g.fp16, C, A, W, Ws, bias, M, N, K);
        check_launch(qw ? "k_gemm_mfma<int8>" : "k_gemm_mfma<fp16>");
        return;
    }
    dim3 grid(cdiv(N, 16), cdiv(M, 16));
    if (qw) hipLaunchKernelGGL(k_gemm_generic<true>, grid, dim3(256), 0, stream(), C, A, W, Ws, bias, M, N, K);
    else hipLaunchKernelGGL(k_gemm_generic<false>, grid, dim3(256), 0, stream(), C, A, W, Ws, bias, M, N, K);
    check_launch("k_gemm_generic");
}

// C = A . W^T (+ bias) followed by the elementwise op `epi` (EPI_GELU, or EPI_RESID: C = resid +
// product, resid may be C itself), in one launch.  Fused-epilogue kernels exist for the
// direct-to-LDS configs the prefill picks; returns false (nothing launched) when the picked config
// has none, for M = 1 (the GEMV), shapes or pointers the MFMA paths cannot take, or (EPI_RESID) C
// or resid rows that are not 8-byte aligned -- the caller then runs the unfused sequence.
bool gemm_fused(uint16_t *C, const uint16_t *A, const void *W, const float *Ws, const uint16_t *bias, int M, int N,
                int K, bool qw, int epi, const uint16_t *resid) {
    if (M <= 1 || N <= 0 || K <= 0 || !mfma_ok(A, W, K, qw)) return false;
    // the residual form reads the residual 4 columns (8 bytes) at a time
    if (epi == EPI_RESID && (!resid || N % 4 || (((uintptr_t)resid | (uintptr_t)C) & 7u))) return false;
    if (epi != EPI_GELU && epi != EPI_RESID) return false;
    if (forced_cfg() < 0 && gemm_skinny(C, A, W, Ws, bias, M, N, K, qw, epi, resid, nullptr, nullptr)) return true;
    const int c = pick_cfg(M, N, K, qw);
    if (c < 0) return false;
    const GemmFn fn = kCfgs[c].fused[qw ? 1 : 0][epi == EPI_RESID ? 1 : 0];
    if (!fn) return false;
    launch_gemm(kCfgs[c], fn, C, A, W, Ws, bias, M, N, K, resid);
    check_launch(qw ? "k_gemm_dl<int8> fused" : "k_gemm_dl<fp16> fused");
    return true;
}

// The prefill's LayerNorm-panel fusion is off unless a config is forced (gpt2_tune_gemm_ln_force):
// measured on MI355X (bench/prefill_bench.py --ln-cfg) the whole P=512 INT8 prefill takes 0.754 ms
// with the best config against 0.608 ms with the LayerNorm launch and the plain GEMM (T=1024: 1.16
// against 0.91 ms; T=128: no faster).  Every work-group of a 32-row block normalizes the same 32 rows
// before its first MFMA (24 to 48 work-groups per row block), each wave reducing 6 to 11 rows in
// sequence, and the 48 KB panel halves the work-groups resident per CU.
static int g_ln_cfg = -1;   // >= 0: the prefill's QKV and fc run that config; -1: off
int gemm_ln_forced() { return g_ln_cfg; }

// C = LayerNorm(X; ln_g, ln_b) . W^T (+ bias), then gelu for EPI_GELU, in one launch (K = 768).
// cfg < 0 takes the forced config, if any.  Returns false (nothing launched) when no LayerNorm-panel kernel
// covers the call: the caller then runs the LayerNorm kernel and the GEMM.
bool gemm_ln(uint16_t *C, const uint16_t *X, const uint16_t *ln_g, const uint16_t *ln_b, const void *W,
             const float *Ws, const uint16_t *bias, int M, int N, int K, bool qw, int epi, int cfg) {
    if (M <= 1 || N <= 0 || K != GPT2_N_EMBD || !mfma_ok(X, W, K, qw)) return false;
    if (!ln_g || !ln_b || (((uintptr_t)ln_g | (uintptr_t)ln_b) & 7u)) return false;
    if (epi != EPI_NONE && epi != EPI_GELU) return false;
    const int c = cfg >= 0 ? (cfg < kNumLnCfgs ? cfg : -1) : g_ln_cfg;
    if (c < 0) return false;
    const GemmLnCfg &g = kLnCfgs[c];
    const int tiles_m = cdiv(M, g.bm), ntiles = tiles_m * cdiv(N, g.bn);
    const int vec = (N % 4 == 0) && (((uintptr_t)C & 7u) == 0);
    hipLaunchKernelGGL(g.fn[qw ? 1 : 0][epi == EPI_GELU ? 1 : 0], dim3(ntiles), dim3(g.threads), 0, stream(), C, X, W,
                       Ws, bias, M, N, K, tiles_m, ntiles, vec, ln_g, ln_b);
    check_launch(qw ? "k_gemm_dl_ln<int8>" : "k_gemm_dl_ln<fp16>");
    return true;
}

// One matmul of the prefill's LayerNorm fold (LnFold): EPI_RESID_LN (C = resid + A.W^T + b into C,
// plus x*gamma and the row partials; N = 768) or EPI_LNF / EPI_LNF_GELU (A = x*gamma, K = 768).
// Returns false (nothing launched) when the picked config has no fold kernel, for M = 1, or where C
// (and the residual) rows are not 8-byte aligned -- the caller then runs the unfolded sequence.
bool gemm_lnfold(int epi, uint16_t *C, const uint16_t *A, const void *W, const float *Ws, const uint16_t *bias, int M,
                 int N, int K, bool qw, const uint16_t *resid, const LnFold &lf) {
    if (M <= 1 || N <= 0 || K <= 0 || !mfma_ok(A, W, K, qw) || N % 4 || ((uintptr_t)C & 7u)) return false;
    if (lf.stride < M) return false;
    if (epi == EPI_RESID_LN) {
        if (N != GPT2_N_EMBD || !resid || ((uintptr_t)resid & 7u) || ((uintptr_t)lf.xg & 7u) || !lf.gamma ||
            !lf.stats_out)
            return false;
    } else if (epi == EPI_LNF || epi == EPI_LNF_GELU) {
        if (K != GPT2_N_EMBD || !lf.stats_in || !lf.gh) return false;
    } else {
        return false;
    }
    const int c = pick_cfg(M, N, K, qw);
    if (c < 0) return false;
    for (const GemmLnfEntry &e : kLnfKernels) {
        if (e.cfg != c || e.qw != qw || e.epi != epi) continue;
        const GemmCfg &g = kCfgs[c];
        if (!cfg_usable(c, M, N, K)) return false;
        const int tiles_m = cdiv(M, g.bm), tiles_n = cdiv(N, g.bn);
        const int ntiles = tiles_m * tiles_n;
        hipLaunchKernelGGL(e.fn, dim3(ntiles), dim3(g.threads), 0, stream(), C, A, W, Ws, bias, M, N, K, tiles_m,
                           ntiles, 1 | (xcd_blocks(g, tiles_m, tiles_n, K, qw) << 4), resid, lf);
        check_launch("k_gemm_dl_lnf");
        return true;
    }
    return false;
}

}  // namespace g2

using namespace g2;

extern "C" void gpt2_matmul_tiled(gpt2_half *C, const gpt2_half *A, const gpt2_half *W, const gpt2_half *bias,
                                  int M, int N, int K) {
    if (gemm_args("gpt2_matmul_tiled: bad shape or null pointer", C, A, W, M, N, K)) return;
    gemm(C, A, W, nullptr, bias, M, N, K, false, -1);
}

extern "C" void gpt2_matmul_int8(gpt2_half *C, const gpt2_half *A, const int8_t *Wq, const float *Ws,
                                 const gpt2_half *bias, int M, int N, int K) {
    if (gemm_args("gpt2_matmul_int8: bad shape or null pointer", C, A, Wq, M, N, K)) return;
    if ((long)M * N > 0 && !Ws) { arg_fail("gpt2_matmul_int8: null scales"); return; }
    gemm(C, A, Wq, Ws, bias, M, N, K, true, -1);
}

extern "C" void gpt2_matmul_naive(gpt2_half *C, const gpt2_half *A, const gpt2_half *W, const gpt2_half *bias,
                                  int M, int N, int K) {
    if (gemm_args("gpt2_matmul_naive: bad shape or null pointer", C, A, W, M, N, K)) return;
    const long total = (long)M * N;
    if (total == 0) return;
    hipLaunchKernelGGL(k_gemm_naive, dim3(cdiv(total, 256)), dim3(256), 0, stream(), C, A, W, bias, M, N, K);
    check_launch("k_gemm_naive");
}

// Tuning hooks (not part of the reference interface): run one GEMM with a fixed tile config.
extern "C" int gpt2_tune_gemm_count(void) { return kNumCfgs; }
extern "C" const char *gpt2_tune_gemm_name(int cfg) { return cfg >= 0 && cfg < kNumCfgs ? kCfgs[cfg].name : "?"; }
extern "C" int gpt2_tune_gemm_pick(int M, int N, int K) { return pick_cfg(M, N, K); }
extern "C" int gpt2_tune_gemm_pick_q(int M, int N, int K, int int8) { return pick_cfg(M, N, K, int8 != 0); }
extern "C" int gpt2_tune_gemm_fits(int cfg, int K) { return cfg >= 0 && cfg < kNumCfgs && cfg_fits(cfg, K); }
// Force one config for every later GEMM whose K it accepts (-1 restores the table).
extern "C" void gpt2_tune_gemm_force(int cfg) { g_force_cfg = (cfg >= 0 && cfg < kNumCfgs) ? cfg : -1; }
extern "C" void gpt2_tune_gemm_run(int cfg, gpt2_half *C, const gpt2_half *A, const void *W, const float *Ws,
                                   const gpt2_half *bias, int M, int N, int K) {
    if (gemm_args("gpt2_tune_gemm_run", C, A, W, M, N, K)) return;
    gemm(C, A, W, Ws, bias, M, N, K, Ws != nullptr, cfg);
}
// The prefill's fused-epilogue GEMMs (epi 1: gelu_new, 2: + resid, which may be C itself), for
// tests: returns 1 when a fused kernel ran, 0 when none covers the call (the prefill then runs the
// plain GEMM and the separate elementwise kernel).
extern "C" int gpt2_tune_gemm_fused(gpt2_half *C, const gpt2_half *A, const void *W, const float *Ws,
                                    const gpt2_half *bias, int M, int N, int K, int epi, const gpt2_half *resid) {
    if (gemm_args("gpt2_tune_gemm_fused", C, A, W, M, N, K)) return 0;
    return gemm_fused(C, A, W, Ws, bias, M, N, K, Ws != nullptr, epi, resid) ? 1 : 0;
}
// The LayerNorm-panel GEMMs: C = LayerNorm(X; g, b) . W^T (+ bias), gelu after for epi 1; cfg -1
// takes the forced config.  Returns 1 when a kernel ran, 0 when none covers the call.
extern "C" int gpt2_tune_gemm_ln_count(void) { return kNumLnCfgs; }
extern "C" const char *gpt2_tune_gemm_ln_name(int cfg) { return cfg >= 0 && cfg < kNumLnCfgs ? kLnCfgs[cfg].name : "?"; }
// Force one LayerNorm-panel config for the prefill's QKV and fc GEMMs (-1: off, the default).
extern "C" void gpt2_tune_gemm_ln_force(int cfg) { g_ln_cfg = (cfg >= 0 && cfg < kNumLnCfgs) ? cfg : -1; }
extern "C" int gpt2_tune_gemm_ln(int cfg, gpt2_half *C, const gpt2_half *X, const gpt2_half *g, const gpt2_half *b,
                                 const void *W, const float *Ws, const gpt2_half *bias, int M, int N, int K, int epi) {
    if (gemm_args("gpt2_tune_gemm_ln", C, X, W, M, N, K)) return 0;
    return gemm_ln(C, X, g, b, W, Ws, bias, M, N, K, Ws != nullptr, epi, cfg) ? 1 : 0;
}
