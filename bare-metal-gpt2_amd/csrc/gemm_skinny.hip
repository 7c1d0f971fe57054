// gemm_skinny.hip -- C = A . W^T (+ bias) for a few rows of A (short prompts), on the MFMA units
// (gfx950).  Same contract as gpt2_matmul_tiled / gpt2_matmul_int8 (cuda/kernels_tiled.cu:24-53,
// cuda/kernels_quant.cu:38-67) for the GPT-2 trunk shapes (K = 768 or 3072, N a multiple of 16).
//
// With M in the tens the product is a weight stream, as the M = 1 GEMV is: W is 0.6-4.7 MB and the
// MFMA work is a fraction of a microsecond.  The tile pipeline (operands staged through an LDS ring,
// one barrier per k-tile, 32-column tiles: 24-96 work-groups for these shapes) spends several round
// trips where one suffices.  Here:
//   * A work-group owns 16 rows of W (one MFMA row block) and 16 rows of A; its four waves split K.
//     Grid = (N / 16) x ceil(M / 16): 48-192 work-groups per 16 rows of A.
//   * Each lane loads its share of its W row straight into registers (16-byte loads, all issued at
//     once: one memory round trip), while the 16 rows of A go to LDS by direct-to-LDS loads (or, with
//     the LayerNorm prologue, are normalized in registers and written there).
//   * One wait, one barrier, then the wave's MFMAs (W as the A operand, the A rows as B), the four
//     waves' sums added in LDS in wave order, and wave 0's epilogue: scale (INT8), bias, then the
//     elementwise op as the unfused sequence would apply it (epi_out).
//   * The LayerNorm prologue (QKV after LN1, fc after LN2) normalizes the block's 16 rows with the
//     LayerNorm kernel's arithmetic (ln_rows768: ln_row768's operations row by row, the rows'
//     reductions interleaved), so the result is bit-identical to the LayerNorm launch followed by
//     this kernel.  Its rows are loaded before the weights and normalized while the weight stream
//     is in flight.
#include "common.h"

namespace g2 {

constexpr int SKN_W = 4;      // waves per work-group: K split four ways
constexpr int SKN_MB = 16;    // rows of A per work-group (the MFMA's B columns)
[[maybe_unused]] constexpr int SKN_TILE = SKN_MB * 128;   // LDS bytes per 64-wide k-tile of the A block

// k offset, inside a wave's share of K, of the 8 values lane group g feeds to MFMA step s.  INT8
// pairs steps 2t and 2t+1 so that one 16-byte load holds both of a lane's slots (k = 64t + 16g + 8h);
// fp16 takes k = 32s + 8g.  A and W use the same map, so every k meets its partner once.
template <bool QW>
__device__ __forceinline__ int skn_k(int s, int g) {
    return QW ? 64 * (s >> 1) + 16 * g + 8 * (s & 1) : 32 * s + 8 * g;
}

template <int K, bool QW, int EPI, bool LNP>
__global__ __launch_bounds__(64 * SKN_W) void k_gemm_skinny(uint16_t *__restrict__ C, const uint16_t *__restrict__ A,
                                                            const void *__restrict__ Wv, const float *__restrict__ Ws,
                                                            const uint16_t *__restrict__ bias, int M, int N, int nbn,
                                                            const uint16_t *resid, const uint16_t *__restrict__ ln_g,
                                                            const uint16_t *__restrict__ ln_b) {
#if defined(__HIP_DEVICE_COMPILE__)   // LDS address-space pointers exist only in the device pass
    constexpr int KT = K / 64;              // 64-wide k-tiles of the A block
    constexpr int KW = K / SKN_W;           // one wave's share of K
    constexpr int NS = KW / 32;             // MFMA steps per wave
    constexpr int NL = QW ? NS / 2 : NS;    // 16-byte W loads per lane
    static_assert(KW % 64 == 0, "a wave's share of K is whole 64-wide tiles");
    static_assert(!LNP || (K == GPT2_N_EMBD && EPI != EPI_RESID), "the LayerNorm prologue: K = 768, no residual");
    static_assert((2 * KT) % SKN_W == 0, "the A block's loads split evenly over the waves");
    // A block [KT][16 rows][128 B] (16-byte chunk c of row r at slot c ^ (r & 7)), then the sums of
    // waves 1..3
    __shared__ __attribute__((aligned(1024))) char lds[KT * SKN_TILE + (SKN_W - 1) * 64 * 16];
    char *const xs = lds;
    f32x4 *const red = reinterpret_cast<f32x4 *>(lds + KT * SKN_TILE);

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lrow = lane & 15, g = lane >> 4;
    const int nb = blockIdx.x % nbn, mb = blockIdx.x / nbn;
    const int n0 = nb * 16, m0 = mb * SKN_MB;
    const int kw0 = wave * KW;

    // Loads, in this order (loads complete in issue order, so a wait for one is a wait for every
    // load issued before it): the LayerNorm prologue's rows and gamma / beta (L2-resident, needed
    // first), this lane's share of W row n0 + lrow (N % 16 == 0: the row exists; all of it in flight
    // at once, from HBM the longest wait), then the epilogue operands.  Compiler barriers keep the
    // order (left to itself the compiler moves the weight loads behind the LayerNorm and the epilogue
    // operands behind the A block's wait).
    f16x4 lg[3], lb[3], lx[4][3];   // LayerNorm prologue: rows wave + 4 r; lane l: elements 256 i + 4 l ..
    if constexpr (LNP) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint16_t *xr = A + (size_t)min(m0 + wave + 4 * r, M - 1) * K;
#pragma unroll
            for (int i = 0; i < 3; ++i) lx[r][i] = *reinterpret_cast<const f16x4 *>(xr + 256 * i + 4 * lane);
        }
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            lg[i] = *reinterpret_cast<const f16x4 *>(ln_g + 256 * i + 4 * lane);
            lb[i] = *reinterpret_cast<const f16x4 *>(ln_b + 256 * i + 4 * lane);
        }
        asm volatile("" ::: "memory");
    }
    i32x4 wl[NL];
    {
        const char *wrow = reinterpret_cast<const char *>(Wv) + (size_t)(n0 + lrow) * K * (QW ? 1 : 2);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int k = kw0 + (QW ? skn_k<true>(2 * i, g) : skn_k<false>(i, g));
            wl[i] = *reinterpret_cast<const i32x4 *>(wrow + (size_t)k * (QW ? 1 : 2));
        }
    }
    // the lane's outputs C[m][nbase .. nbase+3]: scales, bias and residual (rows past M read row M-1
    // and store nothing; the residual may alias C: this lane alone writes those elements)
    const int nbase = n0 + 4 * g, m = m0 + lrow;
    float sc[4];
    uint32_t bs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sc[i] = 1.f;
        if constexpr (QW) sc[i] = Ws[nbase + i];
        bs[i] = *(bias ? bias + nbase + i : A);
    }
    uint2 rs = {0u, 0u};
    if constexpr (EPI == EPI_RESID) rs = *reinterpret_cast<const uint2 *>(resid + (size_t)min(m, M - 1) * N + nbase);
    asm volatile("" ::: "memory");
    if constexpr (LNP) {
        // the LayerNorm's inputs pass through here, so none of its arithmetic is scheduled ahead of
        // the loads above (the compiler would otherwise issue the weight loads after it)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < 3; ++i) asm volatile("" : "+v"(lx[r][i]) : : "memory");
    }

    if constexpr (LNP) {
        // normalized as the LayerNorm kernel does, written where the direct-to-LDS load would have put them
        f16x4 o[4][3];
        ln_rows768<4>(lx, lg, lb, o);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = wave + 4 * r;
#pragma unroll
            for (int i = 0; i < 3; ++i)   // element 256 i + 4 lane: k-tile 4 i + lane / 16, chunk (lane & 15) / 2
                *reinterpret_cast<f16x4 *>(xs + (4 * i + (lane >> 4)) * SKN_TILE + row * 128 +
                                           ((((lane & 15) >> 1) ^ (row & 7)) << 4) + (lane & 1) * 8) = o[r][i];
        }
    } else {
        // load q (two per k-tile) fills rows 8 (q & 1) .. +7 of tile q / 2, lane l slot l & 7 of row
        // 8 (q & 1) + l / 8; wave w issues q = w, w + 4, ...
#pragma unroll
        for (int j = 0; j < 2 * KT / SKN_W; ++j) {
            const int q = wave + SKN_W * j;
            const int r = 8 * (q & 1) + (lane >> 3), c = (lane & 7) ^ (r & 7);
            const uint16_t *src = A + (size_t)min(m0 + r, M - 1) * K + 64 * (q >> 1) + 8 * c;
            __builtin_amdgcn_global_load_lds(src, G2_LDS(xs + q * 1024), 16, 0, 0);
        }
    }
    // the direct-to-LDS A block is complete when this wave's loads have all landed (the LayerNorm
    // path wrote its rows with LDS stores); the barrier then publishes every wave's part
    if constexpr (!LNP) wait_vm<0>();
    lds_barrier();
    // the weights are used from here on (the compiler would otherwise widen INT8 codes inside the
    // LayerNorm prologue, waiting there for the weight stream)
#pragma unroll
    for (int i = 0; i < NL; ++i) asm volatile("" : "+v"(wl[i]));

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        f16x8 w;
        if constexpr (QW) {
            const i32x4 v = wl[s >> 1];
            w = i8x8_to_f16x8((s & 1) ? uint2{(uint32_t)v[2], (uint32_t)v[3]} : uint2{(uint32_t)v[0], (uint32_t)v[1]});
        } else {
            w = __builtin_bit_cast(f16x8, wl[s]);
        }
        const int k = kw0 + skn_k<QW>(s, g), c = (k & 63) >> 3;
        const f16x8 x = *reinterpret_cast<const f16x8 *>(xs + (k >> 6) * SKN_TILE + lrow * 128 + ((c ^ (lrow & 7)) << 4));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, x, acc, 0, 0, 0);
    }
    // lane holds D[n0 + 4g + i][m0 + lrow]; waves 1..3 hand theirs to wave 0, added in wave order
    if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
    lds_barrier();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < SKN_W - 1; ++w) acc += red[w * 64 + lane];
    if (m >= M) return;
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float v = acc[i];
        if constexpr (QW) v = v * sc[i];
        const uint16_t r = (uint16_t)((i < 2 ? rs.x : rs.y) >> (16 * (i & 1)));
        o[i] = epi_out<EPI>(v + (bias ? h2f((uint16_t)bs[i]) : 0.f), r);
    }
    *reinterpret_cast<uint2 *>(C + (size_t)m * N + nbase) =
        uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
#endif
}

typedef void (*SkinnyFn)(uint16_t *, const uint16_t *, const void *, const float *, const uint16_t *, int, int, int,
                         const uint16_t *, const uint16_t *, const uint16_t *);

// [K = 768, 3072][fp16, INT8][epilogue: none, gelu, residual, LayerNorm + none, LayerNorm + gelu]
#define G2_SKN(K, QW) \
    {k_gemm_skinny<K, QW, EPI_NONE, false>, k_gemm_skinny<K, QW, EPI_GELU, false>, k_gemm_skinny<K, QW, EPI_RESID, false>, \
     K == GPT2_N_EMBD ? k_gemm_skinny<GPT2_N_EMBD, QW, EPI_NONE, true> : nullptr,                                       \
     K == GPT2_N_EMBD ? k_gemm_skinny<GPT2_N_EMBD, QW, EPI_GELU, true> : nullptr}
static const SkinnyFn kSkinny[2][2][5] = {{G2_SKN(768, false), G2_SKN(768, true)},
                                          {G2_SKN(3072, false), G2_SKN(3072, true)}};

// Rows of A up to which the skinny kernel takes the trunk shapes.  Measured on MI355X (interleaved
// A/B of the whole prefill against the tile pipeline and the LayerNorm fold): INT8 weights 1.27x at
// T = 8, 1.24x at 16, 1.11x at 24-32, 1.04-1.07x at 40-48, level at 64; fp16 1.12x at 8-16, 1.05-1.07x
// at 24-32, 0.96x at 40 and 0.94x at 64 -- there the fold, which removes the LayerNorm launches,
// beats the skinny kernel's LayerNorm prologue.  gpt2_tune_gemm_skinny overrides both (0: never).
static int g_skinny_max = -1;    // -1: the measured default per weight format
static int g_skinny_calls = 0;   // launches so far (test hook)
int skinny_max_m(bool qw) { return g_skinny_max >= 0 ? g_skinny_max : (qw ? 64 : 32); }

// C = A . W^T (+ bias), then epi (EPI_GELU; EPI_RESID: C = resid + product, resid may be C); with
// ln_g / ln_b, A is first normalized row by row (LayerNorm, K = 768).  Returns false (nothing
// launched) outside its domain: M in [2, skinny_max_m(qw)], K 768 or 3072, N % 16 == 0, 16-byte
// aligned A and W, 8-byte aligned C (and residual, gamma, beta).
bool gemm_skinny(uint16_t *C, const uint16_t *A, const void *W, const float *Ws, const uint16_t *bias, int M, int N,
                 int K, bool qw, int epi, const uint16_t *resid, const uint16_t *ln_g, const uint16_t *ln_b) {
    if (M < 2 || M > skinny_max_m(qw) || N <= 0 || N % 16 || (K != 768 && K != 3072)) return false;
    if (!A || !W || !C || !aligned16(A) || !aligned16(W) || ((uintptr_t)C & 7u) || (qw && !Ws)) return false;
    int e = epi == EPI_NONE ? 0 : epi == EPI_GELU ? 1 : epi == EPI_RESID ? 2 : -1;
    if (e < 0 || (e == 2 && (!resid || ((uintptr_t)resid & 7u)))) return false;
    if (ln_g || ln_b) {
        if (!ln_g || !ln_b || e == 2 || K != GPT2_N_EMBD || (((uintptr_t)ln_g | (uintptr_t)ln_b) & 7u)) return false;
        e += 3;
    }
    const SkinnyFn fn = kSkinny[K == 768 ? 0 : 1][qw ? 1 : 0][e];
    if (!fn) return false;
    const int nbn = N / 16;
    hipLaunchKernelGGL(fn, dim3(nbn * cdiv(M, SKN_MB)), dim3(64 * SKN_W), 0, stream(), C, A, W, Ws, bias, M, N, nbn,
                       resid, ln_g, ln_b);
    check_launch("k_gemm_skinny");
    ++g_skinny_calls;
    return true;
}

}  // namespace g2

// Tuning/test hooks (no reference counterpart): the largest M the skinny kernel takes (0: off, -1:
// the default), the limit in force for fp16 (qw = 0) or INT8 weights, and the number of its
// launches so far.
extern "C" void gpt2_tune_gemm_skinny(int max_m) { g2::g_skinny_max = max_m < 0 ? -1 : max_m; }
extern "C" int gpt2_tune_gemm_skinny_max(int qw) { return g2::skinny_max_m(qw != 0); }
extern "C" int gpt2_tune_gemm_skinny_calls(void) { return g2::g_skinny_calls; }
