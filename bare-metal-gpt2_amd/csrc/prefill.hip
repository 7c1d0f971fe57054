// prefill.hip -- the prefill's 12-layer trunk as ONE persistent kernel (gfx950).
//
// Replaces the per-op launch sequence of the prefill forward (cuda/forward_cuda.cu:77-116: per layer
// LayerNorm, QKV matmul, attention, attn-proj + residual, LayerNorm, fc + gelu, mlp-proj +
// residual) for this library's backends.  Why: on MI355X each launch of a prefill-sized op costs
// ~1.1 us of dispatch gap, ~1 us until its first tile has landed and ~1 us of epilogue drain; at
// P=512 those fixed costs are about half of every GEMM launch (a trunk GEMM's k-loop is 2-5 us).  In
// one kernel the next tile's loads are in flight while the last one finishes, on the same CU.
//
// Design:
//   * The work is a list of tasks in dependency order (host-built, uploaded once per T): per row
//     block of 32 tokens, embedding; per layer, GEMM tiles of 32 rows x 64 (or 32) columns for QKV,
//     attn-proj, fc and mlp-proj, and attention blocks of 16 queries of one head.  Work-groups (two
//     per CU, four waves each) take tasks from an atomic ticket.  A task only waits for tasks with
//     smaller tickets, which are held by running work-groups or done, so the oldest unfinished task
//     can always proceed: no deadlock, whatever the number of resident work-groups.
//   * Dependencies are counters per (layer, stage, row block), bumped once per finished task:
//     QKV(l, rb) needs the 24 mlp-proj tiles of layer l-1 for rb (the embedding for l = 0);
//     attention of a query block needs the QKV tiles of every row block up to its last query
//     (causal); attn-proj(rb) needs the 24 attention blocks of rb; fc(rb) the 12 attn-proj tiles;
//     mlp-proj(rb) the 48 fc tiles.  Early row blocks run ahead into the next layer while later ones
//     are still in attention.
//   * LayerNorm is computed by the GEMM that consumes it: a QKV or fc tile normalizes its 32 rows
//     (whole 768-element rows, fp32 statistics as the LayerNorm kernel) into an fp16 panel in LDS,
//     and only the weight tiles stream through the LDS ring.  Weight tiles do not depend on the
//     activations, so the first ones are requested before the task waits for its inputs.
//   * Visibility across XCDs (each has its own L2): results are stored with device-scope (sc1)
//     stores, which write through to the memory side; a task bumps its counter only after its stores
//     have completed (s_waitcnt vmcnt(0)); consumers poll counters with device-scope loads and then
//     read with ordinary loads.  No buffer is written twice in a launch (each layer has its own
//     buffers in the arena), so no cache can hold a stale copy of a line a consumer reads.
//   * Every poll is bounded; a timeout records an error, and every work-group then leaves.  The last
//     work-group to leave clears the counters and the ticket for the next launch.
//
// Numerics follow the fused multi-launch prefill: fp16 activations between ops, fp32 accumulation,
// LayerNorm with biased variance and eps inside the sqrt, bias (after the INT8 row scale), then gelu
// or the residual add, each rounded to fp16 as separate kernels would.
#include <cstring>
#include <vector>

#include "attn_prefill.h"
#include "common.h"
#include "prefill.h"

namespace g2 {

constexpr int PF_T = 256;                          // threads per work-group
constexpr int PF_RB = 32;                          // rows per row block = GEMM tile rows
constexpr int PF_MAXRB = GPT2_N_CTX / PF_RB;       // 32
constexpr int PF_LDS = 80 * 1024;                  // two work-groups per CU
enum { ST_X = 0, ST_QKV = 1, ST_ATT = 2, ST_MID = 3, ST_H = 4, PF_NST = 5 };
enum { TK_EMB = 0, TK_QKV = 1, TK_ATT = 2, TK_PROJ = 3, TK_FC = 4, TK_MLP = 5 };
constexpr int PF_NCNT = (GPT2_N_LAYER + 1) * PF_NST * PF_MAXRB;
constexpr int PF_SPIN = 1 << 16;                   // default poll rounds before a work-group gives up
constexpr uint32_t PF_NONE = 0xffffffffu;
// Every atomic on a ticket or counter is made by all 64 lanes of wave 0 with the same value 1 (a
// uniform value: the compiler folds it into one atomic of +64, where a per-lane 0/1 value costs a
// 64-step scalar loop), so tickets and counters count in units of PF_ONE.
constexpr uint32_t PF_ONE = 64;

__host__ __device__ constexpr int cidx(int l, int st, int rb) { return (l * PF_NST + st) * PF_MAXRB + rb; }
__host__ __device__ constexpr uint32_t task_word(int type, int l, int a, int b) {
    return (uint32_t)type | ((uint32_t)l << 4) | ((uint32_t)a << 8) | ((uint32_t)b << 16);
}
// tiles per row block of each GEMM (the counters' targets)
constexpr int N_QKV = GPT2_QKV_DIM / 64, N_PROJ = GPT2_N_EMBD / 64, N_FC = GPT2_FFN_DIM / 64, N_MLP = GPT2_N_EMBD / 32;

__device__ __forceinline__ uint32_t ld_dev(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev64(uint16_t *p, uint2 v) {
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// A value every lane of the wave holds alike, as a scalar: branches on it are wave-uniform in the
// compiled code.
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// Wave 0 polls (all its lanes load the same word; every branch is on a scalar copy) until
// *c >= target; false after the poll limit or once another work-group has recorded an error.
__device__ bool pf_poll(const uint32_t *c, uint32_t target, uint32_t *ctl, int spin) {
    for (int round = 0;; ++round) {
        if (uni(ld_dev(c)) >= target) return true;
        if (round >= spin || ((round & 31) == 31 && uni(ld_dev(ctl + 2)))) {
            __hip_atomic_fetch_or(ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // idempotent
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Every wave's stores have completed, then one increment of the task's counter (PF_ONE: every lane
// of wave 0 adds one).
__device__ __forceinline__ void pf_signal(uint32_t *c, bool wave0, uint64_t *tr) {
    if (wave0 && tr) tr[5] = __builtin_amdgcn_s_memrealtime();   // trace: the task's stores are issued
    wait_vm<0>();
    __syncthreads();
    if (wave0 && tr) tr[6] = __builtin_amdgcn_s_memrealtime();   // trace: ... and have completed
    if (wave0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // + PF_ONE
}

// ------------------------------------------------------------------------------------ GEMM tile
// C[m0..m0+31, n0..n0+BN) = epi(A[m0.., 0..K) . W[n0.., 0..K)^T (* s) + b) on 256 threads, with
// v_mfma_f32_16x16x32_f16 in the layout of k_gemm_dl (W rows as the MFMA A operand, activation rows
// as B: each lane holds four consecutive n of one output row).  Waves: WN across the columns, 4/WN
// across the rows.  PANEL: A is LayerNorm(X) of the 32 rows, normalized into an LDS panel before the
// k-loop; otherwise A streams through the ring with W.
template <int BN, bool PANEL, bool QW>
struct TileGeo {
    static constexpr int BM = PF_RB, BK = 64, K = PANEL ? GPT2_N_EMBD : 0;
    static constexpr int WN = BN / 16, WM = 4 / WN, WTM = BM / WM, TM = WTM / 16;
    static constexpr int W_ROWB = QW ? BK : 2 * BK;
    static constexpr int W_BYTES = BN * W_ROWB, A_BYTES = PANEL ? 0 : BM * BK * 2;
    static constexpr int STAGE = A_BYTES + W_BYTES;
    static constexpr int PANEL_BYTES = PANEL ? BM * GPT2_N_EMBD * 2 : 0;
    static constexpr int S = (PF_LDS - PANEL_BYTES) / STAGE > 8 ? 8 : (PF_LDS - PANEL_BYTES) / STAGE;
    static constexpr int A_INS = A_BYTES / 1024, W_INS = W_BYTES / 1024, TOT = A_INS + W_INS;
    static constexpr int LO = TOT / 4, REM = TOT % 4, LMAX = LO + (REM ? 1 : 0);
    static_assert(WN * WM == 4 && TM * 16 == WTM, "four waves of whole 16x16 blocks");
    static_assert(A_BYTES % 1024 == 0 && W_BYTES % 1024 == 0, "1 KB load granules");
    static_assert(S >= 3 && (S - 2) * LMAX < 64, "stages");
    static_assert(PANEL_BYTES + S * STAGE <= PF_LDS, "LDS budget");
};

// LayerNorm of rows m0 .. m0+31 of X (row stride 768) into the LDS panel: wave w normalizes rows
// 8w .. 8w+7 with ln_row768, the LayerNorm kernel's own arithmetic (bit-identical rows).  The panel is 12 k-tile blocks of 32 rows x 128 B, each laid out as a ring stage's
// A tile (16-byte chunk c of row r at (c ^ (r & 7)) * 16).
__device__ __forceinline__ void ln_panel(char *panel, const uint16_t *X, const uint16_t *g, const uint16_t *b, int m0,
                                         int T) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    f16x4 xv[8][3], gg[3], bb[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        gg[i] = *reinterpret_cast<const f16x4 *>(g + 256 * i + 4 * lane);
        bb[i] = *reinterpret_cast<const f16x4 *>(b + 256 * i + 4 * lane);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const uint16_t *xr = X + (size_t)min(m0 + 8 * wave + r, T - 1) * GPT2_N_EMBD;
#pragma unroll
        for (int i = 0; i < 3; ++i) xv[r][i] = *reinterpret_cast<const f16x4 *>(xr + 256 * i + 4 * lane);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        f16x4 o[3];
        ln_row768(xv[r], gg, bb, o);
        const int row = 8 * wave + r;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int kt = 4 * i + (lane >> 4), chunk = (lane & 15) >> 1;
            *reinterpret_cast<f16x4 *>(panel + kt * 4096 + row * 128 + ((chunk ^ (row & 7)) << 4) + (lane & 1) * 8) = o[i];
        }
    }
}

// deps(): the task's dependency wait (thread 0 polls; every thread returns its outcome).
template <int BN, bool PANEL, bool QW, int EPI, class Deps>
__device__ bool pf_gemm(char *lds, Deps deps, const uint16_t *__restrict__ A, int K, const uint16_t *__restrict__ ln_g,
                        const uint16_t *__restrict__ ln_b, const void *__restrict__ Wv, const float *__restrict__ Ws,
                        const uint16_t *__restrict__ bias, const uint16_t *__restrict__ resid, uint16_t *__restrict__ C,
                        int N, int m0, int n0, int T, uint64_t *tr) {
    using G = TileGeo<BN, PANEL, QW>;
    constexpr int S = G::S, BK = G::BK, LMAX = G::LMAX, LO = G::LO, REM = G::REM, TM = G::TM;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn0 = (wave % G::WN) * 16, wm0 = (wave / G::WN) * G::WTM;
    const int nk = K / BK;
    char *panel = lds;
    char *ring = lds + G::PANEL_BYTES;
    const size_t welt = QW ? 1 : 2;

    // this wave's load instructions per stage: global source at k = 0, LDS offset in a stage
    const char *gsrc[LMAX];
    int ldst[LMAX], kstep[LMAX];
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        const int q = wave + 4 * j;
        if (q < G::A_INS) {
            const int row = 8 * q + (lane >> 3), c = (lane & 7) ^ (row & 7);
            gsrc[j] = reinterpret_cast<const char *>(A + (size_t)min(m0 + row, T - 1) * K + c * 8);
            ldst[j] = q * 1024;
            kstep[j] = BK * 2;
        } else {
            const int qw = min(q, G::TOT - 1) - G::A_INS;
            int row, c;
            if constexpr (QW) { row = 16 * qw + (lane >> 2); c = (lane & 3) ^ ((row >> 2) & 3); }
            else { row = 8 * qw + (lane >> 3); c = (lane & 7) ^ (row & 7); }
            gsrc[j] = reinterpret_cast<const char *>(Wv) + (size_t)(n0 + row) * K * welt + c * 16;
            ldst[j] = G::A_BYTES + qw * 1024;
            kstep[j] = BK * (int)welt;
        }
    }
    const int nld = (REM == 0 || wave < REM) ? LMAX : LO;
    auto issue = [&](int kt) {
        char *st = ring + (kt % S) * G::STAGE;
#pragma unroll
        for (int j = 0; j < LMAX; ++j)
            if (j < nld) __builtin_amdgcn_global_load_lds(gsrc[j] + (size_t)kt * kstep[j], G2_LDS(st + ldst[j]), 16, 0, 0);
    };
    auto wait_for = [&](int after) {
        if constexpr (REM == 0) wait_tiles<LO, S - 2>(after);
        else {
            if (wave < REM) wait_tiles<LO + 1, S - 2>(after);
            else wait_tiles<LO, S - 2>(after);
        }
    };

    // epilogue operands that do not depend on the inputs (bias, scales), one fp16 per register
    const int lrow = lane & 15, lgrp = lane >> 4;
    const int nb = n0 + wn0 + 4 * lgrp;
    uint32_t bs_e[4];
    float sc_e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        bs_e[i] = bias[nb + i];
        sc_e[i] = 1.f;
        if constexpr (QW) sc_e[i] = Ws[nb + i];
    }
    // weight tiles (and, streamed, the A tiles) of the first S-1 k-tiles: with a panel they do not
    // depend on the inputs and go out before the wait
    if constexpr (PANEL) {
#pragma unroll
        for (int s = 0; s < S - 1; ++s) issue(s);
    }
    if (!deps()) return false;
    if constexpr (!PANEL) {
#pragma unroll
        for (int s = 0; s < S - 1; ++s) issue(s);
    }
    uint2 rs_e[TM];
#pragma unroll
    for (int b = 0; b < TM; ++b) {
        rs_e[b] = uint2{0u, 0u};
        if constexpr (EPI == EPI_RESID)
            rs_e[b] = *reinterpret_cast<const uint2 *>(resid + (size_t)min(m0 + wm0 + 16 * b + lrow, T - 1) * N + nb);
    }
    if constexpr (PANEL) {
        ln_panel(panel, A, ln_g, ln_b, m0, T);   // waits for every load of this wave (vmcnt 0)
    }

    f32x4 acc[TM];
#pragma unroll
    for (int b = 0; b < TM; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (wave == 0 && tr) tr[3] = __builtin_amdgcn_s_memrealtime();   // trace: k-loop starts
    auto mfma_tile = [&](int kt) {
        const char *st = ring + (kt % S) * G::STAGE;
        const char *ab = PANEL ? panel + kt * 4096 : st;
        const char *wb = st + G::A_BYTES;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int c = ks * 4 + lgrp;
            f16x8 fa[TM];
#pragma unroll
            for (int b = 0; b < TM; ++b) {
                const int r = wm0 + 16 * b + lrow;
                fa[b] = *reinterpret_cast<const f16x8 *>(ab + r * 128 + ((c ^ (r & 7)) << 4));
            }
            const int r = wn0 + lrow;
            f16x8 w;
            if constexpr (QW) {
                const int cq = (ks * 2 + (lgrp >> 1)) ^ ((r >> 2) & 3);
                w = i8x8_to_f16x8(*reinterpret_cast<const uint2 *>(wb + r * 64 + (cq << 4) + ((lgrp & 1) << 3)));
            } else {
                w = *reinterpret_cast<const f16x8 *>(wb + r * 128 + ((c ^ (r & 7)) << 4));
            }
#pragma unroll
            for (int b = 0; b < TM; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, fa[b], acc[b], 0, 0, 0);
        }
    };
    int kt = 0;
    for (; kt + S - 1 < nk; ++kt) {
        wait_for(S - 2);   // tile kt has landed (this wave's part; the barrier: all waves')
        lds_barrier();
        issue(kt + S - 1);
        mfma_tile(kt);
    }
    for (; kt < nk; ++kt) {
        wait_for(nk - 1 - kt);
        lds_barrier();
        mfma_tile(kt);
    }
    if (wave == 0 && tr) tr[4] = __builtin_amdgcn_s_memrealtime();   // trace: k-loop done
    // epilogue: lane holds D[n][m] for n = nb .. nb+3, m = m0 + wm0 + 16 b + lrow
#pragma unroll
    for (int b = 0; b < TM; ++b) {
        const int m = m0 + wm0 + 16 * b + lrow;
        if (m >= T) continue;
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = acc[b][i];
            if constexpr (QW) v = v * sc_e[i];
            const uint32_t rw = i < 2 ? rs_e[b].x : rs_e[b].y;
            o[i] = epi_out<EPI>(v + h2f((uint16_t)bs_e[i]), (uint16_t)(rw >> (16 * (i & 1))));
        }
        st_dev64(C + (size_t)m * N + nb, uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)});
    }
    lds_barrier();   // every wave is done with the ring and the panel before the next task reuses them
    return true;
}

// ------------------------------------------------------------------------------------ the kernel
template <bool Q8>
__global__ __launch_bounds__(PF_T) void k_prefill_persist(const PFArgs a) {
    // 80 KB, so two work-groups share a CU.  The two broadcast words live in its first bytes: they
    // are used only while the LDS is otherwise idle (between tasks, and in a task's dependency wait,
    // before its panel is written or, for streamed tiles and attention, before anything is loaded).
    __shared__ __attribute__((aligned(1024))) char lds[PF_LDS];
    uint32_t &s_task = reinterpret_cast<uint32_t *>(lds)[0];
    uint32_t &s_flag = reinterpret_cast<uint32_t *>(lds)[1];
    // No branch on a path to a barrier may be lane-divergent in the compiled code.  With the ticket
    // fetch, the polls and the counter bumps under `threadIdx.x == 0` (a loop-invariant condition
    // that differs between the lanes of wave 0), the compiler routed the loop's back-edge around
    // them: lanes 1-63 went from a task's end straight back to the barrier before the next task
    // word, re-reading the old word, while thread 0 waited at the inner loop's exit for its own
    // wave's other lanes -- the work-group re-ran its first task forever.  So wave 0 as a whole
    // (a wave-uniform condition) fetches tickets, polls and signals (every lane adding one: units of
    // PF_ONE); the broadcast words are read into scalar registers (uni), which makes the loop, its
    // exits and the task dispatch uniform.
    static_assert(sizeof(AttnLds) <= PF_LDS, "attention LDS fits");
    const int tid = threadIdx.x;
    const bool wave0 = __builtin_amdgcn_readfirstlane(tid >> 6) == 0;
    const int T = a.T, spin = a.spin;
    uint32_t *cnt = a.cnt, *ctl = a.ctl;
    // optional per-task trace, 8 words per ticket (wave 0 writes it; every lane stores the same word,
    // so nothing branches per lane): work-group, then s_memrealtime (100 MHz) when the task word
    // arrived, its inputs were ready, a GEMM's k-loop started and ended, its stores were issued and had
    // completed, and its counter was bumped (0: no such point)
    uint64_t *tr = nullptr;

    for (;;) {
        if (wave0) {
            uint32_t t = PF_NONE;
            if (!uni(ld_dev(ctl + 2))) {
                const uint32_t k = uni(__hip_atomic_fetch_add(ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) / PF_ONE;
                if (k < (uint32_t)a.ntasks) {
                    t = uni(a.tasks[k]);
                    tr = a.trace ? a.trace + 8 * (size_t)k : nullptr;
                }
            }
            s_task = t;   // every lane of wave 0 writes the same word
        }
        __syncthreads();
        const uint32_t tw = uni(s_task);
        __syncthreads();   // s_task is rewritten at the top of the next round
        if (tw == PF_NONE) break;
        if (wave0 && tr) {
            tr[0] = blockIdx.x;
            tr[1] = __builtin_amdgcn_s_memrealtime();
            tr[2] = tr[3] = tr[4] = 0;
        }
        const int type = (int)(tw & 15u), l = (int)((tw >> 4) & 15u), ta = (int)((tw >> 8) & 255u),
                  tb = (int)((tw >> 16) & 255u);
        // one dependency wait: wave 0 polls the counters, every thread gets the outcome
        auto wait_on = [&](auto &&poll_all) {
            if (wave0) {
                s_flag = poll_all() ? 1u : 0u;
                if (tr) tr[2] = __builtin_amdgcn_s_memrealtime();
            }
            __syncthreads();
            const bool ok = uni(s_flag) != 0u;
            __syncthreads();
            return ok;
        };
        bool ok = true;
        if (type == TK_EMB) {
            // x0 rows of row block ta: fp16(wte[id] + wpe[t]); out-of-vocabulary ids embed as wpe alone
            const int rb = ta;
            uint16_t *x0 = a.layers[0].x_in;
            for (int i = tid; i < PF_RB * (GPT2_N_EMBD / 4); i += PF_T) {
                const int t = rb * PF_RB + i / (GPT2_N_EMBD / 4), e = 4 * (i % (GPT2_N_EMBD / 4));
                if (t >= T) break;
                const int id = a.ids[t];
                const f16x4 pe = *reinterpret_cast<const f16x4 *>(a.wpe + (size_t)t * GPT2_N_EMBD + e);
                f16x4 te = {0, 0, 0, 0};
                if ((unsigned)id < (unsigned)GPT2_VOCAB) te = *reinterpret_cast<const f16x4 *>(a.wte + (size_t)id * GPT2_N_EMBD + e);
                uint16_t o[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) o[c] = f2h((float)te[c] + (float)pe[c]);
                st_dev64(x0 + (size_t)t * GPT2_N_EMBD + e, uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16),
                                                                 (uint32_t)o[2] | ((uint32_t)o[3] << 16)});
            }
            pf_signal(cnt + cidx(0, ST_X, rb), wave0, tr);
        } else if (type == TK_ATT) {
            const PFLayer &ly = a.layers[l];
            const int h = ta, q0 = tb * AP_QB;
            const int rlast = (min(q0 + AP_QB, T) - 1) / PF_RB;
            ok = wait_on([&] {
                for (int r = 0; r <= rlast; ++r)
                    if (!pf_poll(cnt + cidx(l, ST_QKV, r), N_QKV * PF_ONE, ctl, spin)) return false;
                return true;
            });
            if (ok) {
                attn_block<true>(*reinterpret_cast<AttnLds *>(lds), ly.att, ly.qkv, T, ly.kc, ly.vc, a.maxT, h, q0);
                pf_signal(cnt + cidx(l, ST_ATT, q0 / PF_RB), wave0, tr);
            }
        } else {
            const PFLayer &ly = a.layers[l];
            const int rb = ta, m0 = rb * PF_RB;
            if (type == TK_QKV) {
                const uint32_t need = (l == 0 ? 1u : (uint32_t)N_MLP) * PF_ONE;
                ok = pf_gemm<64, true, Q8, EPI_NONE>(
                    lds, [&] { return wait_on([&] { return pf_poll(cnt + cidx(l, ST_X, rb), need, ctl, spin); }); },
                    ly.x_in, GPT2_N_EMBD, ly.ln1_g, ly.ln1_b, ly.w[0], ly.s[0], ly.b[0], nullptr, ly.qkv, GPT2_QKV_DIM, m0,
                    64 * tb, T, tr);
                if (ok) pf_signal(cnt + cidx(l, ST_QKV, rb), wave0, tr);
            } else if (type == TK_PROJ) {
                const int nqb = (min(m0 + PF_RB, T) - m0 + AP_QB - 1) / AP_QB;
                ok = pf_gemm<64, false, Q8, EPI_RESID>(
                    lds,
                    [&] { return wait_on([&] { return pf_poll(cnt + cidx(l, ST_ATT, rb), (uint32_t)(GPT2_N_HEAD * nqb) * PF_ONE, ctl, spin); }); },
                    ly.att, GPT2_N_EMBD, nullptr, nullptr, ly.w[1], ly.s[1], ly.b[1], ly.x_in, ly.mid, GPT2_N_EMBD, m0,
                    64 * tb, T, tr);
                if (ok) pf_signal(cnt + cidx(l, ST_MID, rb), wave0, tr);
            } else if (type == TK_FC) {
                ok = pf_gemm<64, true, Q8, EPI_GELU>(
                    lds, [&] { return wait_on([&] { return pf_poll(cnt + cidx(l, ST_MID, rb), N_PROJ * PF_ONE, ctl, spin); }); },
                    ly.mid, GPT2_N_EMBD, ly.ln2_g, ly.ln2_b, ly.w[2], ly.s[2], ly.b[2], nullptr, ly.h, GPT2_FFN_DIM, m0,
                    64 * tb, T, tr);
                if (ok) pf_signal(cnt + cidx(l, ST_H, rb), wave0, tr);
            } else {   // TK_MLP
                ok = pf_gemm<32, false, Q8, EPI_RESID>(
                    lds, [&] { return wait_on([&] { return pf_poll(cnt + cidx(l, ST_H, rb), N_FC * PF_ONE, ctl, spin); }); },
                    ly.h, GPT2_FFN_DIM, nullptr, nullptr, ly.w[3], ly.s[3], ly.b[3], ly.mid, ly.x_out, GPT2_N_EMBD, m0,
                    32 * tb, T, tr);
                if (ok) pf_signal(cnt + cidx(l + 1, ST_X, rb), wave0, tr);
            }
        }
        if (wave0 && tr) tr[7] = __builtin_amdgcn_s_memrealtime();
        if (!ok) break;   // uniform: every thread saw the same wait outcome
    }
    // The last work-group to leave clears the counters and the ticket for the next launch.
    __syncthreads();
    if (wave0) s_flag = uni(__hip_atomic_fetch_add(ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) / PF_ONE;
    __syncthreads();
    if (uni(s_flag) == gridDim.x - 1) {
        for (int i = tid; i < PF_NCNT; i += PF_T) __hip_atomic_store(cnt + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wait_vm<0>();
        __syncthreads();
        if (wave0) {
            // an error of this launch moves to the sticky status word (read by gpt2_prefill_status);
            // every lane of wave 0 performs the same stores (and an idempotent OR)
            const uint32_t e = uni(ld_dev(ctl + 2));
            if (e) __hip_atomic_fetch_or(ctl + 3, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ------------------------------------------------------------------------------ host side
namespace {
// Off by default: correct (the launch sequence's results within the fp16 gates, deterministic), but
// slower than the multi-launch prefill it replaces (P=512 INT8: 1.74 against 0.65 ms).
constexpr bool PF_DEFAULT = false;
bool g_enabled = PF_DEFAULT;
int g_spin = PF_SPIN;
uint64_t *g_trace = nullptr;   // per-task trace buffer (test/tuning hook) and its capacity in tasks
int g_trace_cap = 0;

// One arena per process, on the device of the last launch: its counters, ticket and activation
// buffers serve one launch at a time, so a launch on another stream waits its turn (prefill_persist
// falls back to the launch sequence while the previous stream's launch may still run).
struct Arena {
    int dev = -1, maxT = 0;
    uint16_t *act = nullptr;     // all layer buffers
    uint32_t *cnt = nullptr;     // PF_NCNT counters + 4 control words
    uint32_t *tasks = nullptr;   // task list for taskT
    int taskT = 0, ntasks = 0, cap_tasks = 0;
    int grid = 0;
    bool fits = false;
    hipStream_t last_stream = nullptr;   // the stream of the last launch
    bool unchecked = false;              // launched since the sticky error word was last read
};
Arena g_arena;

// Frees the arena's buffers on their own device (made current for the frees, then restored).
void arena_release(Arena &A) {
    if (A.dev < 0) return;
    int cur = 0;
    const bool have = hipGetDevice(&cur) == hipSuccess;
    if (have && cur != A.dev) (void)hipSetDevice(A.dev);
    gpt2_dfree(A.act);
    gpt2_dfree(A.cnt);
    gpt2_dfree(A.tasks);
    if (have && cur != A.dev) (void)hipSetDevice(cur);
    A = Arena();
}

// Task list in dependency order: embedding per row block, then per layer QKV tiles, attention
// blocks (lightest first: their inputs are ready first), attn-proj, fc and mlp-proj tiles, each by
// row block then column tile.
std::vector<uint32_t> build_tasks(int T) {
    std::vector<uint32_t> t;
    const int nrb = (T + PF_RB - 1) / PF_RB, nqb = (T + AP_QB - 1) / AP_QB;
    for (int rb = 0; rb < nrb; ++rb) t.push_back(task_word(TK_EMB, 0, rb, 0));
    for (int l = 0; l < GPT2_N_LAYER; ++l) {
        for (int rb = 0; rb < nrb; ++rb)
            for (int n = 0; n < N_QKV; ++n) t.push_back(task_word(TK_QKV, l, rb, n));
        for (int qb = 0; qb < nqb; ++qb)
            for (int h = 0; h < GPT2_N_HEAD; ++h) t.push_back(task_word(TK_ATT, l, h, qb));
        for (int rb = 0; rb < nrb; ++rb)
            for (int n = 0; n < N_PROJ; ++n) t.push_back(task_word(TK_PROJ, l, rb, n));
        for (int rb = 0; rb < nrb; ++rb)
            for (int n = 0; n < N_FC; ++n) t.push_back(task_word(TK_FC, l, rb, n));
        for (int rb = 0; rb < nrb; ++rb)
            for (int n = 0; n < N_MLP; ++n) t.push_back(task_word(TK_MLP, l, rb, n));
    }
    return t;
}

constexpr size_t ACT_PER_TOKEN = (size_t)(GPT2_N_LAYER + 1) * GPT2_N_EMBD +
                                 (size_t)GPT2_N_LAYER * (GPT2_QKV_DIM + 2 * GPT2_N_EMBD + GPT2_FFN_DIM);

bool arena_ready(int T, bool q8) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    Arena &A = g_arena;
    if (A.dev != dev) {   // a new device: start over (the old buffers belong to another device)
        arena_release(A);
        A.dev = dev;
        int ncu = 0, per = 0, per8 = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_prefill_persist<false>, PF_T, 0) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per8, k_prefill_persist<true>, PF_T, 0) != hipSuccess)
            return false;
        const int p = per < per8 ? per : per8;
        A.fits = p >= 1;
        A.grid = ncu * (p < 2 ? p : 2);
        A.cnt = (uint32_t *)gpt2_dmalloc((PF_NCNT + 4) * sizeof(uint32_t));
        if (!A.cnt || gpt2_memset(A.cnt, 0, (PF_NCNT + 4) * sizeof(uint32_t))) return false;
    }
    (void)q8;
    if (!A.fits || !A.cnt) return false;
    if (T > A.maxT) {
        gpt2_dfree(A.act);
        A.act = (uint16_t *)gpt2_dmalloc(ACT_PER_TOKEN * 2 * (size_t)T);
        A.maxT = A.act ? T : 0;
        if (!A.act) return false;
    }
    if (T != A.taskT) {
        const std::vector<uint32_t> t = build_tasks(T);
        if ((int)t.size() > A.cap_tasks) {
            gpt2_dfree(A.tasks);
            A.tasks = (uint32_t *)gpt2_dmalloc(t.size() * sizeof(uint32_t));
            A.cap_tasks = A.tasks ? (int)t.size() : 0;
            if (!A.tasks) return false;
        }
        if (gpt2_h2d(A.tasks, t.data(), t.size() * sizeof(uint32_t))) return false;
        A.taskT = T;
        A.ntasks = (int)t.size();
    }
    return true;
}
}  // namespace

void prefill_persist_enable(int on) { g_enabled = on < 0 ? PF_DEFAULT : on != 0; }
bool prefill_persist_enabled() { return g_enabled; }

const uint16_t *prefill_persist(const GPT2Backend *be, const GPT2WeightsGPU *w, const int *d_ids, int T,
                                GPT2KVCache *kv, const uint16_t **embed_out, const uint16_t **layer_out) {
    if (!g_enabled || T < 1 || T > GPT2_N_CTX) return nullptr;
    if (be->matmul != gpt2_matmul_tiled || be->attention != gpt2_attention_flash || be->embed != gpt2_embed ||
        be->layernorm != gpt2_layernorm || be->gelu != gpt2_gelu || be->add != gpt2_add)
        return nullptr;
    const bool q_ok = be->matmul_q == gpt2_matmul_int8;
    const GPT2QWeightsGPU *qw = w->q;
    // one kernel instance per weight kind: every layer matrix INT8 (and the backend takes it), or
    // every one fp16
    int nq = 0;
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        const GPT2QLayerGPU *ql = qw ? &qw->layers[L] : nullptr;
        nq += ql && ql->qkv_w.q && ql->attn_proj_w.q && ql->fc_w.q && ql->proj_w.q;
    }
    const bool q8 = q_ok && nq == GPT2_N_LAYER;
    if (q_ok && nq != 0 && nq != GPT2_N_LAYER) return nullptr;
    Arena &A = g_arena;
    // one launch at a time: on another stream, only once the previous stream has drained
    if (A.last_stream && A.last_stream != stream() && hipStreamQuery(A.last_stream) != hipSuccess) {
        (void)hipGetLastError();   // hipErrorNotReady is not an error of the caller's
        return nullptr;
    }
    // fall back quietly to the multi-launch prefill when the arena cannot be set up; an error the
    // caller has not read yet stays recorded
    const int pending = gpt2_last_error();
    const bool ready = arena_ready(T, q8);
    (void)gpt2_last_error();
    if (pending) set_error(pending, "an earlier call (recorded before the persistent prefill's set-up)");
    if (!ready) return nullptr;
    PFArgs a;
    memset(&a, 0, sizeof(a));
    const size_t t = (size_t)T, E = GPT2_N_EMBD;
    uint16_t *p = A.act;
    uint16_t *x = p;
    p += t * E * (GPT2_N_LAYER + 1);
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        const GPT2LayerGPU &g = w->layers[L];
        PFLayer &y = a.layers[L];
        y.ln1_g = g.ln1_g;
        y.ln1_b = g.ln1_b;
        y.ln2_g = g.ln2_g;
        y.ln2_b = g.ln2_b;
        const gpt2_half *wh[4] = {g.qkv_w, g.attn_proj_w, g.fc_w, g.proj_w};
        const gpt2_half *bh[4] = {g.qkv_b, g.attn_proj_b, g.fc_b, g.proj_b};
        const GPT2QLayerGPU *ql = q8 ? &qw->layers[L] : nullptr;
        const GPT2QW *wq[4] = {ql ? &ql->qkv_w : nullptr, ql ? &ql->attn_proj_w : nullptr, ql ? &ql->fc_w : nullptr,
                               ql ? &ql->proj_w : nullptr};
        for (int i = 0; i < 4; ++i) {
            if (!bh[i]) return nullptr;   // the tiles load every bias unconditionally
            y.w[i] = wq[i] ? (const void *)wq[i]->q : (const void *)wh[i];
            y.s[i] = wq[i] ? wq[i]->s : nullptr;
            y.b[i] = bh[i];
        }
        y.x_in = x + t * E * L;
        y.x_out = x + t * E * (L + 1);
        y.qkv = p;
        p += t * GPT2_QKV_DIM;
        y.att = p;
        p += t * E;
        y.mid = p;
        p += t * E;
        y.h = p;
        p += t * GPT2_FFN_DIM;
        const bool fill = kv && kv->data && L < kv->nLayer && T <= kv->maxT;
        y.kc = fill ? gpt2_kv_K(kv, L) : nullptr;
        y.vc = fill ? gpt2_kv_V(kv, L) : nullptr;
        if (layer_out) layer_out[L] = y.x_out;
    }
    a.wte = w->wte;
    a.wpe = w->wpe;
    a.ids = d_ids;
    a.tasks = A.tasks;
    a.cnt = A.cnt;
    a.ctl = A.cnt + PF_NCNT;
    a.T = T;
    a.maxT = kv && kv->data ? kv->maxT : T;
    a.ntasks = A.ntasks;
    a.spin = g_spin;
    a.trace = (g_trace && g_trace_cap >= A.ntasks) ? g_trace : nullptr;
    if (q8) hipLaunchKernelGGL(k_prefill_persist<true>, dim3(A.grid), dim3(PF_T), 0, stream(), a);
    else hipLaunchKernelGGL(k_prefill_persist<false>, dim3(A.grid), dim3(PF_T), 0, stream(), a);
    check_launch("k_prefill_persist");
    A.last_stream = stream();
    A.unchecked = true;
    if (embed_out) *embed_out = x;
    return x + t * E * GPT2_N_LAYER;
}

}  // namespace g2

// Test / tuning hooks (not part of the reference interface).
// 1 makes every later prefill of this library's backends run the persistent kernel, 0 the
// multi-launch sequence, -1 the default (the multi-launch sequence).
extern "C" void gpt2_tune_prefill_persistent(int on) { g2::prefill_persist_enable(on); }
// Poll rounds before a persistent-prefill work-group gives up, for later launches (< 0: default;
// 0 gives up at the first poll that finds a counter short -- forces the error path with every
// kernel still exiting normally).
extern "C" void gpt2_tune_prefill_spin(int rounds) { g2::g_spin = rounds >= 0 ? rounds : g2::PF_SPIN; }
// Per-task trace of later launches into buf (device memory, 8 x uint64 per task: work-group, then
// s_memrealtime at the task's start, inputs ready, GEMM k-loop start and end, stores issued, stores
// complete, counter bumped; 0 where a task has no such point); a launch with more tasks than cap is
// not traced.  buf = nullptr stops tracing.  Returns the task count of
// a T-token prefill.
extern "C" int gpt2_tune_prefill_trace(unsigned long long *buf, int cap, int T) {
    g2::g_trace = reinterpret_cast<uint64_t *>(buf);
    g2::g_trace_cap = buf ? cap : 0;
    return T >= 1 && T <= GPT2_N_CTX ? (int)g2::build_tasks(T).size() : 0;
}
// Synchronizes and returns (then clears) the persistent prefill's sticky error word: nonzero when a
// launch since the last call gave up waiting (its results are void).  gpt2_sync makes the same check
// and records the error (gpt2_last_error) when the word is set.
extern "C" int gpt2_prefill_status(void) {
    if (!g2::g_arena.cnt) return 0;
    uint32_t e = 0;
    hipStream_t s = g2::g_arena.last_stream ? g2::g_arena.last_stream : g2::stream();
    if (hipStreamSynchronize(s) != hipSuccess) return -1;
    if (hipMemcpy(&e, g2::g_arena.cnt + g2::PF_NCNT + 3, sizeof(e), hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (e) {
        const uint32_t z = 0;
        hipMemcpy(g2::g_arena.cnt + g2::PF_NCNT + 3, &z, sizeof(z), hipMemcpyHostToDevice);
    }
    g2::g_arena.unchecked = false;
    return (int)e;
}

int g2::prefill_persist_take_error() {
    if (!g_arena.unchecked || !g_arena.cnt) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev != g_arena.dev) return 0;
    return gpt2_prefill_status() > 0;
}
