// attn.h -- causal attention helpers shared by the prefill / decode attention kernels and the
// persistent decode step (one wave attends one query over a key range, online softmax).
#pragma once

#include <cmath>

#include "common.h"

namespace g2 {

// One wave attends one query (64 dims) over keys [j0, j1) of one head.  Keys are rows
// `kbase + j*stride`, values `vbase + j*stride` (halves).  Scores: lane = key inside a 64-key chunk,
// each lane reading its own 128-byte key row (64 consecutive rows = contiguous bytes in the cache).
// Context: lane = (key slot l>>3, dim group l&7): eight lanes read one 128-byte value row with
// 16-byte loads, so one load instruction covers 8 keys; every lane accumulates 8 dims over its key
// slot, and the 8 slots are summed once at the end.  Online softmax across chunks (m, l, c[8]).
// Row jcur (if any) is read from kcur / vcur instead of the strided rows: the decode step's own key
// and value, taken straight from its qkv row while the cache copy is being written.
struct AttnState {
    float m, l, c[8];
};

__device__ __forceinline__ void attend_range(const f16x8 (&q)[8], const uint16_t *__restrict__ kbase,
                                             const uint16_t *__restrict__ vbase, long stride, int j0, int j1,
                                             float scale, AttnState &st, int jcur = -1,
                                             const uint16_t *kcur = nullptr, const uint16_t *vcur = nullptr) {
    const int lane = threadIdx.x & 63;
    const int slot = lane >> 3, dg = (lane & 7) * 8;
    for (int jc = j0; jc < j1; jc += 64) {
        const int j = jc + lane;
        float s = -INFINITY;
        if (j < j1) {
            const uint16_t *kr = (j == jcur) ? kcur : kbase + (size_t)j * stride;
            float dot = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const f16x8 kk = *reinterpret_cast<const f16x8 *>(kr + 8 * c);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    dot = __builtin_amdgcn_fdot2(f16x2{q[c][2 * t], q[c][2 * t + 1]}, f16x2{kk[2 * t], kk[2 * t + 1]},
                                                 dot, false);
            }
            s = dot * scale;
        }
        const float mnew = fmaxf(st.m, wave_max(s));   // finite: key jc < j1 is in range
        const float p = (j < j1) ? __expf(s - mnew) : 0.f;
        const float corr = __expf(st.m - mnew);         // st.m = -inf on the first chunk -> 0
        st.l = st.l * corr + wave_sum(p);
        st.m = mnew;
#pragma unroll
        for (int e = 0; e < 8; ++e) st.c[e] *= corr;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int kidx = slot + 8 * t;              // key index inside the chunk
            const float pj = __shfl(p, kidx, 64);
            const int key = jc + kidx;
            if (key < j1) {
                const uint16_t *vr = (key == jcur) ? vcur : vbase + (size_t)key * stride;
                const f16x8 vv = *reinterpret_cast<const f16x8 *>(vr + dg);
#pragma unroll
                for (int e = 0; e < 8; ++e) st.c[e] += pj * (float)vv[e];
            }
        }
    }
}

// Sum the context over the 8 key slots; lanes 0..7 then hold dims 8*lane .. 8*lane+7.
__device__ __forceinline__ void reduce_slots(AttnState &st) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        st.c[e] += __shfl_xor(st.c[e], 8, 64);
        st.c[e] += __shfl_xor(st.c[e], 16, 64);
        st.c[e] += __shfl_xor(st.c[e], 32, 64);
    }
}

__device__ __forceinline__ void load_q(f16x8 (&q)[8], const uint16_t *qp) {
#pragma unroll
    for (int c = 0; c < 8; ++c) q[c] = *reinterpret_cast<const f16x8 *>(qp + 8 * c);
}

__device__ __forceinline__ void init_state(AttnState &st) {
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.c[e] = 0.f;
}

}  // namespace g2
