// attn_prefill.hip -- the causal prefill attention launch (gfx950): one work-group per block of 16
// queries of one head (attn_block in attn_prefill.h).  Replaces the reference's fused attention
// (cuda/kernels_fused.cu:58-140; semantics of cpu/forward_cpu.c:83-116).
//
// Work-groups are assigned XCD-aware (each XCD's L2 serves 1.5 heads), heaviest query blocks first.
#include "attn_prefill.h"

namespace g2 {

__global__ __launch_bounds__(64 * AP_W) void k_attn_prefill_mfma(uint16_t *__restrict__ att,
                                                                  const uint16_t *__restrict__ qkv, int T,
                                                                  uint16_t *__restrict__ Kc, uint16_t *__restrict__ Vc,
                                                                  int maxT) {
    __shared__ AttnLds lds;
    // XCD-aware assignment (work-group b runs on XCD b % 8): XCD x takes every query block of head
    // x and every other block of head 8 + x/2, so its L2 holds the keys and values of 1.5 heads
    // instead of all 12.  Within an XCD the blocks go heaviest first (qi = rank from the last block).
    const int nb = (T + AP_QB - 1) / AP_QB;
    int h, qi;
    {
        const int x = blockIdx.x & 7, k = blockIdx.x >> 3, i3 = k / 3, r3 = k - 3 * i3;
        if (r3 < 2) {
            h = x;
            qi = 2 * i3 + r3;
        } else {
            h = 8 + (x >> 1);
            qi = 2 * i3 + (x & 1);
        }
    }
    if (qi >= nb) return;                      // the grid is rounded up (whole work-group leaves)
    attn_block<false>(lds, att, qkv, T, Kc, Vc, maxT, h, (nb - 1 - qi) * AP_QB);
}

// Kc, Vc (optional): the layer's K and V cache planes ([H][maxT][D]), filled with this prompt's rows
// (the prefill scatter of cuda/kvcache.cu:66-81, done inside the attention launch).
void attention_prefill(uint16_t *att, const uint16_t *qkv, int T, uint16_t *Kc, uint16_t *Vc, int maxT) {
    static_assert(GPT2_N_HEAD == 12, "the XCD assignment covers 12 heads on 8 XCDs");
    hipLaunchKernelGGL(k_attn_prefill_mfma, dim3(8 * 3 * cdiv(cdiv(T, AP_QB), 2)), dim3(64 * AP_W), 0, stream(), att, qkv, T, Kc, Vc,
                       maxT);
    check_launch("k_attn_prefill_mfma");
}

}  // namespace g2
