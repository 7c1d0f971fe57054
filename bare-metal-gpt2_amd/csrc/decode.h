// decode.h -- host interface of the persistent decode step (decode.hip), used by engine.hip.
#pragma once

#include "common.h"

namespace g2 {

// Per-layer weights as the step reads them: matrix i in {qkv, attn_proj, fc, proj} is int8 codes
// with per-row scales when s[i] != nullptr, else fp16.
struct PDLayer {
    const uint16_t *ln1_g, *ln1_b, *ln2_g, *ln2_b;
    const void *w[4];
    const float *s[4];
    const uint16_t *b[4];
};

// Passed by value as the kernel argument (~1.7 KB): the per-layer pointers are then read with
// scalar loads from the argument segment, which never wait behind the step's in-flight vector loads.
struct PDArgs {
    PDLayer layers[GPT2_N_LAYER];
    const uint16_t *wte, *wpe, *lnf_g, *lnf_b;
    const void *head_w;               // tied head: fp16 wte, or int8 codes when head_s != nullptr
    const float *head_s;
    uint16_t *kv;                     // [L][K|V][H][maxT][D]
    int maxT;
    uint16_t *logits;                 // [V] fp16
    int *state;                       // {token, pos, epoch, err, spin}
    int *tokens;                      // tokens[pos+1] = next
    uint64_t *ll;                     // exchange arena, LL_WORDS words
    int *err;                         // nonzero after a poll timed out
    unsigned long long *trace;        // optional: [G][128] phase times (100 MHz clock)
    unsigned hold[3];                 // poll hold-offs (10 ns ticks): attention words, x, gelu(fc)
};

struct PDPlan {
    PDArgs args;
    bool q8;                          // int8 layer matrices (else fp16)
};

// Builds the step's argument block; false when the backend or weights need the multi-kernel step.
bool persist_plan(PDPlan &p, const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv, uint16_t *logits,
                  int *state, int *tokens, uint64_t *ll, int *err);
void persist_launch(const PDPlan &p, hipStream_t s);
size_t persist_ll_bytes();
int persist_spin();   // poll rounds before a work-group gives up (state[4] of new graphs and of each set)

}  // namespace g2
