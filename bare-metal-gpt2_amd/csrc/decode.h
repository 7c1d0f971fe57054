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

struct PDArgs {
    const PDLayer *layers;            // device array [12]
    const uint16_t *wte, *wpe, *lnf_g, *lnf_b;
    const void *head_w;               // tied head: fp16 wte, or int8 codes when head_s != nullptr
    const float *head_s;
    uint16_t *kv;                     // [L][K|V][H][maxT][D]
    int maxT;
    uint16_t *logits;                 // [V] fp16
    int *state;                       // {token, pos, epoch}
    int *tokens;                      // tokens[pos+1] = next
    uint64_t *ll;                     // exchange arena, LL_WORDS words
    int *err;                         // nonzero after a poll timed out
    int spin;                         // poll rounds before a work-group gives up
    unsigned long long *trace;        // optional: [G][128] phase times (100 MHz clock)
};

struct PDPlan {
    PDArgs args;
    PDLayer *d_layers;
};

// Builds the step's argument block (and uploads the per-layer table); false when the backend or
// weights need the multi-kernel step.
bool persist_plan(PDPlan &p, const GPT2Backend *be, const GPT2WeightsGPU *w, GPT2KVCache *kv, uint16_t *logits,
                  int *state, int *tokens, uint64_t *ll, int *err);
void persist_launch(const PDPlan &p, hipStream_t s);
size_t persist_ll_bytes();
void persist_free(PDPlan &p);

}  // namespace g2
