// prefill.h -- host interface of the persistent prefill (prefill.hip), used by engine.hip.
#pragma once

#include "common.h"

namespace g2 {

// Per-layer weights and the layer's activation buffers in the persistent prefill's arena.  Every
// layer has buffers of its own (nothing is rewritten within a launch), so a work-group never finds
// a stale copy of a line in its caches.
struct PFLayer {
    const uint16_t *ln1_g, *ln1_b, *ln2_g, *ln2_b;
    const void *w[4];        // qkv, attn_proj, fc, proj: int8 codes when s[i] != nullptr, else fp16
    const float *s[4];
    const uint16_t *b[4];
    uint16_t *x_in;          // [T,768] residual stream entering the layer
    uint16_t *qkv;           // [T,2304]
    uint16_t *att;           // [T,768]
    uint16_t *mid;           // [T,768] after attn-proj + residual
    uint16_t *h;             // [T,3072] gelu(fc)
    uint16_t *x_out;         // [T,768] after mlp-proj + residual (the next layer's x_in)
    uint16_t *kc, *vc;       // the layer's K and V cache planes ([H][maxT][D]) or nullptr
};

// Passed by value (~2.4 KB of kernel arguments): per-layer pointers are read with scalar loads.
struct PFArgs {
    PFLayer layers[GPT2_N_LAYER];
    const uint16_t *wte, *wpe;
    const int *ids;
    const uint32_t *tasks;   // the task list in dependency order
    uint32_t *cnt;           // completion counters [layer 0..12][stage][row block]
    uint32_t *ctl;           // {ticket, work-groups done, error of this launch, sticky error status}
    int T, maxT, ntasks;
    int spin;                // poll rounds before a work-group gives up
    uint64_t *trace;         // optional: 8 words per ticket (work-group and 7 timestamps)
};

// Runs the 12-layer trunk of a T-token prefill as one kernel: embedding, then per layer LN1 + QKV,
// causal attention (+ the K/V cache fill when kc/vc are set), attn-proj + residual, LN2 + fc + gelu,
// mlp-proj + residual.  Returns the final residual stream [T,768] (nullptr when this path does not
// apply: other backends, mixed fp16/INT8 layers); *layer_out[l] receives each layer's output
// buffer (for captures).  Asynchronous on stream().
const uint16_t *prefill_persist(const GPT2Backend *be, const GPT2WeightsGPU *w, const int *d_ids, int T,
                                GPT2KVCache *kv, const uint16_t **embed_out, const uint16_t **layer_out);

// Test/tuning hooks: on/off switch (1 on, 0 off, -1 the default: off) and the poll limit of later
// launches.
void prefill_persist_enable(int on);
bool prefill_persist_enabled();

}  // namespace g2
