/* ref_harness.c -- exposes the reference's own CPU forward (cpu/forward_cpu.c, model/weights.c),
 * compiled from the files where they lie under /root/reference, to the parity tests.
 *
 * TEST INFRASTRUCTURE ONLY.  This file contains no reference code: it #includes the reference's
 * forward_cpu.c so that its file-static helpers (matmul, layernorm, gelu_new, attention) can be
 * called directly, and adds thin exported wrappers.  The output goes to oracle/_ref/ (git-ignored).
 */
#include "forward_cpu.c"

#include <stdio.h>

void ref_matmul(float *C, const float *A, const float *W, const float *bias, int M, int N, int K) {
    matmul(C, A, W, bias, M, N, K);
}

void ref_layernorm(float *out, const float *x, const float *g, const float *b, int M) {
    layernorm(out, x, g, b, M);
}

float ref_gelu_new(float x) { return gelu_new(x); }

void ref_attention(float *att, const float *qkv, int T) { attention(att, qkv, T); }

/* Load a 'GPT2' v1 file with the reference loader; returns its error code (0 = ok). The handle
 * owns the body until ref_free_weights. */
int ref_load_weights(const char *path, void **handle) {
    GPT2Weights *w = (GPT2Weights *)calloc(1, sizeof(GPT2Weights));
    int rc = gpt2_load_weights(path, w);
    if (rc != 0) { free(w); *handle = NULL; return rc; }
    *handle = w;
    return 0;
}

void ref_free_weights(void *handle) {
    if (!handle) return;
    gpt2_free_weights((GPT2Weights *)handle);
    free(handle);
}

/* Offsets (in floats, from the start of the body) of every tensor the loader hands out, in the
 * order wte, wpe, 12 x {ln1_g, ln1_b, qkv_w, qkv_b, attn_proj_w, attn_proj_b, ln2_g, ln2_b, fc_w,
 * fc_b, proj_w, proj_b}, lnf_g, lnf_b  (148 entries). */
void ref_weight_offsets(const void *handle, long *off) {
    const GPT2Weights *w = (const GPT2Weights *)handle;
    const float *b = w->data;
    int i = 0;
    off[i++] = w->wte - b;
    off[i++] = w->wpe - b;
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        const GPT2Layer *l = &w->layers[L];
        off[i++] = l->ln1_g - b; off[i++] = l->ln1_b - b;
        off[i++] = l->qkv_w - b; off[i++] = l->qkv_b - b;
        off[i++] = l->attn_proj_w - b; off[i++] = l->attn_proj_b - b;
        off[i++] = l->ln2_g - b; off[i++] = l->ln2_b - b;
        off[i++] = l->fc_w - b; off[i++] = l->fc_b - b;
        off[i++] = l->proj_w - b; off[i++] = l->proj_b - b;
    }
    off[i++] = w->lnf_g - b;
    off[i++] = w->lnf_b - b;
}

/* Forward with weights taken from a loaded handle. */
void ref_forward(const void *handle, const int *ids, int T, float *embed, float *blocks,
                 float *final_ln, float *logits, int logits_all) {
    GPT2Caps caps;
    caps.embed = embed;
    caps.blocks = blocks;
    caps.final_ln = final_ln;
    caps.logits = logits;
    caps.logits_all = logits_all;
    gpt2_forward_cpu((const GPT2Weights *)handle, ids, T, &caps);
}

/* Forward with weights bound onto a caller-owned flat body (same layout as the file body). The
 * binding walks the body with the loader's own offsets, read once from a loaded handle. */
void ref_forward_flat(const float *flat, const long *off, const int *ids, int T, float *embed,
                      float *blocks, float *final_ln, float *logits, int logits_all) {
    GPT2Weights w;
    memset(&w, 0, sizeof w);
    float *b = (float *)flat;
    int i = 0;
    w.data = b;
    w.n_floats = GPT2_TOTAL_PARAMS;
    w.wte = b + off[i++];
    w.wpe = b + off[i++];
    for (int L = 0; L < GPT2_N_LAYER; ++L) {
        GPT2Layer *l = &w.layers[L];
        l->ln1_g = b + off[i++]; l->ln1_b = b + off[i++];
        l->qkv_w = b + off[i++]; l->qkv_b = b + off[i++];
        l->attn_proj_w = b + off[i++]; l->attn_proj_b = b + off[i++];
        l->ln2_g = b + off[i++]; l->ln2_b = b + off[i++];
        l->fc_w = b + off[i++]; l->fc_b = b + off[i++];
        l->proj_w = b + off[i++]; l->proj_b = b + off[i++];
    }
    w.lnf_g = b + off[i++];
    w.lnf_b = b + off[i++];
    ref_forward(&w, ids, T, embed, blocks, final_ln, logits, logits_all);
}
