/* boundary_caller.c -- a plain C caller of libgpt2amd.so through the headers under include/ only, the way the
 * reference's host harnesses call its launchers (bench/ab_forward.cu:185-199 dispatches single
 * matmuls, cuda/forward_cuda.cu:77-116 runs the forward, cuda/kvcache.cu:233-269 the decode step).
 * Test infrastructure: tests/test_gpu_c_caller.py writes a seeded 'GPT2' v1 weight file and the
 * token ids, runs this program, and checks every output file against the CPU oracle.
 *
 *   boundary_caller <weights.bin> <backend> <ids.i32> <T> <n_decode> <out_prefix>
 *
 * Writes (fp16 little-endian unless noted):
 *   <out>.mm        layer 0's QKV matmul of the embedded tokens through gpt2_matmul_dispatch [T,2304]
 *   <out>.logits    gpt2_forward_cuda logits for every row [T,50257]
 *   <out>.decode    logits of n_decode eager greedy steps after gpt2_prefill_fill_cache [n,50257]
 *   <out>.tokens    int32: the prefill's greedy token, the n_decode greedy tokens of the eager steps,
 *                   then those of the graph run from the same cache prefix
 * and prints one line per stage; exits nonzero on any library error.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gpt2_kernels.h"
#include "gpt2_kvcache.h"

static int check(const char *what) {
    int e = gpt2_last_error();
    if (e) {
        fprintf(stderr, "%s: library error %d (%s)\n", what, e, gpt2_error_string(e));
        return 1;
    }
    return 0;
}

static int write_dev(const char *prefix, const char *ext, const void *dptr, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s.%s", prefix, ext);
    void *h = malloc(bytes ? bytes : 1);
    if (!h || gpt2_d2h(h, dptr, bytes)) { free(h); return 1; }
    FILE *f = fopen(path, "wb");
    int bad = !f || fwrite(h, 1, bytes, f) != bytes;
    if (f) bad |= fclose(f) != 0;
    free(h);
    return bad;
}

static float h2f(gpt2_half h) {   /* IEEE fp16 -> fp32 on the host */
    unsigned s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    union { unsigned u; float f; } v;
    if (e == 0) {
        float f = (float)m / 1024.0f / 16384.0f;   /* subnormal: m * 2^-24 */
        return s ? -f : f;
    }
    v.u = (s << 31) | ((e == 31 ? 255u : e + 112u) << 23) | (m << 13);
    return v.f;
}

/* greedy token: the lowest index among the maxima of the fp16 logits (the step's own rule) */
static int argmax16(const gpt2_half *lg, int n) {
    int best = 0;
    float bv = h2f(lg[0]);
    for (int i = 1; i < n; ++i) {
        float v = h2f(lg[i]);
        if (v > bv) { bv = v; best = i; }
    }
    return best;
}

int main(int argc, char **argv) {
    if (argc != 7) {
        fprintf(stderr, "usage: %s <weights.bin> <backend> <ids.i32> <T> <n_decode> <out_prefix>\n", argv[0]);
        return 2;
    }
    const char *wpath = argv[1], *bename = argv[2], *idpath = argv[3], *out = argv[6];
    const int T = atoi(argv[4]), ND = atoi(argv[5]);
    const int V = GPT2_VOCAB, E = GPT2_N_EMBD;
    if (T < 1 || ND < 0 || T + ND > GPT2_N_CTX) { fprintf(stderr, "bad T / n_decode\n"); return 2; }

    int *ids = (int *)malloc((size_t)T * sizeof(int));
    FILE *fi = fopen(idpath, "rb");
    if (!ids || !fi || fread(ids, sizeof(int), (size_t)T, fi) != (size_t)T) { fprintf(stderr, "ids\n"); return 2; }
    fclose(fi);

    /* the reference harness's setup: backend by name, fp32 file -> fp16 device weights, INT8 if the
     * backend has an INT8 slot (here quantized on the device instead of read from a 'GPQ8' file) */
    const GPT2Backend *be = gpt2_backend_by_name(bename);
    GPT2Weights w;
    int rc = gpt2_load_weights(wpath, &w);
    if (rc) { fprintf(stderr, "gpt2_load_weights: %d\n", rc); return 1; }
    GPT2WeightsGPU g;
    gpt2_upload_fp16(&w, &g);
    if (check("gpt2_upload_fp16")) return 1;
    GPT2QWeightsGPU q;
    memset(&q, 0, sizeof q);
    if (be->matmul_q && gpt2_quant_build(&g, &q, NULL)) { check("gpt2_quant_build"); return 1; }
    printf("setup: backend %s, %zu weights, int8 %s\n", be->name, w.n_floats, g.q ? "yes" : "no");

    GPT2ScratchGPU s;
    gpt2_scratch_alloc(&s, GPT2_N_CTX);
    int *d_ids = (int *)gpt2_dmalloc((size_t)GPT2_N_CTX * sizeof(int));
    gpt2_half *d_logits = (gpt2_half *)gpt2_dmalloc((size_t)T * V * sizeof(gpt2_half));
    gpt2_half *d_dec = (gpt2_half *)gpt2_dmalloc((size_t)(ND ? ND : 1) * V * sizeof(gpt2_half));
    int *d_tokens = (int *)gpt2_dmalloc((size_t)GPT2_N_CTX * sizeof(int));
    if (check("alloc") || !d_ids || !d_logits || !d_dec || !d_tokens) return 1;
    gpt2_h2d(d_ids, ids, (size_t)T * sizeof(int));

    /* 1. one matmul through the dispatch rule, as bench/ab_forward.cu does: layer 0's QKV of the
     *    embedded tokens (x = wte[ids] + wpe[pos]) */
    const GPT2QLayerGPU *ql = g.q ? &g.q->layers[0] : NULL;
    be->embed(s.x, g.wte, g.wpe, d_ids, T, E);
    gpt2_matmul_dispatch(be, s.qkv, s.x, g.layers[0].qkv_w, ql ? &ql->qkv_w : NULL, g.layers[0].qkv_b, T,
                         GPT2_QKV_DIM, E);
    gpt2_sync();
    if (check("matmul_dispatch") || write_dev(out, "mm", s.qkv, (size_t)T * GPT2_QKV_DIM * 2)) return 1;
    printf("matmul: [%d x %d] . [%d x %d]^T\n", T, E, GPT2_QKV_DIM, E);

    /* 2. the prefill forward with logits for every row */
    GPT2CapsGPU caps;
    memset(&caps, 0, sizeof caps);
    caps.logits = d_logits;
    caps.logits_all = 1;
    gpt2_forward_cuda(be, &g, d_ids, T, &s, &caps);
    gpt2_sync();
    if (check("gpt2_forward_cuda") || write_dev(out, "logits", d_logits, (size_t)T * V * 2)) return 1;
    printf("forward: T=%d, logits for every row\n", T);

    /* 3. prefill into the KV cache, then greedy eager decode steps */
    GPT2KVCache kv;
    if (gpt2_kv_alloc(&kv, GPT2_N_CTX)) { check("gpt2_kv_alloc"); return 1; }
    caps.logits_all = 0;   /* last row only */
    caps.logits = d_dec;
    gpt2_prefill_fill_cache(be, &g, &kv, d_ids, T, &s, &caps);
    gpt2_sync();
    if (check("gpt2_prefill_fill_cache")) return 1;
    gpt2_half *row = (gpt2_half *)malloc((size_t)V * sizeof(gpt2_half));
    int *toks = (int *)malloc((size_t)(2 * ND + 1) * sizeof(int));
    gpt2_d2h(row, d_dec, (size_t)V * 2);
    const int first = argmax16(row, V);
    int tok = first;
    toks[0] = first;
    for (int i = 0; i < ND; ++i) {
        gpt2_decode_step_cuda(be, &g, &kv, tok, T + i, &s, d_dec + (size_t)i * V, NULL);
        gpt2_d2h(row, d_dec + (size_t)i * V, (size_t)V * 2);
        tok = argmax16(row, V);
        toks[1 + i] = tok;
    }
    gpt2_sync();
    if (check("gpt2_decode_step_cuda") || write_dev(out, "decode", d_dec, (size_t)ND * V * 2)) return 1;
    printf("decode: %d eager steps from position %d (first token %d)\n", ND, T, first);

    /* 4. the same greedy run replayed as a graph from the same cache prefix */
    kv.len = T;   /* the replays rewrite positions T .. T+n_decode-1 */
    GPT2DecodeGraph *dg = gpt2_decode_graph_create(be, &g, &kv, &s, d_dec, d_tokens);
    if (!dg) { check("gpt2_decode_graph_create"); return 1; }
    int pos = 0;
    if (gpt2_decode_graph_set(dg, first, T) || gpt2_decode_graph_run(dg, ND) ||
        gpt2_decode_graph_sync(dg, &tok, &pos)) {
        check("decode graph");
        return 1;
    }
    if (ND > 0) gpt2_d2h(toks + 1 + ND, d_tokens + T + 1, (size_t)ND * sizeof(int));
    printf("graph: mode %d, %d steps, final position %d\n", gpt2_decode_graph_mode(dg), ND, pos);
    gpt2_decode_graph_destroy(dg);
    {
        char path[4096];
        snprintf(path, sizeof path, "%s.tokens", out);
        FILE *f = fopen(path, "wb");
        if (!f || fwrite(toks, sizeof(int), (size_t)2 * ND + 1, f) != (size_t)2 * ND + 1) return 1;
        fclose(f);
    }

    free(row);
    free(toks);
    free(ids);
    gpt2_kv_free(&kv);
    gpt2_dfree(d_tokens);
    gpt2_dfree(d_dec);
    gpt2_dfree(d_logits);
    gpt2_dfree(d_ids);
    gpt2_scratch_free(&s);
    gpt2_quant_free(&q);
    gpt2_free_gpu(&g);
    gpt2_free_weights(&w);
    if (check("teardown")) return 1;
    printf("ok\n");
    return 0;
}
