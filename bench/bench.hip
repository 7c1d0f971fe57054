// bench.hip -- native timing loops for bench.py (the role of cuda/common.cuh:27-62 cuda_bench and the
// harness loops in bench/*.cu).  Launch loops run here, not in Python, so the host never throttles
// the GPU; hipEvents are recorded on the stream the kernels are launched on.
#include <algorithm>
#include <vector>

#include "common.h"

extern "C" {

// Tuning hooks of libgpt2amd.so (csrc/gemm.hip, csrc/gemv.hip): one GEMM on a fixed tile config, the
// fused-epilogue GEMM, the LayerNorm-panel GEMM, one GEMV on a fixed config.  Weak, so this harness also loads against an older build of the
// library that lacks them (bench/ab_build.sh); the ops that need a missing hook record an error.
__attribute__((weak)) void gpt2_tune_gemm_run(int cfg, gpt2_half *C, const gpt2_half *A, const void *W,
                                              const float *Ws, const gpt2_half *bias, int M, int N, int K);
__attribute__((weak)) int gpt2_tune_gemm_fused(gpt2_half *C, const gpt2_half *A, const void *W, const float *Ws,
                                               const gpt2_half *bias, int M, int N, int K, int epi,
                                               const gpt2_half *resid);
__attribute__((weak)) int gpt2_tune_gemm_ln(int cfg, gpt2_half *C, const gpt2_half *X, const gpt2_half *g,
                                            const gpt2_half *b, const void *W, const float *Ws, const gpt2_half *bias,
                                            int M, int N, int K, int epi);
__attribute__((weak)) void gpt2_tune_gemv_run(int cfg, gpt2_half *C, const gpt2_half *A, const void *W,
                                              const float *Ws, const gpt2_half *bias, int N, int K);
static int missing_hook = 0;

// One timed operation: kind 0 = fp16 GEMM (gpt2_matmul_tiled), 1 = INT8 GEMM (gpt2_matmul_int8),
// 2 = fp16 GEMV (gpt2_gemv_fp16), 3 = INT8 GEMV (gpt2_gemv_int8), 4 = causal prefill attention
// (gpt2_attention_flash: C = att, A = qkv, M = T), 5 = LayerNorm (gpt2_layernorm: C = out, A = x,
// W = gamma, bias = beta, M rows of K), 6 = the GEMM with the residual add fused (C = C + A.W^T + b,
// gpt2_tune_gemm_fused epi 2), 7 = residual add (gpt2_add: C += A, M*N elements), 8 = the GEMM with
// gelu fused (gpt2_tune_gemm_fused epi 1), 9 = gelu in place (gpt2_gelu, M*N elements), 16 + c = the GEMM
// on tile config c (gpt2_tune_gemm_run; INT8 weights when Ws is not NULL), for sweeps that mix
// configs in one step, 64 + c = the LayerNorm-panel GEMM on LN config c (gpt2_tune_gemm_ln, K = 768,
// the bias standing in for gamma and beta: a timing form only), 256 + c = the GEMV on config c
// (gpt2_tune_gemv_run; INT8 codes when Ws is not NULL).
typedef struct {
    int kind;
    gpt2_half *C;
    const gpt2_half *A;
    const void *W;
    const float *Ws;
    const gpt2_half *bias;
    int M, N, K;
} GPT2BenchOp;

static void run_op(const GPT2BenchOp &o) {
    switch (o.kind) {
        case 0: gpt2_matmul_tiled(o.C, o.A, (const gpt2_half *)o.W, o.bias, o.M, o.N, o.K); break;
        case 1: gpt2_matmul_int8(o.C, o.A, (const int8_t *)o.W, o.Ws, o.bias, o.M, o.N, o.K); break;
        case 2: gpt2_gemv_fp16(o.C, o.A, (const gpt2_half *)o.W, o.bias, o.N, o.K); break;
        case 4: gpt2_attention_flash(o.C, o.A, o.M, GPT2_N_EMBD, GPT2_N_HEAD, GPT2_HEAD_DIM); break;
        case 3: gpt2_gemv_int8(o.C, o.A, (const int8_t *)o.W, o.Ws, o.bias, o.N, o.K); break;
        case 5: gpt2_layernorm(o.C, o.A, (const gpt2_half *)o.W, o.bias, o.M, o.K); break;
        case 6:
            if (gpt2_tune_gemm_fused) gpt2_tune_gemm_fused(o.C, o.A, o.W, o.Ws, o.bias, o.M, o.N, o.K, g2::EPI_RESID, o.C);
            else missing_hook = 1;
            break;
        case 7: gpt2_add(o.C, o.A, (size_t)o.M * o.N); break;
        case 8:
            if (gpt2_tune_gemm_fused) gpt2_tune_gemm_fused(o.C, o.A, o.W, o.Ws, o.bias, o.M, o.N, o.K, g2::EPI_GELU, nullptr);
            else missing_hook = 1;
            break;
        case 9: gpt2_gelu(o.C, (size_t)o.M * o.N); break;
        default:
            if (o.kind >= 256) {
                if (gpt2_tune_gemv_run) gpt2_tune_gemv_run(o.kind - 256, o.C, o.A, o.W, o.Ws, o.bias, o.N, o.K);
                else missing_hook = 1;
            } else if (o.kind >= 64 && gpt2_tune_gemm_ln)   // LayerNorm-panel GEMM on LN config kind - 64; the bias doubles as gamma and beta
                gpt2_tune_gemm_ln(o.kind - 64, o.C, o.A, o.bias, o.bias, o.W, o.Ws, o.bias, o.M, o.N, o.K, 0);
            else if (o.kind < 64 && gpt2_tune_gemm_run) gpt2_tune_gemm_run(o.kind - 16, o.C, o.A, o.W, o.Ws, o.bias, o.M, o.N, o.K);
            else missing_hook = 1;
            break;
    }
}

// Runs ops[0..n) in order, `warmup` untimed rounds then `iters` timed rounds, and returns the mean
// milliseconds per round in *ms_round.  If ms_per_op is not NULL, each op is then timed alone over
// `iters` back-to-back launches and its mean per launch is stored in ms_per_op[i].
int gpt2_bench_ops(const GPT2BenchOp *ops, int n, int warmup, int iters, float *ms_round, float *ms_per_op) {
    if (!ops || n <= 0 || iters <= 0) return 1;
    hipStream_t s = (hipStream_t)gpt2_get_stream();
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
    for (int w = 0; w < warmup; ++w)
        for (int i = 0; i < n; ++i) run_op(ops[i]);
    hipStreamSynchronize(s);
    hipEventRecord(a, s);
    for (int it = 0; it < iters; ++it)
        for (int i = 0; i < n; ++i) run_op(ops[i]);
    hipEventRecord(b, s);
    hipEventSynchronize(b);
    float ms = 0.f;
    hipEventElapsedTime(&ms, a, b);
    if (ms_round) *ms_round = ms / iters;
    if (ms_per_op) {
        for (int i = 0; i < n; ++i) {
            for (int w = 0; w < 3; ++w) run_op(ops[i]);
            hipStreamSynchronize(s);
            hipEventRecord(a, s);
            for (int it = 0; it < iters; ++it) run_op(ops[i]);
            hipEventRecord(b, s);
            hipEventSynchronize(b);
            hipEventElapsedTime(&ms, a, b);
            ms_per_op[i] = ms / iters;
        }
    }
    hipEventDestroy(a);
    hipEventDestroy(b);
    return gpt2_last_error();
}

// Per-step timing: `warmup` untimed rounds of ops[0..n), then `iters` rounds, each between its own
// pair of events (iters + 1 events recorded on the launch stream, consecutive rounds sharing one), so
// the caller gets every round's time for a median and [min, max], not only their mean.  *ms_total is
// first event to last.
int gpt2_bench_ops_steps(const GPT2BenchOp *ops, int n, int warmup, int iters, float *ms_steps, float *ms_total) {
    if (!ops || n <= 0 || iters <= 0 || !ms_steps) return 1;
    hipStream_t s = (hipStream_t)gpt2_get_stream();
    std::vector<hipEvent_t> ev(iters + 1, nullptr);
    for (auto &e : ev)
        if (hipEventCreate(&e) != hipSuccess) return 1;
    for (int w = 0; w < warmup; ++w)
        for (int i = 0; i < n; ++i) run_op(ops[i]);
    hipStreamSynchronize(s);
    hipEventRecord(ev[0], s);
    for (int it = 0; it < iters; ++it) {
        for (int i = 0; i < n; ++i) run_op(ops[i]);
        hipEventRecord(ev[it + 1], s);
    }
    hipEventSynchronize(ev[iters]);
    for (int it = 0; it < iters; ++it) hipEventElapsedTime(&ms_steps[it], ev[it], ev[it + 1]);
    if (ms_total) hipEventElapsedTime(ms_total, ev[0], ev[iters]);
    for (auto &e : ev) hipEventDestroy(e);
    if (missing_hook) { missing_hook = 0; return 2; }
    return gpt2_last_error();
}

// The same timed rounds as gpt2_bench_ops, but one round of ops[0..n) is captured once into a
// hipGraph on a stream of its own and each round is one replay of it (the launch cost of a prefill
// captured per token count, as a server does for fixed prefill buckets).
int gpt2_bench_ops_graph(const GPT2BenchOp *ops, int n, int warmup, int iters, float *ms_round) {
    if (!ops || n <= 0 || iters <= 0) return 1;
    hipStream_t prev = (hipStream_t)gpt2_get_stream(), s = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e == hipSuccess) {
        gpt2_set_stream(s);
        for (int i = 0; i < n; ++i) run_op(ops[i]);   // first launches outside the capture
        e = hipStreamSynchronize(s);
    }
    if (e == hipSuccess) e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
        for (int i = 0; i < n; ++i) run_op(ops[i]);
        e = hipStreamEndCapture(s, &graph);
    }
    gpt2_set_stream(prev);
    if (e == hipSuccess) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    for (int w = 0; e == hipSuccess && w < warmup; ++w) e = hipGraphLaunch(exec, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess) e = hipEventRecord(a, s);
    for (int it = 0; e == hipSuccess && it < iters; ++it) e = hipGraphLaunch(exec, s);
    if (e == hipSuccess) e = hipEventRecord(b, s);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    if (e == hipSuccess && ms_round) *ms_round = ms / iters;
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    if (exec) hipGraphExecDestroy(exec);
    if (graph) hipGraphDestroy(graph);
    if (s) hipStreamDestroy(s);
    if (e != hipSuccess) return (int)e;
    return gpt2_last_error();
}

// Times `steps` graph replays (one decode token each) with events on the graph's stream.
struct GPT2DecodeGraph;
int gpt2_decode_graph_run(GPT2DecodeGraph *g, int steps);

// Times one call of fn(ctx) enqueued on the library stream.
int gpt2_bench_time(void (*fn)(void *), void *ctx, float *ms) {
    hipStream_t s = (hipStream_t)gpt2_get_stream();
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    hipStreamSynchronize(s);
    hipEventRecord(a, s);
    fn(ctx);
    hipEventRecord(b, s);
    hipEventSynchronize(b);
    hipEventElapsedTime(ms, a, b);
    hipEventDestroy(a);
    hipEventDestroy(b);
    return gpt2_last_error();
}

// Device properties for the report: CU count, clock (kHz) and memory clock/bus width.
int gpt2_device_info(int *cus, int *clock_khz, char *name, int name_len) {
    hipDeviceProp_t p;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) return 1;
    if (cus) *cus = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    if (name && name_len > 0) {
        snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
    }
    return 0;
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------
// Roofline denominators (the role of bench/microbench.cu:51-208 in the reference): the dispatch
// floor of an empty kernel, an HBM read stream, and the fp16 MFMA issue rate.

__global__ void k_empty() {}

// Each thread streams 16-byte vectors with a grid stride, U independent nontemporal loads in
// flight, and folds them into one word so the loads cannot be removed; one word per block is
// written.  (Measured on MI355X over 4 GiB: 6.3-6.6 TB/s for U = 4-8 and 4096-8192 blocks.)
template <int U>
__global__ __launch_bounds__(256) void k_read_stream(const i32x4 *__restrict__ src, size_t n16, int *__restrict__ sink) {
    i32x4 acc = {0, 0, 0, 0};
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        i32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u];
    }
    for (; i < n16; i += stride) acc ^= src[i];
    const int v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (v == 0x7fffffff) sink[blockIdx.x] = v;   // practically never taken; keeps the loads live
}

// fp16 MFMA issue rate with v_mfma_f32_32x32x16_f16, four independent accumulators per wave, one
// wave per SIMD: the instruction that reaches the dense rate on gfx950 (32 cycles per 32 KFLOP per
// wave, measured; v_mfma_f32_16x16x32_f16 reaches ~27 cycles per 16 KFLOP even with 16 accumulators).
__global__ __launch_bounds__(256) void k_mfma_peak(float *__restrict__ out, int iters) {
    f16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (f16)(0.001f * (threadIdx.x + i));
        b[i] = (f16)(0.002f * (threadIdx.x - i));
    }
    f32x16 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) s += acc[j][0];
    if (s == 12345.678f) out[blockIdx.x] = s;
}

extern "C" {

// Mean milliseconds per launch of an empty kernel (grid 1 x 64), back to back.
int gpt2_bench_empty(int iters, float *ms) {
    hipStream_t s = (hipStream_t)gpt2_get_stream();
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    for (int i = 0; i < 10; ++i) hipLaunchKernelGGL(k_empty, dim3(1), dim3(64), 0, s);
    hipStreamSynchronize(s);
    hipEventRecord(a, s);
    for (int i = 0; i < iters; ++i) hipLaunchKernelGGL(k_empty, dim3(1), dim3(64), 0, s);
    hipEventRecord(b, s);
    hipEventSynchronize(b);
    hipEventElapsedTime(ms, a, b);
    *ms /= iters;
    hipEventDestroy(a);
    hipEventDestroy(b);
    return gpt2_last_error();
}

// Read-stream GB/s over `bytes` of device memory (use >> 256 MB so the MALL cannot hold it).
int gpt2_bench_read(const void *buf, size_t bytes, int iters, float *ms) {
    hipStream_t s = (hipStream_t)gpt2_get_stream();
    int *sink = (int *)gpt2_dmalloc(4096 * 4);
    if (!sink) return 1;
    const size_t n16 = bytes / 16;
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    // the faster of two launch shapes (4 loads in flight on 8192 blocks, 8 on 4096)
    float best = 0.f;
    for (int shape = 0; shape < 2; ++shape) {
        auto launch = [&]() {
            if (shape == 0) hipLaunchKernelGGL(k_read_stream<4>, dim3(8192), dim3(256), 0, s, (const i32x4 *)buf, n16, sink);
            else hipLaunchKernelGGL(k_read_stream<8>, dim3(4096), dim3(256), 0, s, (const i32x4 *)buf, n16, sink);
        };
        launch();
        hipStreamSynchronize(s);
        hipEventRecord(a, s);
        for (int i = 0; i < iters; ++i) launch();
        hipEventRecord(b, s);
        hipEventSynchronize(b);
        float t = 0.f;
        hipEventElapsedTime(&t, a, b);
        t /= iters;
        if (shape == 0 || t < best) best = t;
    }
    *ms = best;
    hipEventDestroy(a);
    hipEventDestroy(b);
    gpt2_dfree(sink);
    return gpt2_last_error();
}

// fp16 MFMA issue rate: returns milliseconds for `iters` rounds on `blocks` work-groups of 4 waves;
// FLOP = blocks * 4 waves * iters * 4 * 32*32*16*2.
int gpt2_bench_mfma(int blocks, int iters, float *ms) {
    hipStream_t s = (hipStream_t)gpt2_get_stream();
    float *out = (float *)gpt2_dmalloc(blocks * 4);
    if (!out) return 1;
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    hipLaunchKernelGGL(k_mfma_peak, dim3(blocks), dim3(256), 0, s, out, 16);
    hipStreamSynchronize(s);
    hipEventRecord(a, s);
    hipLaunchKernelGGL(k_mfma_peak, dim3(blocks), dim3(256), 0, s, out, iters);
    hipEventRecord(b, s);
    hipEventSynchronize(b);
    hipEventElapsedTime(ms, a, b);
    hipEventDestroy(a);
    hipEventDestroy(b);
    gpt2_dfree(out);
    return gpt2_last_error();
}

}  // extern "C"

// Plain 16-byte copy of a known size: the calibration point for the FETCH_SIZE / WRITE_SIZE
// counters (HBM bytes per dispatch) used to report a kernel's measured traffic.
__global__ __launch_bounds__(256) void k_copy16(i32x4 *__restrict__ dst, const i32x4 *__restrict__ src, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

extern "C" int gpt2_bench_copy(void *dst, const void *src, size_t bytes, float *ms) {
    hipStream_t s = (hipStream_t)gpt2_get_stream();
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    hipEventRecord(a, s);
    hipLaunchKernelGGL(k_copy16, dim3(4096), dim3(256), 0, s, (i32x4 *)dst, (const i32x4 *)src, bytes / 16);
    hipEventRecord(b, s);
    hipEventSynchronize(b);
    hipEventElapsedTime(ms, a, b);
    hipEventDestroy(a);
    hipEventDestroy(b);
    return gpt2_last_error();
}
