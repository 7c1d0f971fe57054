// bench.hip -- native timing loops for bench.py (the role of cuda/common.cuh:27-62 cuda_bench and the
// harness loops in bench/*.cu).  Launch loops run here, not in Python, so the host never throttles
// the GPU; hipEvents are recorded on the stream the kernels are launched on.
#include <algorithm>
#include <vector>

#include "common.h"

extern "C" {

// One timed operation: kind 0 = fp16 GEMM (gpt2_matmul_tiled), 1 = INT8 GEMM (gpt2_matmul_int8),
// 2 = fp16 GEMV (gpt2_gemv_fp16), 3 = INT8 GEMV (gpt2_gemv_int8).
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
        default: gpt2_gemv_int8(o.C, o.A, (const int8_t *)o.W, o.Ws, o.bias, o.N, o.K); break;
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
