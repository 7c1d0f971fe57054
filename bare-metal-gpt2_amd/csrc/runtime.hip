// runtime.hip -- stream selection, error recording, device-memory helpers and the fp32->fp16
// conversion kernel.  Replaces cuda/common.cuh:17-66 (CUDA_CHECK / dmalloc / h2d / d2h), reshaped
// into C-ABI calls that report errors instead of exiting.
#include <atomic>
#include <cstdio>
#include <cstring>

#include "common.h"

namespace g2 {

static hipStream_t g_stream = nullptr;
static std::atomic<int> g_err{0};
static char g_err_what[256];

hipStream_t stream() { return g_stream; }

void set_error(int code, const char *what) {
    int expected = 0;
    if (g_err.compare_exchange_strong(expected, code)) {
        snprintf(g_err_what, sizeof g_err_what, "%s", what ? what : "");
    }
}

void check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) set_error((int)e, what);
}

}  // namespace g2

using namespace g2;

// A non-null stream is what graph capture needs, so selecting one also resolves the no-allocation
// forward's static scratch address for the current device (outside any capture that follows).
extern "C" void gpt2_set_stream(void *s) {
    g_stream = (hipStream_t)s;
    if (s) noalloc_prepare();
}
extern "C" void *gpt2_get_stream(void) { return (void *)g_stream; }

extern "C" int gpt2_last_error(void) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) set_error((int)e, "hipGetLastError");
    return g_err.exchange(0);
}

extern "C" const char *gpt2_error_string(int code) {
    static thread_local char buf[384];
    if (code == 0) return "no error";
    const char *kind = code == E_ARG      ? "invalid argument"
                       : code == E_ALIGN  ? "misaligned pointer"
                       : code == E_FORMAT ? "bad file format"
                       : code == E_CAPACITY ? "capacity exceeded"
                       : code == E_STATE  ? "invalid state"
                       : hipGetErrorString((hipError_t)code);
    snprintf(buf, sizeof buf, "%s (%s)", kind, g_err_what);
    return buf;
}

// Every device allocation of the library goes through gpt2_dmalloc; the count is a test hook
// (gpt2_test_dmalloc_calls) for entry points that promise to allocate nothing.
static std::atomic<long> g_dmalloc_calls{0};

extern "C" long gpt2_test_dmalloc_calls(void) { return g_dmalloc_calls.load(); }

// Test hook: free device memory on the current device (hipMemGetInfo), or -1 on failure.
extern "C" long long gpt2_test_mem_free(void) {
    size_t f = 0, t = 0;
    return hipMemGetInfo(&f, &t) == hipSuccess ? (long long)f : -1;
}

extern "C" void *gpt2_dmalloc(size_t bytes) {
    g_dmalloc_calls.fetch_add(1);
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        set_error((int)e, "hipMalloc");
        return nullptr;
    }
    return p;
}

extern "C" void gpt2_dfree(void *p) {
    if (p) {
        hipError_t e = hipFree(p);
        if (e != hipSuccess) set_error((int)e, "hipFree");
    }
}

static int copy(void *d, const void *s, size_t n, hipMemcpyKind k, const char *what) {
    if (n == 0) return 0;
    hipError_t e = hipMemcpyAsync(d, s, n, k, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        set_error((int)e, what);
        return (int)e;
    }
    return 0;
}

extern "C" int gpt2_h2d(void *d, const void *s, size_t n) { return copy(d, s, n, hipMemcpyHostToDevice, "h2d"); }
extern "C" int gpt2_d2h(void *d, const void *s, size_t n) { return copy(d, s, n, hipMemcpyDeviceToHost, "d2h"); }
extern "C" int gpt2_d2d(void *d, const void *s, size_t n) {
    if (n == 0) return 0;
    hipError_t e = hipMemcpyAsync(d, s, n, hipMemcpyDeviceToDevice, g_stream);
    if (e != hipSuccess) { set_error((int)e, "d2d"); return (int)e; }
    return 0;
}

extern "C" int gpt2_memset(void *d, int v, size_t n) {
    hipError_t e = hipMemsetAsync(d, v, n, g_stream);
    if (e != hipSuccess) { set_error((int)e, "memset"); return (int)e; }
    return 0;
}

extern "C" int gpt2_sync(void) {
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) { set_error((int)e, "sync"); return (int)e; }
    if (prefill_persist_take_error()) {
        set_error(E_STATE, "persistent prefill gave up waiting on a dependency (its outputs are void)");
        return E_STATE;
    }
    return 0;
}

// fp32 -> fp16 with v_cvt_f16_f32 (IEEE round to nearest even, like __float2half in
// cuda/forward_cuda.cu:36).  Four elements per thread, grid-stride.
__global__ void k_f32_to_f16(uint16_t *__restrict__ dst, const float *__restrict__ src, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = f2h(src[i]);
}

extern "C" void gpt2_f32_to_f16(gpt2_half *dst, const float *src, size_t n) {
    if (n == 0) return;
    if (!dst || !src) { arg_fail("gpt2_f32_to_f16: null pointer"); return; }
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    k_f32_to_f16<<<(unsigned)blocks, 256, 0, g_stream>>>(dst, src, n);
    check_launch("k_f32_to_f16");
}
