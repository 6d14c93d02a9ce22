// bench_loop.cpp -- libvk_bench.so: the harness timing loops behind a C ABI
// (include/vk_bench.h).  Reference loop: results/ralph_loop_fable/src/
// main.cpp:52-62.
#include <hip/hip_runtime.h>

#include "vk_bench.h"

namespace {
struct Events {
    hipEvent_t a = nullptr, b = nullptr;
    bool ok = false;
    Events() { ok = hipEventCreate(&a) == hipSuccess && hipEventCreate(&b) == hipSuccess; }
    ~Events() {
        if (a) (void)hipEventDestroy(a);
        if (b) (void)hipEventDestroy(b);
    }
};
}  // namespace

extern "C" int vkb_reference_loop(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n,
                                  size_t k, const void* A, const void* B, void* C, void* stream, int warmup,
                                  int iters, float* per_iter_ms) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < warmup; i++) {
        int st = vk_gemm(version, in_dtype, out_dtype, m, n, k, A, B, C, stream);
        if (st != VK_OK) return st;
    }
    Events ev;
    if (!ev.ok) return VK_ERR_HIP;
    for (int i = 0; i < iters; i++) {
        if (hipEventRecord(ev.a, s) != hipSuccess) return VK_ERR_HIP;
        int st = vk_gemm(version, in_dtype, out_dtype, m, n, k, A, B, C, stream);
        if (st != VK_OK) return st;
        if (hipEventRecord(ev.b, s) != hipSuccess) return VK_ERR_HIP;
        if (hipEventSynchronize(ev.b) != hipSuccess) return VK_ERR_HIP;
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, ev.a, ev.b) != hipSuccess) return VK_ERR_HIP;
        if (per_iter_ms) per_iter_ms[i] = ms;
    }
    return VK_OK;
}

extern "C" int vkb_back_to_back(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n,
                                size_t k, const void* A, const void* B, void* C, void* stream, int iters,
                                float* total_ms) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    Events ev;
    if (!ev.ok) return VK_ERR_HIP;
    if (hipEventRecord(ev.a, s) != hipSuccess) return VK_ERR_HIP;
    for (int i = 0; i < iters; i++) {
        int st = vk_gemm(version, in_dtype, out_dtype, m, n, k, A, B, C, stream);
        if (st != VK_OK) return st;
    }
    if (hipEventRecord(ev.b, s) != hipSuccess) return VK_ERR_HIP;
    if (hipEventSynchronize(ev.b) != hipSuccess) return VK_ERR_HIP;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, ev.a, ev.b) != hipSuccess) return VK_ERR_HIP;
    if (total_ms) *total_ms = ms;
    return VK_OK;
}

extern "C" int vkb_stream_loop(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n,
                               size_t k, const void* A, const void* B, void* C, void* stream, int warmup,
                               int iters, float* total_ms) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (iters <= 0) return VK_ERR_SHAPE;
    for (int i = 0; i < warmup; i++) {
        int st = vk_gemm(version, in_dtype, out_dtype, m, n, k, A, B, C, stream);
        if (st != VK_OK) return st;
    }
    if (hipDeviceSynchronize() != hipSuccess) return VK_ERR_HIP;
    Events ev;
    if (!ev.ok) return VK_ERR_HIP;
    if (hipEventRecord(ev.a, s) != hipSuccess) return VK_ERR_HIP;
    for (int i = 0; i < iters; i++) {
        int st = vk_gemm(version, in_dtype, out_dtype, m, n, k, A, B, C, stream);
        if (st != VK_OK) return st;
    }
    if (hipEventRecord(ev.b, s) != hipSuccess) return VK_ERR_HIP;
    if (hipEventSynchronize(ev.b) != hipSuccess) return VK_ERR_HIP;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, ev.a, ev.b) != hipSuccess) return VK_ERR_HIP;
    if (total_ms) *total_ms = ms;
    return hipDeviceSynchronize() == hipSuccess ? VK_OK : VK_ERR_HIP;
}
