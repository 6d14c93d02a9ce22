// clock_probe.cpp -- the shader clock while a GEMM runs back to back.
//
// MI355X runs a sustained matrix-core load at a power-limited clock that
// depends on the kernel and on its data.  A one-wave probe kernel on a second
// stream samples s_memtime (shader clock) and s_memrealtime (100 MHz
// constant clock) while `iters` launches of the GEMM run on the first stream;
// each window of 200 samples gives the clock over ~4 ms.  Inputs are
// uniform[-1,1) fp16, as in bench.py.
//
// Usage: clock_probe [version] [m] [n] [k] [iters] [f16|f32]   (output dtype = input dtype)
//
// The probe wave needs a few VGPRs on one CU: a GEMM whose workgroups use all
// 512 VGPRs of every SIMD (fp16 versions 6 and 7) is displaced by it and the
// figures then do not describe the GEMM alone.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "playground/utils.hpp"
#include "vk_gemm.h"

namespace {
constexpr int kSamples = 8000;
constexpr int kWindow = 200;

// One wave; exits after kSamples samples (about 20 us apart).
__global__ void clock_probe_kernel(unsigned long long* out) {
    for (int i = 0; i < kSamples; i++) {
        const unsigned long long t = __builtin_amdgcn_s_memtime();
        const unsigned long long r = __builtin_amdgcn_s_memrealtime();
        if (threadIdx.x == 0) {
            out[2 * i] = t;
            out[2 * i + 1] = r;
        }
        for (int s = 0; s < 4; s++) __builtin_amdgcn_s_sleep(127);
    }
}
}  // namespace

int main(int argc, char** argv) {
    const int version = argc > 1 ? std::atoi(argv[1]) : 5;
    const size_t m = argc > 2 ? std::strtoul(argv[2], nullptr, 10) : 4096;
    const size_t n = argc > 3 ? std::strtoul(argv[3], nullptr, 10) : 4096;
    const size_t k = argc > 4 ? std::strtoul(argv[4], nullptr, 10) : 4096;
    const int iters = argc > 5 ? std::atoi(argv[5]) : 2000;
    const bool f32 = argc > 6 && std::string(argv[6]) == "f32";
    const vk_dtype dt = f32 ? VK_DTYPE_F32 : VK_DTYPE_F16;
    const size_t es = f32 ? 4 : 2;
    const int st0 = vk_gemm_check(version, dt, dt, m, n, k, (void*)4096, (void*)4096,
                                  (void*)4096);
    if (st0 != VK_OK || iters < 1) {
        std::fprintf(stderr, "clock_probe: version %d rejects %zux%zux%zu (%s)\n", version, m, n, k,
                     vk_status_string(st0));
        return 1;
    }
    std::vector<_Float16> h(std::max(m * k, k * n));
    std::vector<float> hf(f32 ? h.size() : 0);
    std::mt19937 gen(20261201);
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    for (auto& x : h) x = (_Float16)dist(gen);
    for (size_t i = 0; i < hf.size(); i++) hf[i] = (float)h[i];
    void *A = nullptr, *B = nullptr, *C = nullptr;
    unsigned long long* d = nullptr;
    PLAYGROUND_HIP_CHECK(hipMalloc(&A, m * k * es));
    PLAYGROUND_HIP_CHECK(hipMalloc(&B, k * n * es));
    PLAYGROUND_HIP_CHECK(hipMalloc(&C, m * n * es));
    PLAYGROUND_HIP_CHECK(hipMalloc(&d, kSamples * 16));
    const void* src = f32 ? (const void*)hf.data() : (const void*)h.data();
    PLAYGROUND_HIP_CHECK(hipMemcpy(A, src, m * k * es, hipMemcpyHostToDevice));
    PLAYGROUND_HIP_CHECK(hipMemcpy(B, src, k * n * es, hipMemcpyHostToDevice));
    hipStream_t s1, s2;
    PLAYGROUND_HIP_CHECK(hipStreamCreate(&s1));
    PLAYGROUND_HIP_CHECK(hipStreamCreate(&s2));
    auto run = [&](int count) {
        for (int i = 0; i < count; i++) {
            const int st = vk_gemm(version, dt, dt, m, n, k, A, B, C, s1);
            if (st != VK_OK) {
                std::fprintf(stderr, "clock_probe: vk_gemm failed: %s\n", vk_status_string(st));
                std::exit(1);
            }
        }
    };
    run(10);
    PLAYGROUND_HIP_CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    PLAYGROUND_HIP_CHECK(hipEventCreate(&e0));
    PLAYGROUND_HIP_CHECK(hipEventCreate(&e1));
    hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, s2, d);
    PLAYGROUND_HIP_CHECK(hipGetLastError());
    PLAYGROUND_HIP_CHECK(hipEventRecord(e0, s1));
    run(iters);
    PLAYGROUND_HIP_CHECK(hipEventRecord(e1, s1));
    PLAYGROUND_HIP_CHECK(hipDeviceSynchronize());
    float ms = 0.0f;
    PLAYGROUND_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    std::vector<unsigned long long> o(2 * kSamples);
    PLAYGROUND_HIP_CHECK(hipMemcpy(o.data(), d, kSamples * 16, hipMemcpyDeviceToHost));
    const double per = ms / iters;
    std::printf("%s %zux%zux%zu: %d launches back to back, %.4f ms each, %.1f TFLOPS\n", vk_gemm_name(version, dt), m,
                n, k, iters, per, 2.0 * m * n * k / per / 1e9);
    std::printf("probe: %d samples over %.0f us (GEMM run: %.0f us)\n", kSamples,
                (o[2 * (kSamples - 1) + 1] - o[1]) / 100.0, ms * 1e3);
    for (int w = 0; w + kWindow < kSamples; w += kWindow) {
        const double dc = (double)(o[2 * (w + kWindow)] - o[2 * w]);
        const double dr = (double)(o[2 * (w + kWindow) + 1] - o[2 * w + 1]);
        std::printf("t=%8.0f us  clock %5.0f MHz\n", (o[2 * w + 1] - o[1]) / 100.0, dc / dr * 100.0);
    }
    PLAYGROUND_HIP_CHECK(hipFree(A));
    PLAYGROUND_HIP_CHECK(hipFree(B));
    PLAYGROUND_HIP_CHECK(hipFree(C));
    PLAYGROUND_HIP_CHECK(hipFree(d));
    return 0;
}
