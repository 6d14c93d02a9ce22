// mfma_stream.cpp -- the matrix cores' own ceiling under MI355X's power
// limit: every CU runs nothing but MFMAs (fp16, or fp32 for the f32_ mixes)
// on operands held in registers
// (2 waves per SIMD, as version 7), back to back for a settle phase and then
// 20 timed launches, while the driver's metrics table is sampled
// (libvk_bench.so).  One JSON line per operand mix:
//
//   chain2   v_mfma_f32_16x16x32_f16, each accumulator's two MFMAs back to
//            back (version 7's order), random uniform[-1,1) operands
//   rotate   the same instructions rotating over the 16 accumulators
//   m32      v_mfma_f32_32x32x16_f16 (4 accumulators of 16 registers), rotating
//   zero     chain2 with all-zero operands
//   chain4   as chain2 with each accumulator's four MFMAs back to back
//   chain8   as chain2 with each accumulator's eight MFMAs back to back
//   gemm     chains of 2 over a GEMM's operands (accumulator (i, j) takes
//            A(i, k) B(j, k) for k = 0, 1; A, B registers change with k),
//            blocks in row order, every chain k = 0 then 1 (version 7's
//            order): consecutive MFMAs share no operand register
//   snake    the same chains, alternate ones in k = 1, 0 order and the
//            blocks snaked along j, so that each chain starts on the
//            operand register (A, or B at a row change) the previous one
//            ended on
//   *_w1     the same mix with one wave per SIMD (256-thread workgroups)
//   f32_32x32x2  v_mfma_f32_32x32x2_f32 rotating over 8 accumulators of 16
//            registers (fp32 operands, one register each), as fp32 version 2
//   f32_16x16x4  v_mfma_f32_16x16x4_f32 rotating over 16 accumulators
//   f32_*_w1 the fp32 mixes with one wave per SIMD
//
// No GEMM reaches more than its mix's figure on the same board: the figure
// prices the MFMA work alone, with no loads, LDS traffic or barriers.
//
//   vibekernel_amd/harness/bin/mfma_stream [settle_ms [mix,mix,...]]
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "playground/utils.hpp"
#include "vk_bench.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kThreads = 512;       // 8 waves: 2 per SIMD
constexpr int kLdsPin = 96 * 1024;

template <int kMode>
__global__ __launch_bounds__(kThreads) void mfma_stream(const half8* __restrict__ src, float* __restrict__ dst,
                                                       int iters) {
  const size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x;
  half8 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a[i] = src[t * 8 + i];
    b[i] = src[t * 8 + 4 + i];
  }
  float s = 0.0f;
  if constexpr (kMode == 7 || kMode == 8) {
    // fp32 operands: one register each, 4 per lane of A and of B
    float af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      af[i] = (float)a[i][0] + (float)a[i][1];
      bf[i] = (float)b[i][0] + (float)b[i][1];
    }
    if constexpr (kMode == 7) {
      float16v acc[8];
#pragma unroll
      for (int j = 0; j < 8; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;
      for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
          for (int j = 0; j < 8; j++) {
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[(j + r) & 3], bf[j & 3], acc[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
      }
#pragma unroll
      for (int j = 0; j < 8; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += acc[j][r];
    } else {
      float4v acc[16];
#pragma unroll
      for (int j = 0; j < 16; j++) acc[j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
      for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
          for (int j = 0; j < 16; j++) {
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[(j + r) & 3], bf[j >> 2], acc[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
      }
#pragma unroll
      for (int j = 0; j < 16; j++) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    }
  } else if constexpr (kMode == 2) {
    float16v acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
      for (int r = 0; r < 8; r++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[(j + r) & 3], b[j], acc[j], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) s += acc[j][r];
  } else {
    float4v acc[16];
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    for (int it = 0; it < iters; it++) {
      if constexpr (kMode == 1) {  // rotate: every accumulator once, then again
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
          for (int j = 0; j < 16; j++) {
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[(j + r) & 3], b[j >> 2], acc[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
      } else if constexpr (kMode == 5 || kMode == 6) {
        // 4 x 4 blocks; A(i, k) = a[2 (i & 1) + k], B(j, k) = b[2 (j & 1) + k]
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const int j = kMode == 6 && (i & 1) ? 3 - jj : jj;
            const int c = 4 * i + jj;                       // chain number
            const int k0 = kMode == 6 ? (c & 1) : 0;        // first k of the chain
#pragma unroll
            for (int r = 0; r < 2; r++) {
              const int k = k0 ^ r;
              acc[4 * i + j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2 * (i & 1) + k], b[2 * (j & 1) + k],
                                                                      acc[4 * i + j], 0, 0, 0);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
      } else {  // chains of kChain: each accumulator's MFMAs back to back
        constexpr int kChain = kMode == 3 ? 4 : kMode == 4 ? 8 : 2;
#pragma unroll
        for (int j = 0; j < 16; j++)
#pragma unroll
          for (int c = 0; c < kChain; c++) {
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[(j + c) & 3], b[j >> 2], acc[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; j++) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  }
  dst[t] = s;  // keeps the work
}

struct Mix {
  const char* name;
  int mode;
  bool zero;
  double flop_per_mfma;
  int mfma_per_iter;  // per wave
  int threads;        // per workgroup (one per CU): 512 = 2 waves per SIMD, 256 = 1
  double flop_clk_cu = 4096.0;  // dense peak per clock per CU (fp16 4096, fp32 256)
};

int main(int argc, char** argv) {
  const double settle_ms = argc > 1 ? std::atof(argv[1]) : 2500.0;
  const std::string only = argc > 2 ? std::string(",") + argv[2] + "," : std::string();
  int dev = 0, cus = 0;
  PLAYGROUND_HIP_CHECK(hipGetDevice(&dev));
  PLAYGROUND_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int grid = cus;  // one 512-thread workgroup per CU
  const size_t lanes = (size_t)grid * kThreads;
  std::vector<_Float16> host(lanes * 64);
  std::mt19937 rng(20261201);
  std::uniform_real_distribution<float> u(-1.0f, 1.0f);
  for (auto& h : host) h = (_Float16)u(rng);
  half8 *d_rand = nullptr, *d_zero = nullptr;
  float* d_out = nullptr;
  PLAYGROUND_HIP_CHECK(hipMalloc(&d_rand, host.size() * sizeof(_Float16)));
  PLAYGROUND_HIP_CHECK(hipMalloc(&d_zero, host.size() * sizeof(_Float16)));
  PLAYGROUND_HIP_CHECK(hipMalloc(&d_out, lanes * sizeof(float)));
  PLAYGROUND_HIP_CHECK(hipMemcpy(d_rand, host.data(), host.size() * sizeof(_Float16), hipMemcpyHostToDevice));
  PLAYGROUND_HIP_CHECK(hipMemset(d_zero, 0, host.size() * sizeof(_Float16)));
  const bool clock_ok = vkb_clock_open() == VK_OK;
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<0>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<1>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<2>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<3>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<4>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<5>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<6>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<7>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));
  PLAYGROUND_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_stream<8>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPin));

  constexpr double k16 = 16.0 * 16 * 32 * 2;
  const Mix mixes[] = {{"chain2", 0, false, k16, 32, 512},    {"rotate", 1, false, k16, 32, 512},
                       {"m32", 2, false, 32.0 * 32 * 16 * 2, 32, 512},
                       {"zero", 0, true, k16, 32, 512},      {"chain4", 3, false, k16, 64, 512},
                       {"chain8", 4, false, k16, 128, 512},  {"gemm", 5, false, k16, 32, 512},
                       {"snake", 6, false, k16, 32, 512},    {"chain2_w1", 0, false, k16, 32, 256},
                       {"rotate_w1", 1, false, k16, 32, 256}, {"snake_w1", 6, false, k16, 32, 256},
                       {"f32_32x32x2", 7, false, 32.0 * 32 * 2 * 2, 32, 512, 256.0},
                       {"f32_16x16x4", 8, false, 16.0 * 16 * 4 * 2, 32, 512, 256.0},
                       {"f32_32x32x2_w1", 7, false, 32.0 * 32 * 2 * 2, 32, 256, 256.0},
                       {"f32_16x16x4_w1", 8, false, 16.0 * 16 * 4 * 2, 32, 256, 256.0}};
  for (const Mix& mx : mixes) {
    if (!only.empty() && only.find(std::string(",") + mx.name + ",") == std::string::npos) continue;
    const half8* src = mx.zero ? d_zero : d_rand;
    // about 1 ms per launch at the full rate
    const int iters = (mx.mode == 2 || mx.mode >= 7 ? 1024 : 2048) * 32 / mx.mfma_per_iter;
    // 96 KB of (unused) dynamic LDS per workgroup: one workgroup per CU
    auto launch = [&]() {
      if (mx.mode == 0)
        hipLaunchKernelGGL(mfma_stream<0>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
      else if (mx.mode == 1)
        hipLaunchKernelGGL(mfma_stream<1>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
      else if (mx.mode == 2)
        hipLaunchKernelGGL(mfma_stream<2>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
      else if (mx.mode == 3)
        hipLaunchKernelGGL(mfma_stream<3>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
      else if (mx.mode == 4)
        hipLaunchKernelGGL(mfma_stream<4>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
      else if (mx.mode == 5)
        hipLaunchKernelGGL(mfma_stream<5>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
      else if (mx.mode == 6)
        hipLaunchKernelGGL(mfma_stream<6>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
      else if (mx.mode == 7)
        hipLaunchKernelGGL(mfma_stream<7>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
      else
        hipLaunchKernelGGL(mfma_stream<8>, dim3(grid), dim3(mx.threads), kLdsPin, 0, src, d_out, iters);
    };
    bool sampling = false;
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
      for (int i = 0; i < 10; i++) launch();
      PLAYGROUND_HIP_CHECK(hipGetLastError());
      PLAYGROUND_HIP_CHECK(hipDeviceSynchronize());
      const double el = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
      if (el >= settle_ms) break;
      if (!sampling && clock_ok && el >= settle_ms / 2) sampling = vkb_clock_start(1000) == VK_OK;
    }
    hipEvent_t e0, e1;
    PLAYGROUND_HIP_CHECK(hipEventCreate(&e0));
    PLAYGROUND_HIP_CHECK(hipEventCreate(&e1));
    PLAYGROUND_HIP_CHECK(hipEventRecord(e0, 0));
    for (int i = 0; i < 20; i++) launch();
    PLAYGROUND_HIP_CHECK(hipEventRecord(e1, 0));
    PLAYGROUND_HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    PLAYGROUND_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    PLAYGROUND_HIP_CHECK(hipEventDestroy(e0));
    PLAYGROUND_HIP_CHECK(hipEventDestroy(e1));
    vkb_clock_sample smp[64];
    int ns = 0;
    if (sampling) {
      ns = vkb_clock_samples(smp, 64);
      vkb_clock_stats st;
      vkb_clock_stop(&st);
    }
    const double flop = (double)grid * (mx.threads / 64) * mx.mfma_per_iter * iters * mx.flop_per_mfma * 20;
    const double tflops = flop / (ms * 1e-3) / 1e12;
    std::printf("{\"mix\": \"%s\", \"waves_per_simd\": %d, \"tflops\": %.1f, \"ms_per_launch\": %.4f, \"cus\": %d",
                mx.name, mx.threads / 256, tflops, ms / 20, cus);
    if (ns > 0) {
      const vkb_clock_sample& s = smp[(ns < 64 ? ns : 64) - 1];  // the last refresh before the timed launches
      std::printf(", \"sclk_mhz\": %.1f, \"socket_w\": %.1f, \"xcd_mhz\": [", s.gfx_mhz, s.socket_w);
      for (int x = 0; x < 8; x++) std::printf("%s%.0f", x ? ", " : "", s.xcd_mhz[x]);
      std::printf("], \"frac_of_peak_at_sclk\": %.4f", tflops / (cus * mx.flop_clk_cu * s.gfx_mhz * 1e6 / 1e12));
    }
    const double spec = cus * mx.flop_clk_cu * 2.4e9 / 1e12;  // 2516.6 (fp16) or 157.3 (fp32) on 256 CUs
    std::printf(", \"frac_of_spec_peak\": %.4f, \"spec_peak_tflops\": %.1f}\n", tflops / spec, spec);
    std::fflush(stdout);
  }
  PLAYGROUND_HIP_CHECK(hipFree(d_rand));
  PLAYGROUND_HIP_CHECK(hipFree(d_zero));
  PLAYGROUND_HIP_CHECK(hipFree(d_out));
  return 0;
}
