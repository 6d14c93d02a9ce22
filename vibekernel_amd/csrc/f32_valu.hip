// f32_valu.hip -- fp32 SGEMM on the vector ALUs (version 1 for fp32).
//
// The reference has the fp32 harness path (results/naive_cycle4/include/
// playground/system.hpp:35-41, results/naive_fable_cycle2/src/CMakeLists.txt:5-11)
// and its v0 ground truth (matmul_f32_v0_cblas.cpp:8-12) but no hand-written
// fp32 kernel; its only GPU fp32 version called cublasSgemm.  This is a
// register-blocked VALU kernel:
//   * 128x256 workgroup tile, BK = 16, 256 threads, 8x16 outputs per thread
//     held as 4x4 register blocks (rows ty*4 and 64+ty*4, columns
//     64*g + tx*4 for g = 0..3) so the LDS operand reads are 16-byte and
//     conflict-free;
//   * A is stored k-major in LDS (transposed on the store) and B as loaded;
//   * the next k-tile is prefetched from HBM into registers while the current
//     one is multiplied, then written to the other LDS buffer (one barrier per
//     k-tile); the k-steps are unrolled by 2, so the compiler keeps two
//     k-steps of fragments live, not the whole k-tile.
// Roofline: the VOP2 FMA (`v_fmac_f32_e32`, what this compiles to) runs at
// the full 157.3 TFLOP/s rate on MI355X (measured 146.7 on independent
// chains; the VOP3 form runs at half).  What limits the kernel is the LDS
// return path: each 16-byte read returns 1 KB per wave whatever the
// broadcast, so it is the reads per FMA that count: 6 per 128 FMAs here
// (8x16 outputs) against 4 per 64 at 8x8 -- measured 91.0 against 82.9
// TFLOP/s on one box.
#include "vk_device.hpp"
#include "vk_internal.hpp"

namespace vk {
namespace {

constexpr int kTM = 128;             // tile rows
constexpr int kCG = 4;               // 64-column groups per tile
constexpr int kTN = 64 * kCG;        // tile columns
constexpr int kBK = 16;
constexpr int kApitch = kTM + 4;     // As_t[k][m] row pitch (floats)
constexpr int kLdA = kTM * kBK / 4 / 256;  // float4 loads of A per thread per k-tile
constexpr int kLdB = kBK * kTN / 4 / 256;  // float4 loads of B per thread per k-tile
static_assert(kLdA == 2 && kLdB == 4, "tile load mapping");

template <bool kCheck>
__global__ __launch_bounds__(256) void f32_valu_kernel(const float* __restrict__ A,
                                                       const float* __restrict__ B,
                                                       float* __restrict__ C, int64_t M, int64_t N,
                                                       int64_t K) {
  __shared__ __attribute__((aligned(16))) float As[2][kBK * kApitch];
  __shared__ __attribute__((aligned(16))) float Bs[2][kBK * kTN];

  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * kTM;
  const int64_t n0 = (int64_t)blockIdx.x * kTN;

  // Global load mapping: A: 128 rows x BK/4 float4 per row; B: BK rows x TN/4 float4.
  constexpr int kC4A = kBK / 4;   // float4 per A row
  constexpr int kC4B = kTN / 4;   // float4 per B row
  float4v ra[kLdA], rb[kLdB];
  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int e = 0; e < kLdA; e++) {
      const int idx = tid + 256 * e;
      const int row = idx / kC4A, c4 = idx % kC4A;
      const int64_t gr = m0 + row, gc = k0 + c4 * 4;
      if (!kCheck) {
        ra[e] = *reinterpret_cast<const float4v*>(&A[gr * K + gc]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++)
          ra[e][q] = (gr < M && gc + q < K) ? A[gr * K + gc + q] : 0.0f;
      }
    }
#pragma unroll
    for (int e = 0; e < kLdB; e++) {
      const int idx = tid + 256 * e;
      const int krow = idx / kC4B, c4 = idx % kC4B;
      const int64_t gr = k0 + krow, gc = n0 + c4 * 4;
      if (!kCheck) {
        rb[e] = *reinterpret_cast<const float4v*>(&B[gr * N + gc]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++)
          rb[e][q] = (gr < K && gc + q < N) ? B[gr * N + gc + q] : 0.0f;
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int e = 0; e < kLdA; e++) {
      const int idx = tid + 256 * e;
      const int row = idx / kC4A, c4 = idx % kC4A;
#pragma unroll
      for (int q = 0; q < 4; q++) As[buf][(c4 * 4 + q) * kApitch + row] = ra[e][q];
    }
#pragma unroll
    for (int e = 0; e < kLdB; e++) {
      const int idx = tid + 256 * e;
      const int krow = idx / kC4B, c4 = idx % kC4B;
      *reinterpret_cast<float4v*>(&Bs[buf][krow * kTN + c4 * 4]) = rb[e];
    }
  };

  float acc[8][4 * kCG];
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 4 * kCG; j++) acc[i][j] = 0.0f;

  const int64_t nk = (K + kBK - 1) / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; kt++) {
    const int cur = (int)(kt & 1);
    if (kt + 1 < nk) load_tile((kt + 1) * kBK);
#pragma unroll 2
    for (int kk = 0; kk < kBK; kk++) {
      const float4v a0 = *reinterpret_cast<const float4v*>(&As[cur][kk * kApitch + ty * 4]);
      const float4v a1 = *reinterpret_cast<const float4v*>(&As[cur][kk * kApitch + 64 + ty * 4]);
      float a[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      float b[4 * kCG];
#pragma unroll
      for (int g = 0; g < kCG; g++) {
        const float4v bg = *reinterpret_cast<const float4v*>(&Bs[cur][kk * kTN + 64 * g + tx * 4]);
#pragma unroll
        for (int q = 0; q < 4; q++) b[4 * g + q] = bg[q];
      }
#pragma unroll
      for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4 * kCG; j++) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    if (kt + 1 < nk) {
      store_tile(cur ^ 1);
      __syncthreads();
    }
  }

#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int64_t row = m0 + (i < 4 ? ty * 4 + i : 64 + ty * 4 + (i - 4));
#pragma unroll
    for (int g = 0; g < kCG; g++) {
      const int64_t col = n0 + g * 64 + tx * 4;
      if (!kCheck) {
        float4v v = {acc[i][g * 4 + 0], acc[i][g * 4 + 1], acc[i][g * 4 + 2], acc[i][g * 4 + 3]};
        *reinterpret_cast<float4v*>(&C[row * N + col]) = v;
      } else if (row < M) {
#pragma unroll
        for (int q = 0; q < 4; q++)
          if (col + q < N) C[row * N + col + q] = acc[i][g * 4 + q];
      }
    }
  }
}

hipError_t launch_f32(const GemmArgs& a) {
  dim3 grid((unsigned)((a.n + kTN - 1) / kTN), (unsigned)((a.m + kTM - 1) / kTM));
  const float* A = static_cast<const float*>(a.A);
  const float* B = static_cast<const float*>(a.B);
  float* C = static_cast<float*>(a.C);
  const bool full = a.m % kTM == 0 && a.n % kTN == 0 && a.k % kBK == 0 &&
                    ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 &&
                    ((uintptr_t)C & 15) == 0;
  if (full)
    hipLaunchKernelGGL(f32_valu_kernel<false>, grid, dim3(256), 0, a.stream, A, B, C, (int64_t)a.m,
                       (int64_t)a.n, (int64_t)a.k);
  else
    hipLaunchKernelGGL(f32_valu_kernel<true>, grid, dim3(256), 0, a.stream, A, B, C, (int64_t)a.m,
                       (int64_t)a.n, (int64_t)a.k);
  return hipGetLastError();
}

bool f32_shape_ok(size_t m, size_t n, size_t k) {
  (void)n;
  (void)k;
  return (m + kTM - 1) / kTM <= 65535;
}

}  // namespace

void register_f32_valu() {
  KernelEntry e{};
  e.version = 1;
  e.in_dtype = VK_DTYPE_F32;
  e.name = "f32_v1_valu";
  e.caps = make_caps(1, VK_DTYPE_F32, kOutF32, 1, 1, 1, 4, kTM, kTN, kBK, 256,
                     2 * kBK * (kApitch + kTN) * 4, 0, 0);
  e.launch = launch_f32;
  e.workspace = nullptr;
  e.shape_ok = f32_shape_ok;
  register_kernel(e);
}

}  // namespace vk
