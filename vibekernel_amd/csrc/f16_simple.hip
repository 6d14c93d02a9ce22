// f16_simple.hip -- version 1 for fp16: the correctness anchor.
//
// Plays the role of the reference's first tensor-core kernel
// (results/ralph_loop_fable/src/matmul_f16/matmul_f16_v1_wmma.cu:15-95: one
// 128x128 tile per 256-thread block, fp32 accumulation), written for CDNA4:
//   * 4 waves of 64 lanes, each owning a 64x64 quadrant as 2x2
//     v_mfma_f32_32x32x16_f16 blocks with fp32 accumulators;
//   * one LDS stage of A (128 x 32) and B^T (128 x 32); B is transposed while
//     it is stored so both operands are read as 16-byte rows;
//   * every global access is bounds-checked and every shape is accepted
//     (m, n, k >= 0; k = 0 writes zeros), unlike the reference kernels, which
//     assume tile-divisible shapes.
// It is deliberately simple: no direct-to-LDS loads, no double buffering.
#include "vk_device.hpp"
#include "vk_internal.hpp"

namespace vk {
namespace {

constexpr int kTile = 128;
constexpr int kBK = 32;
constexpr int kPad = 8;            // row pitch 40 halves = 80 B keeps 16 B alignment
constexpr int kPitch = kBK + kPad;

template <typename OutT>
__global__ __launch_bounds__(256) void f16_simple_kernel(const half_t* __restrict__ A,
                                                         const half_t* __restrict__ B,
                                                         OutT* __restrict__ C, int64_t M, int64_t N,
                                                         int64_t K) {
  __shared__ __attribute__((aligned(16))) half_t As[kTile * kPitch];
  __shared__ __attribute__((aligned(16))) half_t Bt[kTile * kPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * kTile;
  const int64_t n0 = (int64_t)blockIdx.x * kTile;

  float16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  for (int64_t k0 = 0; k0 < K; k0 += kBK) {
    // A tile: 128 rows x 32 k; consecutive threads read consecutive k.
#pragma unroll
    for (int e = 0; e < (kTile * kBK) / 256; e++) {
      const int idx = tid + 256 * e;
      const int row = idx / kBK, col = idx % kBK;
      const int64_t gr = m0 + row, gc = k0 + col;
      half_t v = (half_t)0.0f;
      if (gr < M && gc < K) v = A[gr * K + gc];
      As[row * kPitch + col] = v;
    }
    // B tile: 32 k x 128 n, stored transposed as Bt[n][k].
#pragma unroll
    for (int e = 0; e < (kTile * kBK) / 256; e++) {
      const int idx = tid + 256 * e;
      const int krow = idx / kTile, ncol = idx % kTile;
      const int64_t gr = k0 + krow, gc = n0 + ncol;
      half_t v = (half_t)0.0f;
      if (gr < K && gc < N) v = B[gr * N + gc];
      Bt[ncol * kPitch + krow] = v;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ks++) {
      half8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; i++)
        a[i] = *reinterpret_cast<const half8*>(
            &As[(wm * 64 + i * 32 + (lane & 31)) * kPitch + ks * 16 + (lane >> 5) * 8]);
#pragma unroll
      for (int j = 0; j < 2; j++)
        b[j] = *reinterpret_cast<const half8*>(
            &Bt[(wn * 64 + j * 32 + (lane & 31)) * kPitch + ks * 16 + (lane >> 5) * 8]);
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = mfma32x32x16(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
        if (row < M && col < N) C[row * N + col] = convert_out<OutT>(acc[i][j][r]);
      }
}

hipError_t launch_simple(const GemmArgs& a) {
  if (a.m == 0 || a.n == 0) return hipSuccess;
  dim3 grid((unsigned)((a.n + kTile - 1) / kTile), (unsigned)((a.m + kTile - 1) / kTile));
  const half_t* A = static_cast<const half_t*>(a.A);
  const half_t* B = static_cast<const half_t*>(a.B);
  if (a.out_dtype == VK_DTYPE_F16)
    hipLaunchKernelGGL(f16_simple_kernel<half_t>, grid, dim3(256), 0, a.stream, A, B,
                       static_cast<half_t*>(a.C), (int64_t)a.m, (int64_t)a.n, (int64_t)a.k);
  else
    hipLaunchKernelGGL(f16_simple_kernel<float>, grid, dim3(256), 0, a.stream, A, B,
                       static_cast<float*>(a.C), (int64_t)a.m, (int64_t)a.n, (int64_t)a.k);
  return hipGetLastError();
}

bool simple_shape_ok(size_t m, size_t n, size_t k) {
  // grid.y = ceil(m / 128) must fit the 65535 limit of the y dimension
  (void)n;
  (void)k;
  return (m + kTile - 1) / kTile <= 65535;
}

}  // namespace

void register_f16_simple() {
  KernelEntry e{};
  e.version = 1;
  e.in_dtype = VK_DTYPE_F16;
  e.name = "f16_v1_simple";
  e.caps = make_caps(1, VK_DTYPE_F16, kOutF16 | kOutF32, 1, 1, 1, 2, kTile, kTile, kBK, 256,
                     2 * kTile * kPitch * 2, 0, 0);
  e.launch = launch_simple;
  e.workspace = nullptr;
  e.shape_ok = simple_shape_ok;
  register_kernel(e);
}

}  // namespace vk
