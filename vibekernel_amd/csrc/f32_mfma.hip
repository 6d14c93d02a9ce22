// f32_mfma.hip -- fp32 GEMM on the matrix cores (version 2 for fp32).
//
// Same operator as fp32 version 1 (f32_valu.hip: the harness's fp32 path,
// results/naive_cycle4/include/playground/system.hpp:35-41, ground truth
// matmul_f32_v0_cblas.cpp:8-12), computed with v_mfma_f32_32x32x2_f32.
// Measured on MI355X with random, changing operands on all CUs (2 waves per
// SIMD): that instruction sustains 148.7 TFLOP/s of the 157.3 dense fp32
// figure, while the 16x16x4 form reaches only ~74 and the VALU kernel (plain
// FMAs, LDS-bound at 8x8 outputs per thread) 89.6 at 4096^3.  An fp32 MFMA
// does 64 FLOP per clock per SIMD -- 16x fewer than the fp16 form -- so the
// operand traffic per cycle is small and the kernel can be simple:
//  * 256x256 tile, 8 waves; wave w owns rows 128*(w/4) .. +127 and columns
//    64*(w%4) .. +63: 4x2 blocks of 32x32 (128 fp32 accumulators per lane);
//  * 16-deep k-tiles (A 256x16 and B 16x256 fp32, 32 KB) in a 4-stage LDS
//    ring filled by direct-to-LDS loads (4 per wave per k-tile), one barrier
//    per k-tile;
//  * per k-tile each wave reads its fragments (8 ds_read_b128 of A, 16
//    ds_read_b32 of B) and issues 64 MFMAs of 64 cycles.
// Fragments: the MFMA takes lane l's A value as X[l%32][l/32] and its B value
// as Y[l/32][l%32] (2 k per instruction).  Step s of a k-tile pairs k = s
// (lanes 0..31) with k = 8 + s (lanes 32..63), so a lane's A values for the
// 8 steps are 8 consecutive k of one row (two 16-byte reads) and its B values
// one column of 8 k-rows.  Result: lane l, register r holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32] of the block.
// LDS swizzles (physical 16-byte chunk = logical ^ f(row)):
//  * A rows are 64 B (4 chunks): f = (row / 4) % 4, so 16 consecutive rows
//    reading one logical chunk hit 16 distinct slots of the 256-byte bank
//    space;
//  * B k-rows are 1 KB (64 chunks): f = 8 for k-rows 8..15, so the two lane
//    halves (k and k + 8, same columns) use opposite halves of the banks.
// The k-order of the sum differs from the oracle's sequential chain (pairs
// of products per step), so parity is the fp32 accumulation bound, not bit
// equality.
#include "vk_device.hpp"
#include "vk_internal.hpp"
#include "vk_tile.hpp"

#include <atomic>

namespace vk {
namespace {

constexpr int kBM = 256, kBN = 256;
constexpr int kBK = 16;  // fp32 k per k-tile
constexpr int kNS = 4;   // LDS ring stages
constexpr int kThreads = 512;
constexpr int kABytes = kBM * kBK * 4;  // 16 KB: 256 rows x 64 B
constexpr int kBBytes = kBK * kBN * 4;  // 16 KB: 16 k-rows x 1 KB
constexpr int kStageBytes = kABytes + kBBytes;
constexpr int kLdsBytes = kNS * kStageBytes;  // 128 KB
constexpr int kDma = 4;                       // direct-to-LDS instructions per wave per k-tile
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");

typedef float float16v_ __attribute__((ext_vector_type(16)));

__host__ __device__ constexpr int swz_a32(int row) { return (row >> 2) & 3; }
__host__ __device__ constexpr int swz_b32(int krow) { return ((krow >> 3) & 1) << 3; }

__device__ __forceinline__ float lds_read_f32(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) float*>(addr);
}
__device__ __forceinline__ float4v lds_read_f4(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) float4v*>(addr);
}

__global__ __launch_bounds__(kThreads) void f32_mfma_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                            float* __restrict__ C, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, gw = wave & 3;
  int tm, tn;
  tile_of(blockIdx.x, M / kBM, N / kBN, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  // ---- direct-to-LDS duty: A instructions 2w, 2w+1 (rows 16i .. 16i+15),
  // B instructions 2w, 2w+1 (k-row i) of every k-tile ----
  uint32_t voffA[2], voffB[2];
#pragma unroll
  for (int d = 0; d < 2; d++) {
    const int i = 2 * wave + d;
    const int row = 16 * i + (lane >> 2);
    const int ca = (lane & 3) ^ swz_a32(row);
    voffA[d] = (uint32_t)(((size_t)row * K + ca * 4) * 4);
    const int cb = lane ^ swz_b32(i);
    voffB[d] = (uint32_t)(((size_t)i * N + cb * 4) * 4);
  }
  const char* gA = reinterpret_cast<const char*>(A) + (size_t)m0 * K * 4;
  const char* gB = reinterpret_cast<const char*>(B) + (size_t)n0 * 4;
  auto issue = [&](int kt, int slot) {
    const uint32_t s = lds_base + slot * kStageBytes;
#pragma unroll
    for (int d = 0; d < 2; d++) {
      const int i = 2 * wave + d;
      dma16(gA + (size_t)kt * kBK * 4, voffA[d], s + i * 1024);
      dma16(gB + (size_t)kt * kBK * N * 4, voffB[d], s + kABytes + i * 1024);
    }
  };

  // ---- fragment addresses inside a stage ----
  const int h = lane >> 5;
  uint32_t aoff[4][2];
#pragma unroll
  for (int bi = 0; bi < 4; bi++) {
    const int row = grp * 128 + bi * 32 + (lane & 31);
#pragma unroll
    for (int c = 0; c < 2; c++) aoff[bi][c] = row * 64 + 16 * ((2 * h + c) ^ swz_a32(row));
  }
  uint32_t boff[2];
#pragma unroll
  for (int bj = 0; bj < 2; bj++) {
    const int col = gw * 64 + bj * 32 + (lane & 31);
    // k-row 8h + s: bit 3 is h, so the swizzle is the same for all 8 steps
    boff[bj] = kABytes + (8 * h) * 1024 + 16 * ((col >> 2) ^ (h << 3)) + 4 * (col & 3);
  }

  float16v_ acc[4][2];
#pragma unroll
  for (int bi = 0; bi < 4; bi++)
#pragma unroll
    for (int bj = 0; bj < 2; bj++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[bi][bj][r] = 0.0f;
  prefer_agpr_accumulators();

  const int nk = K / kBK;
#pragma unroll
  for (int st = 0; st < kNS - 1; st++) issue(min(st, nk - 1), st);

  for (int t = 0; t < nk; t++) {
    // This wave's loads of k-tile t are in; then everyone's (barrier), which
    // also ends every wave's reads of the slot the next issue refills.
    wait_vmcnt<(kNS - 2) * kDma>();
    lds_barrier();
    issue(min(t + kNS - 1, nk - 1), (t + kNS - 1) % kNS);
    const uint32_t s = lds_base + (t % kNS) * kStageBytes;
    float a[4][8], b[2][8];
#pragma unroll
    for (int bi = 0; bi < 4; bi++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const float4v v = lds_read_f4(s + aoff[bi][c]);
        a[bi][4 * c + 0] = v[0];
        a[bi][4 * c + 1] = v[1];
        a[bi][4 * c + 2] = v[2];
        a[bi][4 * c + 3] = v[3];
      }
#pragma unroll
    for (int bj = 0; bj < 2; bj++)
#pragma unroll
      for (int st = 0; st < 8; st++) b[bj][st] = lds_read_f32(s + boff[bj] + st * 1024);
#pragma unroll
    for (int st = 0; st < 8; st++)
#pragma unroll
      for (int bi = 0; bi < 4; bi++)
#pragma unroll
        for (int bj = 0; bj < 2; bj++)
          acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[bi][st], b[bj][st], acc[bi][bj], 0, 0, 0);
  }
  wait_vmcnt<0>();  // clamped refills past the last k-tile

  // ---- epilogue: lane l, register r of block (bi, bj) ->
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32: 128-byte row segments ----
  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  float* Cw = C + (size_t)(m0 + grp * 128) * N + n0 + gw * 64;
#pragma unroll
  for (int bi = 0; bi < 4; bi++)
#pragma unroll
    for (int bj = 0; bj < 2; bj++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = bi * 32 + 8 * (r >> 2) + 4 * (lane_e >> 5) + (r & 3);
        Cw[(size_t)row * N + bj * 32 + (lane_e & 31)] = acc[bi][bj][r];
      }
}

hipError_t launch_f32_mfma(const GemmArgs& a) {
  static std::atomic<uint64_t> attr_done{0};
  hipError_t e = ensure_lds_attr(f32_mfma_kernel, kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  const int tiles = (int)((a.m / kBM) * (a.n / kBN));
  hipLaunchKernelGGL(f32_mfma_kernel, dim3(tiles), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const float*>(a.A), static_cast<const float*>(a.B), static_cast<float*>(a.C),
                     (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

// 32-bit lane offsets: 16 rows of A per instruction span (16 * K + 4) floats
// beyond the k-tile base and one k-row of B spans N floats; the per-k-tile and
// per-tile steps are 64-bit scalar bases.
bool f32_mfma_shape_ok(size_t m, size_t n, size_t k) {
  return (size_t)256 * k * 4 < (1ull << 31) && (size_t)kBK * n * 4 < (1ull << 31) &&
         (m / kBM) * (n / kBN) < (1ull << 31);
}

}  // namespace

void register_f32_mfma() {
  KernelEntry e{};
  e.version = 2;
  e.in_dtype = VK_DTYPE_F32;
  e.name = "f32_v2_mfma256";
  e.caps = make_caps(2, VK_DTYPE_F32, kOutF32, kBM, kBN, kBK, 16, kBM, kBN, kBK, kThreads, kLdsBytes, 0, 0);
  e.launch = launch_f32_mfma;
  e.workspace = nullptr;
  e.shape_ok = f32_mfma_shape_ok;
  register_kernel(e);
}

}  // namespace vk
