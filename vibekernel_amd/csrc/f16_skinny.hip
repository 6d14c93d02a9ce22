// f16_skinny.hip -- fp16 GEMM for skinny A (decode-like: M <= 64), version 4.
//
// The reference has no path for this shape: its fast kernels need
// M % 256 == 0 and would launch min(G, numTiles) = 0 blocks at M = 16
// (results/ralph_loop_fable/src/matmul_f16/matmul_f16_v42_shfl2.cu:124, :520-527).
// At M = 16, N = K = 8192 the work is 2.1 GFLOP on 134 MB of B: the bound is
// HBM bandwidth, not the matrix cores.  Design:
//  * one 256-thread workgroup per 32-column block of B (grid = N / 32); the
//    4 waves split K into private quarters, so the k-loop has no barriers:
//    each wave streams its own B[k-range][32 cols] and A[0:M][k-range]
//    through a private NSTAGE-deep LDS ring with direct-to-LDS loads;
//  * fragments: A with ds_read_b128, B with the LDS transpose read, feeding
//    v_mfma_f32_16x16x32_f16 (16 rows of A per block, fp32 accumulation);
//  * the 4 partial 16x32 blocks per row block are summed through LDS at the
//    end (fixed order: wave 0 + 1 + 2 + 3) and written as fp16 or fp32;
//  * column block b runs on XCD b / 32 (workgroup id = 8 * (b % 32) + b / 32),
//    so the two 32-column blocks that share each 128-byte line of B are read
//    through the same L2.
#include "vk_device.hpp"
#include "vk_internal.hpp"
#include "vk_tile.hpp"

#include <atomic>

namespace vk {
namespace {

constexpr int kCols = 32;      // columns of B per workgroup
constexpr int kWaves = 4;
constexpr int kKStep = 32;     // k per stage (one 16x16x32 MFMA deep)

template <int MB>  // row blocks of 16: M = 16 * MB
struct SkinnyCfg {
  static constexpr int kBBytes = kKStep * kCols * 2;          // 2 KB: 32 rows x 64 B
  static constexpr int kABytes = 16 * MB * kKStep * 2;        // MB KB: rows x 64 B
  static constexpr int kStageBytes = kBBytes + kABytes;
  static constexpr int kStages = (36 * 1024) / kStageBytes;    // per wave, 36 KB budget
  static constexpr int kWaveBytes = kStages * kStageBytes;
  static constexpr int kLdsBytes = kWaves * kWaveBytes;
  static constexpr int kDmaB = kBBytes / 1024;                // 2 instructions (16 rows each)
  static constexpr int kDmaA = kABytes / 1024;                // MB instructions (16 rows each)
  static constexpr int kDmaPerStage = kDmaB + kDmaA;
  static_assert(kStages >= 4, "pipeline depth");
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

template <int MB, typename OutT>
__global__ __launch_bounds__(256, 1) void f16_skinny_kernel(const half_t* __restrict__ A,
                                                            const half_t* __restrict__ B,
                                                            OutT* __restrict__ C, int M, int N,
                                                            int K) {
  using G = SkinnyCfg<MB>;
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // Workgroup -> column block: 32 consecutive blocks per XCD.
  const int nblk = N / kCols;
  int cb = blockIdx.x;
  if ((nblk & 7) == 0) cb = (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3);
  const int n0 = cb * kCols;

  const int kq = K / kWaves;        // this wave's k range: [wave * kq, (wave+1) * kq)
  const int nsteps = kq / kKStep;
  const int kbeg = wave * kq;

  // DMA lane mapping: one instruction = 16 rows x 64 B (4 chunks of 16 B).
  const int drow = lane >> 2, dchunk = lane & 3;
  const char* gB = reinterpret_cast<const char*>(B) + ((size_t)kbeg * N + n0) * 2;
  const char* gA = reinterpret_cast<const char*>(A) + (size_t)kbeg * 2;
  uint32_t offB[G::kDmaB], offA[G::kDmaA];
#pragma unroll
  for (int i = 0; i < G::kDmaB; i++) offB[i] = (uint32_t)(((i * 16 + drow) * (size_t)N + dchunk * 8) * 2);
#pragma unroll
  for (int i = 0; i < G::kDmaA; i++) offA[i] = (uint32_t)(((i * 16 + drow) * (size_t)K + dchunk * 8) * 2);
  const uint32_t wbase = lds_addr32(lds) + wave * G::kWaveBytes;

  auto issue = [&](int stage, int step) {
    const uint32_t s = wbase + stage * G::kStageBytes;
    const size_t kb = (size_t)step * kKStep;
#pragma unroll
    for (int i = 0; i < G::kDmaB; i++) dma16(gB + kb * N * 2, offB[i], s + i * 1024);
#pragma unroll
    for (int i = 0; i < G::kDmaA; i++) dma16(gA + kb * 2, offA[i], s + G::kBBytes + i * 1024);
  };

  // Fragment addresses inside a stage.
  // B (16x16x32 B operand): lane 16g + 4jj + q names row 8*(g/2)... for the
  // 16-column block c: rows 8*(lane/16) + 4h + jj, columns 16c + 4q..+3.
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  const uint32_t boff = (uint32_t)((8 * g + jj) * 64 + (4 * q) * 2);
  // A (16x16x32 A operand): lane l holds A[l%16][8*(l/16) .. +7] = row l%16,
  // 16-byte chunk l/16 of that row.
  const uint32_t aoff = (uint32_t)(G::kBBytes + (lane & 15) * 64 + (lane >> 4) * 16);

  float4v acc[MB][2];
#pragma unroll
  for (int r = 0; r < MB; r++)
#pragma unroll
    for (int c = 0; c < 2; c++) acc[r][c] = float4v{0.f, 0.f, 0.f, 0.f};

  // Prologue: kStages-1 steps in flight (clamped: a short k range re-reads
  // its last step into buffers that are never consumed).
#pragma unroll
  for (int s = 0; s < G::kStages - 1; s++) issue(s, min(s, nsteps - 1));

  for (int step = 0; step < nsteps; step++) {
    const int stage = step % G::kStages;
    // Refill the stage consumed in the previous iteration (this wave alone
    // reads its ring, and its reads of that stage completed: lgkmcnt below).
    issue((step + G::kStages - 1) % G::kStages, min(step + G::kStages - 1, nsteps - 1));
    wait_vmcnt<(G::kStages - 1) * G::kDmaPerStage>();  // step `step` has landed
    const uint32_t s = wbase + stage * G::kStageBytes;
    half8 b[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const uint32_t p = s + boff + c * 32;
      const half4 lo = lds_read_tr16_at(p);
      const half4 hi = lds_read_tr16_at(p + 4 * 64);
      b[c] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int r = 0; r < MB; r++) {
      const half8 a = *reinterpret_cast<const __attribute__((address_space(3))) half8*>(s + aoff + r * 1024);
#pragma unroll
      for (int c = 0; c < 2; c++) acc[r][c] = mfma16x16x32(a, b[c], acc[r][c]);
    }
    // All reads of this stage must complete before a later iteration's DMA
    // refills it.
    wait_lgkmcnt0();
  }
  wait_vmcnt<0>();  // clamped tail refills

  // Cross-wave reduction through LDS (the rings are dead now): each wave
  // stores its MB x 16 x 32 partial block; then all 256 threads sum the four
  // partials of one output element in wave order and store it.
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
  const int pitch = kCols;  // floats per row
#pragma unroll
  for (int r = 0; r < MB; r++)
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        // 16x16x32 D layout: lane l, register e -> row 4*(l/16) + e, column l%16
        const int row = r * 16 + 4 * (lane >> 4) + e;
        const int col = c * 16 + (lane & 15);
        red[(wave * 16 * MB + row) * pitch + col] = acc[r][c][e];
      }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 16 * MB * kCols; idx += 256) {
    const int row = idx / kCols, col = idx % kCols;
    float v = red[row * pitch + col];
#pragma unroll
    for (int w = 1; w < kWaves; w++) v += red[(w * 16 * MB + row) * pitch + col];
    if (row < M) C[(size_t)row * N + n0 + col] = convert_out<OutT>(v);
  }
}

template <int MB, typename OutT>
hipError_t launch_skinny_t(const GemmArgs& a) {
  using G = SkinnyCfg<MB>;
  static std::atomic<uint64_t> done{0};
  auto kfn = f16_skinny_kernel<MB, OutT>;
  hipError_t e = ensure_lds_attr(kfn, G::kLdsBytes, a.device, done);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kfn, dim3((unsigned)(a.n / kCols)), dim3(256), G::kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B),
                     static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

template <int MB>
hipError_t launch_mb(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_skinny_t<MB, half_t>(a) : launch_skinny_t<MB, float>(a);
}

hipError_t launch_skinny(const GemmArgs& a) {
  switch ((a.m + 15) / 16) {
    case 1: return launch_mb<1>(a);
    case 2: return launch_mb<2>(a);
    case 3: return launch_mb<3>(a);
    default: return launch_mb<4>(a);
  }
}

// M a multiple of 16 up to 64; N a multiple of 32; K a multiple of 128 (4
// waves x 32); the per-lane 32-bit byte offsets (up to 64 rows of A, 32 rows
// of B) must not overflow.
bool skinny_shape_ok(size_t m, size_t n, size_t k) {
  return m >= 16 && m <= 64 && (size_t)64 * k * 2 < (1ull << 31) && (size_t)32 * n * 2 < (1ull << 31) &&
         n / kCols < (1ull << 31);
}

}  // namespace

void register_f16_skinny() {
  KernelEntry e{};
  e.version = 4;
  e.in_dtype = VK_DTYPE_F16;
  e.name = "f16_v4_skinny_m64";
  e.caps = make_caps(4, VK_DTYPE_F16, kOutF16 | kOutF32, 16, kCols, kWaves * kKStep, 16, 64, kCols,
                     kKStep, 256, SkinnyCfg<4>::kLdsBytes, 0, 0, 64);
  e.launch = launch_skinny;
  e.workspace = nullptr;
  e.shape_ok = skinny_shape_ok;
  register_kernel(e);
}

}  // namespace vk
