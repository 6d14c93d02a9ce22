// f16_skinny_sk.hip -- fp16 GEMM for skinny A (decode-like: M <= 64), version 8:
// split-K over workgroups with a deterministic in-kernel reduction.
//
// Same job as version 4 (f16_skinny.hip); the reference has no path for this
// shape (results/ralph_loop_fable/src/matmul_f16/matmul_f16_v42_shfl2.cu:124,
// :520-527).  At M = 16, N = K = 8192 the GEMM streams 128 MiB of B once: the
// bound is HBM bandwidth.  Measured on MI355X with a streaming-read kernel
// (direct-to-LDS loads of all of an 8192 x 8192 fp16 B, no compute): a
// workgroup that owns a 64-byte column strip of B reaches 3.5 TB/s, a 128-byte
// strip 6.4 TB/s, 256-byte strips with K split over 4 workgroups 6.7 TB/s.
// Version 4 owns 64-byte strips.  Here:
//  * a workgroup owns NC = 128 columns (256-byte rows of B; the kernel is
//    written for NC = 256 as well) and 1/KS of K; grid = (N / NC) x KS with
//    KS the power of two that brings the grid to 256 workgroups (KS = 4 at
//    N = 8192);
//  * 4 waves; per 32-deep k-step each wave loads 8 rows of B (direct-to-LDS,
//    1 KB per instruction) and waves 0..MB-1 one 16-row block of A; a ring of
//    up to 8 stages (7 k-steps of B in flight), one barrier per k-step;
//  * wave w computes columns w*NC/4 .. of the block (NC/64 blocks of 16) for
//    all M rows with v_mfma_f32_16x16x32_f16 (A with ds_read_b128, B with the
//    transpose read);
//  * each workgroup writes its fp32 partial (M x NC) to the workspace; the
//    last of the KS workgroups of a column block (a counter in the
//    workspace, device-scope atomic after the partials are complete) sums the
//    KS partials in k order -- the same order whichever workgroup arrives
//    last, so results are bit-reproducible -- writes C and resets the counter.
//  * workgroup b computes k part b % KS of column block b / KS, so the KS
//    parts of a column block run on KS different XCDs (workgroup b runs on
//    XCD b % 8).  Measured against dealing each XCD a contiguous run of
//    column blocks (all KS parts of a block on one XCD): 24.8 vs 25.3 us per
//    launch at 16 x 8192 x 8192.  Per-workgroup timelines show the XCDs
//    themselves streaming at different rates (the slowest ~1.3x the fastest
//    under either dealing), which is what keeps the kernel at ~0.8 of the
//    streaming limit: the last workgroups end ~4 us after the mean.
#include "vk_device.hpp"
#include "vk_internal.hpp"
#include "vk_tile.hpp"

#include <atomic>
#include <type_traits>

namespace vk {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kKStep = 32;     // k per stage (one 16x16x32 MFMA deep)

template <int NC, int MB>  // NC columns per workgroup, M <= 16 * MB rows
struct SkCfg {
  static constexpr int kChunks = NC / 8;                        // 16-byte chunks per B row
  static constexpr int kRowsPerDma = 1024 / (NC * 2);           // B rows per 1 KB load
  static constexpr int kBDma = 8 / kRowsPerDma;                 // B loads per wave per k-step
  static constexpr int kBStageBytes = kKStep * NC * 2;          // 8 or 16 KB
  static constexpr int kAStageBytes = 16 * MB * kKStep * 2;     // MB KB: rows x 64 B
  static constexpr int kStageBytes = kBStageBytes + kAStageBytes;
  static constexpr int kStages = (159 * 1024) / kStageBytes < 8 ? (159 * 1024) / kStageBytes : 8;
  static constexpr int kLdsBytes = kStages * kStageBytes;
  static constexpr int kWaveCols = NC / kWaves;                 // 32 or 64
  static constexpr int kColBlocks = kWaveCols / 16;             // per wave
  static_assert(kStages >= 4, "pipeline depth");
  static_assert((kStages - 1) * (kBDma + 1) <= 63, "vmcnt range");
};

// Swizzles (physical chunk = logical chunk ^ f(row)), applied by choosing
// which global chunk each lane of a direct-to-LDS load fetches.
// B rows of 16 chunks (NC = 128): a transpose read names 4 k-rows x 2 chunks
// per 16 lanes and 2 such groups 8 k-rows apart per 32 lanes; 2*(k%4) ^
// 8*bit3(k) puts them on 16 distinct 16-byte slots.  Rows of 32 chunks
// (NC = 256): {0, 6, 12, 10}[k % 4] ^ 2*bit3(k), as the 256-column tiles.
template <int NC>
__host__ __device__ constexpr int swz_bk(int krow) {
  return NC == 128 ? (2 * (krow & 3)) ^ (((krow >> 3) & 1) << 3) : swz_b(krow) ^ (((krow >> 3) & 1) << 1);
}
// A rows are 64 B = 4 chunks; a fragment read names 16 rows x 1 chunk per 16
// lanes; chunk ^ (row/4)%4 spreads them over 16 slots.
__host__ __device__ constexpr int swz_a64(int row) { return (row >> 2) & 3; }

// 128-column blocks: measured at 16 x 8192 x 8192, NC = 128 with K split 4
// ways took 24.3 us, NC = 256 with K split 8 ways 28.1 us (the larger
// k-split costs more in the final reduction than the wider rows gain).
int pick_nc(size_t) { return 128; }

// Number of workgroups sharing a column block's K range: a power of two up
// to 8 that brings the grid to 256 and divides K into 32-deep steps.
int pick_ks(size_t n, size_t k) {
  const size_t ncb = n / pick_nc(n);
  int ks = 1;
  while (ks < 8 && ncb * ks < 256 && k % ((size_t)kKStep * ks * 2) == 0) ks *= 2;
  return ks;
}

template <int NC, int MB, typename OutT>
__global__ __launch_bounds__(kThreads, 1) void f16_skinny_sk_kernel(const half_t* __restrict__ A,
                                                                    const half_t* __restrict__ B,
                                                                    OutT* __restrict__ C, int M, int N, int K,
                                                                    int ks_count, float* __restrict__ part,
                                                                    unsigned* __restrict__ counters) {
  using G = SkCfg<NC, MB>;
  constexpr int S = G::kStages;
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const int cid = blockIdx.x;
  const int cb = cid / ks_count, kp = cid - cb * ks_count;
  const int n0 = cb * NC;
  const int kc = K / ks_count;  // k rows of this workgroup
  const int kbeg = kp * kc;
  const int nsteps = kc / kKStep;

  // Direct-to-LDS duty per k-step.  B: load i covers k-rows 8w + i*R .. +R-1
  // (R = 1024 / (2 NC) rows of NC/8 chunks; lane l: row l / (NC/8), slot
  // l % (NC/8)).  A: wave w < MB covers rows 16w .. 16w+15 (4 chunks each;
  // lane l: row l/4, slot l%4).
  uint32_t offB[G::kBDma];
#pragma unroll
  for (int i = 0; i < G::kBDma; i++) {
    const int krow = 8 * wave + i * G::kRowsPerDma + lane / G::kChunks;
    const int c = (lane % G::kChunks) ^ swz_bk<NC>(krow);
    offB[i] = (uint32_t)(((size_t)krow * N + c * 8) * 2);
  }
  const int arow = 16 * wave + (lane >> 2);
  const uint32_t offA = (uint32_t)(((size_t)arow * K + (((lane & 3) ^ swz_a64(arow)) * 8)) * 2);
  const char* gB = reinterpret_cast<const char*>(B) + ((size_t)kbeg * N + n0) * 2;
  const char* gA = reinterpret_cast<const char*>(A) + (size_t)kbeg * 2;
  const uint32_t lbase = lds_addr32(lds);
  const bool loads_a = wave < MB;

  auto issue = [&](int stage, int step) {
    const uint32_t s = lbase + stage * G::kStageBytes;
    const size_t kb = (size_t)step * kKStep;
#pragma unroll
    for (int i = 0; i < G::kBDma; i++) dma16(gB + kb * N * 2, offB[i], s + (8 * wave + i * G::kRowsPerDma) * NC * 2);
    if (loads_a) dma16(gA + kb * 2, offA, s + G::kBStageBytes + wave * 1024);
  };

  // Fragment addresses inside a stage.
  // B (MFMA B operand, 16x16x32): lane 16g + 4jj + q names k-row
  // 8g + 4h + jj, columns w*NC/4 + 16c + 4q .. +3; the transpose read hands
  // lane 16g + i the 4 k of column 16c + i.
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  const int krow0 = 8 * g + jj;  // plus 4h: bits 0, 1, 3 unchanged
  uint32_t boff[G::kColBlocks];
#pragma unroll
  for (int c = 0; c < G::kColBlocks; c++) {
    const int chunk = (G::kWaveCols / 8) * wave + 2 * c + (q >> 1);
    boff[c] = (uint32_t)(krow0 * NC * 2 + 16 * (chunk ^ swz_bk<NC>(krow0)) + 8 * (q & 1));
  }
  // A (MFMA A operand): lane l holds A[l%16][8*(l/16) .. +7]: row l%16,
  // chunk l/16 of that row.
  const int ar = lane & 15;
  const uint32_t aoff = (uint32_t)(G::kBStageBytes + ar * 64 + 16 * ((lane >> 4) ^ swz_a64(ar)));

  float4v acc[MB][G::kColBlocks];
#pragma unroll
  for (int r = 0; r < MB; r++)
#pragma unroll
    for (int c = 0; c < G::kColBlocks; c++) acc[r][c] = float4v{0.f, 0.f, 0.f, 0.f};

  // Prologue: S-1 steps in flight (clamped refills of a short k range land in
  // stages that are never read).
#pragma unroll
  for (int st = 0; st < S - 1; st++) issue(st, min(st, nsteps - 1));

  for (int step = 0; step < nsteps; step++) {
    const int stage = step % S;
    // This wave's loads of `step` landed, then everyone's (barrier); the
    // barrier also ends every wave's reads of the previous stage.
    if (loads_a)
      wait_vmcnt<(S - 2) * (G::kBDma + 1)>();
    else
      wait_vmcnt<(S - 2) * G::kBDma>();
    lds_barrier();
    issue((step + S - 1) % S, min(step + S - 1, nsteps - 1));
    const uint32_t sb = lbase + stage * G::kStageBytes;
    half8 b[G::kColBlocks];
#pragma unroll
    for (int c = 0; c < G::kColBlocks; c++) {
      const half4 lo = lds_read_tr16_at(sb + boff[c]);
      const half4 hi = lds_read_tr16_at(sb + boff[c] + 4 * NC * 2);
      b[c] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int r = 0; r < MB; r++) {
      const half8 a = lds_read_h8(sb + aoff + r * 1024);
#pragma unroll
      for (int c = 0; c < G::kColBlocks; c++) acc[r][c] = mfma16x16x32(a, b[c], acc[r][c]);
    }
  }
  wait_vmcnt<0>();  // clamped tail refills

  // Partial of this workgroup: part[(cb * KS + kp)][16*MB rows][NC cols].
  // D layout: lane l, register e -> row 4*(l/16) + e, column l%16 of the block.
  //
  // Cross-workgroup hand-off without a cache write-back: the partials are
  // written and read with agent-scope coherent accesses (relaxed atomic
  // stores and loads: global_store/global_load with sc1, which do not stay
  // dirty in, or get served stale from, an XCD's own L2), and each wave
  // waits until its stores have completed (vmcnt(0)) before the counter is
  // incremented.  A __threadfence() would do the same by writing back the
  // whole L2 of the XCD, which measured ~25 us per launch with 256
  // workgroups fencing.
  const size_t pstride = (size_t)16 * MB * NC;
  float* mine = part + ((size_t)cb * ks_count + kp) * pstride;
#pragma unroll
  for (int r = 0; r < MB; r++)
#pragma unroll
    for (int c = 0; c < G::kColBlocks; c++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        __hip_atomic_store(&mine[(size_t)(16 * r + 4 * (lane >> 4) + e) * NC + G::kWaveCols * wave + 16 * c + (lane & 15)],
                           acc[r][c][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  wait_vmcnt0_ordered();  // every wave's partial is in memory before the barrier and the counter

  // The last arrival of the column block reduces.
  __shared__ int s_last;
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(&counters[cb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (unsigned)(ks_count - 1);
  __syncthreads();
  if (!s_last) return;
  // Thread t owns column t % NC of rows t / NC, + RS, ..; loads are issued in
  // batches of up to 64 before their (k-ordered) sums.
  constexpr int RS = kThreads / NC;   // row step
  constexpr int RPT = 16 * MB / RS;   // rows per thread
  const float* col0 = part + (size_t)cb * ks_count * pstride;
  const int col = threadIdx.x % NC;
  const int r0 = threadIdx.x / NC;
  auto reduce = [&](auto nparts) {
    constexpr int P = decltype(nparts)::value;
    // rows per batch: the largest power of two that divides RPT, at most 64 / P
    constexpr int RP2 = RPT & -RPT;
    constexpr int RB = (64 / P < RP2) ? 64 / P : RP2;
    static_assert(RPT % RB == 0, "row batches");
#pragma unroll
    for (int b0 = 0; b0 < RPT; b0 += RB) {
      float x[P][RB];
#pragma unroll
      for (int p = 0; p < P; p++)
#pragma unroll
        for (int i = 0; i < RB; i++)
          x[p][i] = __hip_atomic_load(&col0[(size_t)p * pstride + (size_t)(r0 + RS * (b0 + i)) * NC + col],
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int i = 0; i < RB; i++) {
        float v = 0.0f;
#pragma unroll
        for (int p = 0; p < P; p++) v += x[p][i];
        const int row = r0 + RS * (b0 + i);
        if (row < M) C[(size_t)row * N + n0 + col] = convert_out<OutT>(v);
      }
    }
  };
  switch (ks_count) {
    case 1: reduce(std::integral_constant<int, 1>{}); break;
    case 2: reduce(std::integral_constant<int, 2>{}); break;
    case 4: reduce(std::integral_constant<int, 4>{}); break;
    default: reduce(std::integral_constant<int, 8>{}); break;
  }
  // Every part has arrived: reset for the next call.
  if (threadIdx.x == 0) __hip_atomic_store(&counters[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t sk_counter_bytes(size_t n) { return ((n / 128) * sizeof(unsigned) + 255) & ~(size_t)255; }

size_t sk_workspace(size_t m, size_t n, size_t k, int) {
  const int mb = (int)((m + 15) / 16);
  return sk_counter_bytes(n) + (size_t)pick_ks(n, k) * n * 16 * mb * sizeof(float);
}

template <int NC, int MB, typename OutT>
hipError_t launch_sk_t(const GemmArgs& a) {
  using G = SkCfg<NC, MB>;
  static std::atomic<uint64_t> done{0};
  auto kfn = f16_skinny_sk_kernel<NC, MB, OutT>;
  hipError_t e = ensure_lds_attr(kfn, G::kLdsBytes, a.device, done);
  if (e != hipSuccess) return e;
  const int ks = pick_ks(a.n, a.k);
  unsigned* counters = static_cast<unsigned*>(a.workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + sk_counter_bytes(a.n));
  if (!a.workspace_clean) {
    e = zero_words(counters, sk_counter_bytes(a.n) / 4, a.stream);
    if (e != hipSuccess) return e;
  }
  const unsigned grid = (unsigned)((a.n / NC) * ks);
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kThreads), G::kLdsBytes, a.stream, static_cast<const half_t*>(a.A),
                     static_cast<const half_t*>(a.B), static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k, ks,
                     part, counters);
  return hipGetLastError();
}

template <int NC, int MB>
hipError_t launch_mb(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_sk_t<NC, MB, half_t>(a) : launch_sk_t<NC, MB, float>(a);
}

template <int NC>
hipError_t launch_nc(const GemmArgs& a) {
  switch ((a.m + 15) / 16) {
    case 1: return launch_mb<NC, 1>(a);
    case 2: return launch_mb<NC, 2>(a);
    case 3: return launch_mb<NC, 3>(a);
    default: return launch_mb<NC, 4>(a);
  }
}

hipError_t launch_sk(const GemmArgs& a) { return launch_nc<128>(a); }

// M a multiple of 16 up to 64; N a multiple of 128; K a multiple of 32; the
// per-lane 32-bit byte offsets (up to 64 rows of A, 32 rows of B) must not
// overflow.
bool sk_shape_ok(size_t m, size_t n, size_t k) {
  return m >= 16 && m <= 64 && (size_t)64 * k * 2 < (1ull << 31) && (size_t)32 * n * 2 < (1ull << 31) &&
         (n / 128) * 8 < (1ull << 31);
}

}  // namespace

void register_f16_skinny_sk() {
  KernelEntry e{};
  e.version = 8;
  e.in_dtype = VK_DTYPE_F16;
  e.name = "f16_v8_skinny_splitk";
  e.caps = make_caps(8, VK_DTYPE_F16, kOutF16 | kOutF32, 16, 128, kKStep, 16, 64, 128, kKStep, kThreads,
                     SkCfg<128, 4>::kLdsBytes, 0, 1, 64);
  e.launch = launch_sk;
  e.workspace = sk_workspace;
  e.shape_ok = sk_shape_ok;
  register_kernel(e);
}

}  // namespace vk
