// f16_skinny_wk.hip -- fp16 GEMM for skinny A (batched decode: M <= 128),
// version 14: K split over the waves of a workgroup and over workgroups.
//
// Same job as version 8 (f16_skinny_sk.hip); the reference has no path for
// this shape (results/ralph_loop_fable/src/matmul_f16/matmul_f16_v42_shfl2.cu:124,
// :520-527).  Version 8 gives each of a workgroup's 4 waves a share of the
// outputs over the workgroup's whole k range, so every wave reads the A
// fragments of every k-step from LDS; at M = 128 that LDS read traffic bounds
// its k-loop (per-workgroup timelines: 23.9 us of k-loop where the B stream
// alone takes ~20), and 4 k pieces per column block hand 12 MB of fp32
// partials from workgroup to workgroup at N = K = 8192.  Here:
//  * a workgroup owns NC = 64 columns (128-byte rows of B) and 1/ks of K
//    (pieces of whole 32-deep steps); grid = ceil(N / 64) x ks, ks a power
//    of two up to 8 that keeps one workgroup per CU, or more where that
//    fills idle CUs with pieces of at least 32 steps (ks = 2 at N = 8192 on
//    256 CUs: the partials are 4 MB; 3 at N = 5120, K = 4096: 80 column
//    blocks x 3 on 240 CUs);
//  * wave w computes the workgroup's whole M x 64 block over k-steps (32
//    deep) w, w + 4, w + 8, ... of the workgroup's range, on its own: its
//    own loads, its own LDS ring, no barrier in the k-loop.  Every byte of A
//    and B is used by exactly one wave, so A goes from memory (L2: all column
//    blocks read the same 2 MB) straight into registers as MFMA A fragments
//    (16 rows x 64 bytes per load), and only B, which the MFMA needs
//    transposed, goes through LDS (direct-to-LDS, 4 KB per k-step, read with
//    the transpose read);
//  * loads run D k-steps ahead in the wave (D = 7 up to 64 rows, 3 above,
//    over rings of D + 1 A fragment buffers in registers and B stages in
//    LDS), all on the in-order vmcnt, waited for with constant counts;
//  * a wave's step count is padded to a multiple of D + 1 with steps whose
//    loads lie past the ends of buffer resources sized to A and B (zeros,
//    no memory touched), so the loop has no remainder (a remainder's second
//    copy of the body cost the 128-row instance ~330 register moves per
//    ring); their products add +0.0 to accumulators that started at +0.0,
//    which leaves them unchanged;
//  * after the k-loop the 4 waves' M x 64 fp32 sums meet in LDS, and wave q
//    adds column block q of the 4 in wave order;
//  * with K split over workgroups, wave q of each piece hands its M x 16
//    block off as version 8 does (per-(column block, wave) counter; the last
//    arrival sums the pieces in k order, its own from registers), so C does
//    not depend on the arrival order.
// Each output is the sum over its k-steps in the fixed order: steps of wave
// 0, 1, 2, 3 (each ascending) within a piece, then the pieces ascending.
#include "vk_device.hpp"
#include "vk_internal.hpp"
#include "vk_tile.hpp"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace vk {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kKStep = 32;                 // k per step (one 16x16x32 MFMA deep)
constexpr int kMaxRows = 128;
constexpr int kNC = 64;                    // columns per workgroup
constexpr size_t kCounterBytes = 4096;     // (column block, wave) counters
constexpr int kMaxPieces = 8;              // K pieces per column block

// MB 16-row blocks.
template <int MB>
struct WkCfg {
  static constexpr int kCB = kNC / 16;                   // 16-column blocks (one per wave in the reduction)
  static constexpr int kChunks = kNC / 8;                // 16-byte chunks per B row
  static constexpr int kRowsPerLoad = 1024 / (kNC * 2);  // B rows per 1 KB direct-to-LDS load
  static constexpr int kBLoads = kKStep / kRowsPerLoad;  // per step
  static constexpr int kBStage = kKStep * kNC * 2;       // 4 KB
  static constexpr int kD = MB <= 4 ? 7 : 3;             // loads run kD steps ahead
  static constexpr int kS = kD + 1;                      // B stages and A buffers per wave
  static constexpr int kL = kBLoads + MB;                // loads per step
  static_assert(kD * kL <= 63, "vmcnt range");
  static_assert(kCB == kWaves, "each wave sums one column block");
  static constexpr int kRing = kWaves * kS * kBStage;    // k-loop LDS
  static constexpr int kRegion = MB * kCB * 1024;        // a wave's sums in the reduction
  static constexpr int kRed = kWaves * kRegion;
  static constexpr int kLdsBytes = kRing > kRed ? kRing : kRed;
};

// Swizzle of the B stage rows (physical chunk = logical chunk ^ f(k-row)),
// applied by choosing which global chunk each lane of a direct-to-LDS load
// fetches.  A transpose read names, per 32 lanes, k-rows {0,1,2,3,8,9,10,11}
// (+4 for the upper half) x 2 chunks; the 128-byte rows alternate between
// the two halves of the 256-byte bank line, and chunk ^ (2 bit1(k) ^
// 4 bit3(k)) puts each half's 4 rows x 2 chunks on 8 distinct 16-byte slots.
// Bit 2 of k is not used, so the upper half's rows share their swizzle with
// the lower half's.
__host__ __device__ constexpr int swz_wk(int krow) { return (((krow >> 1) & 1) << 1) ^ (((krow >> 3) & 1) << 2); }

// 16 bytes per lane from a buffer resource into registers, untracked by the
// compiler (inline asm): it would otherwise wait for every older load,
// direct-to-LDS ones included, before the first use.  Callers wait with
// wait_vmcnt before the result is used.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ half8 buf_load_h8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  half8 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(r), "s"(soff));
  return v;
}
#pragma clang diagnostic pop

// s_waitcnt with only an lgkmcnt limit (vmcnt and expcnt at their maxima).
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __builtin_amdgcn_s_waitcnt(0xc07f | (N << 8));
}

template <int MB, typename OutT>
__global__ __launch_bounds__(kThreads, 1) void f16_skinny_wk_kernel(const half_t* __restrict__ A,
                                                                    const half_t* __restrict__ B,
                                                                    OutT* __restrict__ C, int M, int N, int K,
                                                                    int ks_count, float* __restrict__ part,
                                                                    unsigned* __restrict__ counters) {
  using G = WkCfg<MB>;
  constexpr int D = G::kD, S = G::kS, L = G::kL, kCB = G::kCB, kBStage = G::kBStage;
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  prefer_agpr_accumulators();

  const int cb = blockIdx.x / ks_count, kp = blockIdx.x - cb * ks_count;
  const int n0 = cb * kNC;
  // Piece kp of the K / 32 steps: steps floor(kp T / ks) .. floor((kp + 1) T / ks) - 1.
  const int tsteps = K / kKStep;
  const int sbeg = (int)((long long)kp * tsteps / ks_count);
  const int kbeg = sbeg * kKStep;
  const int nsteps = (int)((long long)(kp + 1) * tsteps / ks_count) - sbeg;  // k-steps of this workgroup
  const int ns = nsteps > wave ? (nsteps - wave + kWaves - 1) / kWaves : 0;  // this wave's steps
  const int ns_pad = (ns + S - 1) / S * S;  // plus steps of zeros
  const uint32_t lbase = lds_addr32(lds);
  const uint32_t wring = lbase + (uint32_t)(wave * S * kBStage);

  // B: load i of a step covers k-rows 8i + l / 8 (8 rows of 8 chunks); lane
  // l lands at chunk slot l % 8 and fetches chunk (l % 8) ^ swz(row),
  // through a buffer resource over the K x N matrix.  In a last column block
  // that N cuts short (N a multiple of 8) a chunk past N is replaced by the
  // block's last valid chunk of the same row: valid memory, and the columns
  // past N are never stored.
  const int cvalid = min(kNC, N - n0) / 8;
  uint32_t offB[G::kBLoads];
#pragma unroll
  for (int i = 0; i < G::kBLoads; i++) {
    const int krow = G::kRowsPerLoad * i + lane / G::kChunks;
    const int c = min((lane % G::kChunks) ^ swz_wk(krow), cvalid - 1);
    offB[i] = (uint32_t)(((size_t)krow * N + c * 8) * 2);
  }
  const uint32_t b_end = (uint32_t)K * (uint32_t)N * 2u;
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(B), 0, (int)b_end, kBufferWord3);
  const uint32_t b0 = ((uint32_t)(kbeg + wave * kKStep) * (uint32_t)N + (uint32_t)n0) * 2u;  // this wave's first step
  const uint32_t bstep = (uint32_t)(kWaves * kKStep) * (uint32_t)N * 2u;  // between this wave's steps

  // A: fragment r of a step is rows 16r .. 16r + 15, lane l holding row
  // 16r + l % 16, k 8(l / 16) .. +7 of the step (the MFMA A layout); a row
  // past M reads row M - 1 (its products land in rows that are never stored).
  const uint32_t a_end = (uint32_t)M * (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(A), 0, (int)a_end, kBufferWord3);
  uint32_t offA[MB];
#pragma unroll
  for (int r = 0; r < MB; r++)
    offA[r] = (uint32_t)(min(16 * r + (lane & 15), M - 1)) * (uint32_t)K * 2u + (uint32_t)(lane >> 4) * 16u;
  const uint32_t a0 = (uint32_t)(kbeg + wave * kKStep) * 2u;  // byte offset of this wave's first step
  const uint32_t astep = (uint32_t)(kWaves * kKStep) * 2u;

  // Transpose reads of B: lane (g = l/16, jj = (l/4)%4, q = l%4) names k-row
  // 8g + jj (and + 4), columns 16c + 4q .. +3 = chunk 2c + q/2, bytes 8(q%2).
  const int krow0 = 8 * (lane >> 4) + ((lane >> 2) & 3);
  uint32_t boff[kCB];
#pragma unroll
  for (int c = 0; c < kCB; c++) {
    const int chunk = 2 * c + ((lane & 3) >> 1);
    boff[c] = wring + (uint32_t)(krow0 * kNC * 2 + 16 * (chunk ^ swz_wk(krow0)) + 8 * (lane & 1));
  }

  float4v acc[MB][kCB];
#pragma unroll
  for (int r = 0; r < MB; r++)
#pragma unroll
    for (int c = 0; c < kCB; c++) acc[r][c] = float4v{0.f, 0.f, 0.f, 0.f};

  half8 abuf[S][MB];   // A fragments of the steps in flight
  half8 bfr[kCB];      // B fragments of the current step

  // Loads of this wave's step j into stage and buffer SL; a step past the
  // wave's last (padding, or prefetch past the end) reads zeros from past
  // the resources' ends.
  auto issue = [&](auto slot, int j) {
    constexpr int SL = decltype(slot)::value;
    const bool live = j < ns;
    const uint32_t sb = live ? b0 + (uint32_t)j * bstep : b_end;
#pragma unroll
    for (int i = 0; i < G::kBLoads; i++) dma16_buf(brs, offB[i], sb, wring + SL * kBStage + i * 1024);
    const uint32_t sa = live ? a0 + (uint32_t)j * astep : a_end;
#pragma unroll
    for (int r = 0; r < MB; r++) abuf[SL][r] = buf_load_h8(ars, offA[r], sa);
  };
  auto read_b = [&](auto slot) {
    constexpr int SL = decltype(slot)::value;
    static_for<kCB>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      const half4 lo = lds_read_tr16_off<SL * kBStage>(boff[c]);
      const half4 hi = lds_read_tr16_off<SL * kBStage + 4 * kNC * 2>(boff[c]);
      bfr[c] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    });
  };

  if (ns_pad > 0) {
    static_for<D>([&](auto u) { issue(u, decltype(u)::value); });
    // Step j = j0 + u: stage and buffer u (j0 is a multiple of S).  The
    // step's fragment reads wait for their data (a few hundred cycles, where
    // a step of this memory-bound loop takes thousands); the loads of step
    // j + D go into the stage and buffer step j - 1 used, whose reads and
    // MFMAs are done.
    auto step = [&](auto uu, int j0) {
      constexpr int u = decltype(uu)::value;
      wait_vmcnt<(D - 1) * L>();  // step j landed (j + 1 .. j + D - 1 may be in flight)
      __builtin_amdgcn_sched_barrier(0);
      read_b(std::integral_constant<int, u>{});
      issue(std::integral_constant<int, (u + D) % S>{}, j0 + u + D);
      wait_lgkmcnt<0>();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 0; r < MB; r++)
#pragma unroll
        for (int c = 0; c < kCB; c++) acc[r][c] = mfma16x16x32(abuf[u][r], bfr[c], acc[r][c]);
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int j0 = 0; j0 < ns_pad; j0 += S) static_for<S>([&](auto uu) { step(uu, j0); });
    // The loads past the last step are never used, but land after their
    // instructions: their registers stay allocated (used below) until the
    // counter is drained.
    wait_vmcnt<0>();
#pragma unroll
    for (int sl = 0; sl < S; sl++)
#pragma unroll
      for (int r = 0; r < MB; r++) asm volatile("" ::"v"(abuf[sl][r]));
  }

  // The 4 waves' sums meet in LDS (the ring is free once every wave is past
  // its k-loop): wave w's block (r, c) at w * MB * 4 KB + (4r + c) KB, lane
  // l's 16 bytes at 16 l; wave q adds column block q of the 4, in wave order.
  float4v red[MB];
  lds_barrier();
#pragma unroll
  for (int r = 0; r < MB; r++)
#pragma unroll
    for (int c = 0; c < kCB; c++)
      lds_write16(lbase + wave * G::kRegion + (uint32_t)(r * kCB + c) * 1024 + lane * 16, acc[r][c]);
  lds_barrier();
#pragma unroll
  for (int r = 0; r < MB; r++) {
    const uint32_t at = lbase + (uint32_t)(r * kCB + wave) * 1024 + lane * 16;
    float4v t = __builtin_bit_cast(float4v, lds_read16(at));
#pragma unroll
    for (int w = 1; w < kWaves; w++) t += __builtin_bit_cast(float4v, lds_read16(at + w * G::kRegion));
    red[r] = t;
  }

  // Block (r, wave): lane l, register e -> row 16r + 4(l/16) + e, column
  // n0 + 16 wave + l % 16.
  const int col = n0 + 16 * wave + (lane & 15);
  const int rq = 4 * (lane >> 4);
  auto store_c = [&](int r, const float4v& v) {
    if (col >= N) return;  // past N (a last column block cut short)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int row = 16 * r + rq + e;
      if (row < M) C[(size_t)row * N + col] = convert_out<OutT>(v[e]);
    }
  };
  constexpr int NB = MB;  // blocks of this wave
  if (ks_count == 1) {
#pragma unroll
    for (int r = 0; r < MB; r++) store_c(r, red[r]);
    return;
  }

  // K split over workgroups.  Slot (cb, piece q) holds 4 wave regions of NB
  // blocks x 64 lanes x 16 bytes (every access a coalesced 1 KB row).  Wave
  // w of each piece hands off on counter (cb, w): it reads the counter, and
  // if every other piece has arrived it is the last and skips its store;
  // otherwise it stores its partial, waits for the stores and increments the
  // counter.  The last arrival sums the pieces in k order (its own from
  // registers), writes C and resets the counter for the next call.
  constexpr uint32_t kWaveRegion = NB * 1024;
  constexpr uint32_t kSlotBytes = kWaves * kWaveRegion;
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      part, 0, (int)((uint32_t)((N + kNC - 1) / kNC) * (uint32_t)ks_count * kSlotBytes), kBufferWord3);
  auto soff = [&](int q) { return (uint32_t)(cb * ks_count + q) * kSlotBytes + (uint32_t)wave * kWaveRegion; };
  const uint32_t vlane = (uint32_t)lane * 16;
  unsigned* cnt = counters + cb * kWaves + wave;
  const unsigned seen =
      __builtin_amdgcn_readfirstlane(__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  if (seen != (unsigned)(ks_count - 1)) {
#pragma unroll
    for (int b = 0; b < NB; b++) store_partial(prs, vlane + b * 1024, soff(kp), red[b]);
    wait_vmcnt0_ordered();  // the partial is in memory before the counter moves
    unsigned old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_amdgcn_readfirstlane(old) != (unsigned)(ks_count - 1)) return;
  }
  // The counter read that made this wave the last stays before the reads of
  // the other pieces.
  asm volatile("" ::: "memory");
  auto fold = [&](auto nparts) {
    constexpr int P = decltype(nparts)::value;
    constexpr int BB = (32 / P < NB) ? 32 / P : NB;  // blocks per batch: up to 32 loads in flight
#pragma unroll
    for (int b0 = 0; b0 < NB; b0 += BB) {
      float4v x[P][BB];
#pragma unroll
      for (int q = 0; q < P; q++) {
        if (q != kp) {
#pragma unroll
          for (int i = 0; i < BB; i++)
            if (b0 + i < NB) x[q][i] = load_partial(prs, vlane + (b0 + i) * 1024, soff(q));
        } else {
#pragma unroll
          for (int i = 0; i < BB; i++)
            if (b0 + i < NB) x[q][i] = red[b0 + i];
        }
      }
#pragma unroll
      for (int i = 0; i < BB; i++) {
        if (b0 + i < NB) {
          float4v t = x[0][i];
#pragma unroll
          for (int q = 1; q < P; q++) t += x[q][i];
          store_c(b0 + i, t);
        }
      }
    }
  };
  static_assert(kMaxPieces == 8, "one case per piece count");
  switch (ks_count) {
    case 2: fold(std::integral_constant<int, 2>{}); break;
    case 3: fold(std::integral_constant<int, 3>{}); break;
    case 4: fold(std::integral_constant<int, 4>{}); break;
    case 5: fold(std::integral_constant<int, 5>{}); break;
    case 6: fold(std::integral_constant<int, 6>{}); break;
    case 7: fold(std::integral_constant<int, 7>{}); break;
    default: fold(std::integral_constant<int, 8>{}); break;
  }
  if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int wk_mb(size_t m) { return (int)((m + 15) / 16); }

// Workgroups sharing a column block's K range (pieces of K / 32 steps, as
// equal as the steps allow), while the counters fit their 4 KB: the largest
// power of two up to 8 that keeps the grid to one workgroup per CU with at
// least 8 steps per piece (2 per wave); or, where that leaves CUs idle, as
// many as fill them if the pieces keep at least 32 steps.  Measured (us per
// launch, one box, M = 1 / 16 / 64 / 128): 5120 x 4096 in 3 pieces 12.5 /
// 12.5 / 16.8 / 21.6 against 12.7 / 13.2 / 19.4 / 26.7 in 2; 5120 x 8192
// 18.3 / 19.0 / 24.4 / 34.1 against 19.4 / 21.3 / 31.1 / 45.3; but 2560 x
// 4096 in 6 pieces of 21 steps 8.0 / 8.7 / 13.6 / 18.1 against 7.1 / 8.0 /
// 12.6 / 17.9 in 4: short pieces cost more in partials than the CUs gain.
int wk_pick_ks(size_t n, size_t k, int num_cus) {
  const size_t ncb = (n + kNC - 1) / kNC;
  if (ncb == 0 || ncb * kWaves * sizeof(unsigned) > kCounterBytes) return 1;
  const size_t steps = k / kKStep;
  int ks = 1;
  while (ks < kMaxPieces && ncb * ks * 2 <= (size_t)num_cus && steps / (ks * 2) >= 8) ks *= 2;
  const size_t fill = std::min<size_t>(kMaxPieces, (size_t)num_cus / ncb);
  if (fill > (size_t)ks && steps / fill >= 32) ks = (int)fill;
  return ks;
}

// Workspace: the fixed 4 KB of counters (the same place for every shape, so
// the library workspace stays clean from one call to the next), then the
// partials.  Unsplit shapes need none.
size_t wk_workspace(size_t m, size_t n, size_t k, int num_cus) {
  const int ks = wk_pick_ks(n, k, num_cus);
  if (ks == 1) return 0;
  const size_t ncb = (n + kNC - 1) / kNC;
  return kCounterBytes + (size_t)ks * ncb * kWaves * wk_mb(m) * 1024;
}

template <int MB, typename OutT>
hipError_t launch_wk_t(const GemmArgs& a) {
  using G = WkCfg<MB>;
  static std::atomic<uint64_t> done{0};
  auto kfn = f16_skinny_wk_kernel<MB, OutT>;
  hipError_t e = ensure_lds_attr(kfn, G::kLdsBytes, a.device, done);
  if (e != hipSuccess) return e;
  const int ks = wk_pick_ks(a.n, a.k, a.num_cus);
  unsigned* counters = nullptr;
  float* part = nullptr;
  if (ks > 1) {
    if (((a.n + kNC - 1) / kNC) * kWaves * sizeof(unsigned) > kCounterBytes) return hipErrorInvalidValue;
    counters = static_cast<unsigned*>(a.workspace);
    part = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + kCounterBytes);
    if (!a.workspace_clean) {
      e = zero_words(counters, kCounterBytes / 4, a.stream);
      if (e != hipSuccess) return e;
    }
  }
  const unsigned grid = (unsigned)(((a.n + kNC - 1) / kNC) * ks);
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kThreads), G::kLdsBytes, a.stream, static_cast<const half_t*>(a.A),
                     static_cast<const half_t*>(a.B), static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k, ks,
                     part, counters);
  return hipGetLastError();
}

template <int MB>
hipError_t launch_mb(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_wk_t<MB, half_t>(a) : launch_wk_t<MB, float>(a);
}

hipError_t launch_wk(const GemmArgs& a) {
  switch (wk_mb(a.m)) {
    case 1: return launch_mb<1>(a);
    case 2: return launch_mb<2>(a);
    case 3: return launch_mb<3>(a);
    case 4: return launch_mb<4>(a);
    case 5: return launch_mb<5>(a);
    case 6: return launch_mb<6>(a);
    case 7: return launch_mb<7>(a);
    default: return launch_mb<8>(a);
  }
}

// Any M up to 128, N a multiple of 8, K a multiple of 32; the byte sizes of
// A and of B (plus a step of rows: the zero loads start at its end) must fit
// the buffer resources' 31-bit ranges, and so must the partials'.
bool wk_shape_ok(size_t m, size_t n, size_t k) {
  return m >= 1 && m <= kMaxRows && m * k * 2 < (1ull << 31) && (k + kKStep) * n * 2 < (1ull << 31) &&
         ((n + kNC - 1) / kNC) * 8 * kWaves * 8 * 1024 < (1ull << 31);
}

}  // namespace

void register_f16_skinny_wk() {
  KernelEntry e{};
  e.version = 14;
  e.in_dtype = VK_DTYPE_F16;
  e.name = "f16_v14_skinny_wavek";
  e.caps = make_caps(14, VK_DTYPE_F16, kOutF16 | kOutF32, 1, 8, kKStep, 16, kMaxRows, kNC, kKStep, kThreads,
                     WkCfg<8>::kLdsBytes, 0, 1, kMaxRows);
  e.launch = launch_wk;
  e.workspace = wk_workspace;
  e.shape_ok = wk_shape_ok;
  register_kernel(e);
}

}  // namespace vk
