// f16_skinny_sk.hip -- fp16 GEMM for skinny A (decode-like: any M <= 256), version 8:
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
//    written for NC = 256 as well) and 1/KS of K (pieces of whole 32-deep
//    steps); grid = ceil(N / NC) x KS with KS the largest power of two (up
//    to 8) that keeps the grid within one workgroup per CU (KS = 4 at
//    N = 8192 on 256 CUs);
//  * 4 waves; per 32-deep k-step each wave loads 8 rows of B (direct-to-LDS,
//    1 KB per instruction) and wave w the 16-row blocks w and w + 4 of A that
//    exist (MB = M / 16 blocks); a ring of up to 8 stages (6-7 k-steps of B
//    in flight), one barrier per k-step, the fragment reads of one k-step
//    overlapping the MFMAs of the one before;
//  * wave w computes columns w*NC/4 .. of the block (NC/64 blocks of 16) for
//    all M rows with v_mfma_f32_16x16x32_f16 (A with ds_read_b128, B with the
//    transpose read);
//  * each wave writes its fp32 partial (M x NC/4) to the workspace; the last
//    of the KS waves holding the same columns (a counter per column block and
//    wave in the workspace, device-scope atomic after the partial is complete)
//    sums the KS partials in k order -- the same order whichever part arrives
//    last, so results are bit-reproducible -- writes C and resets the counter.
//    At M = 128 one workgroup's partial is 64 KB: the partials are laid out so
//    that every access is a coalesced 1 KB row per wave instruction, and the
//    last arrival keeps its own part in registers.  Measured at
//    128 x 8192 x 8192 against one counter per column block and 4-byte
//    accesses: the reductions at the end of the launch took 3.5-4.7 us
//    instead of 9 us.
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

#include <algorithm>
#include <atomic>
#include <type_traits>

// Timeline build (make timeline -> libvk_gemm_timeline.so, VK_TIMELINE=1):
// wave 0 of each workgroup also records its XCD, its k part and step count,
// and the 100 MHz real-time clock at entry, at the end of its k-loop and when
// it leaves (after its partial's hand-off, or after the sums for the last
// arrival); vk_timeline_sk_read() copies them out.  The product library is
// built with VK_TIMELINE=0 and records nothing.
#ifndef VK_TIMELINE
#define VK_TIMELINE 0
#endif
#if VK_TIMELINE
constexpr int kSkTimelineGroups = 4096;  // workgroups recorded (the first 4096 of a launch)
__device__ unsigned long long vk_timeline_sk[kSkTimelineGroups * 6];
extern "C" int vk_timeline_sk_read(unsigned long long* host, int records) {
  if (records < 0 || records > kSkTimelineGroups) return -3;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(vk_timeline_sk), sizeof(unsigned long long) * 6 * records, 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : -7;
}
#endif

namespace vk {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kKStep = 32;     // k per stage (one 16x16x32 MFMA deep)

// NC columns per workgroup, M <= 16 * MB rows.  Up to 7 row blocks every
// wave holds all rows and NC/4 columns; from 8 on (MB even) the waves form
// 2 x 2, each holding half the rows and NC/2 columns, which halves the A
// fragments a wave reads per k-step (M = 128: 32.0-32.4 us against 33.4-34.0
// with the 4 x 1 layout; M = 96: no difference).
template <int NC, int MB>
struct SkCfg {
  static constexpr int kWR = MB >= 8 ? 2 : 1;                   // wave rows
  static constexpr int kWC = kWaves / kWR;                      // wave columns
  static constexpr int kMBW = MB / kWR;                         // row blocks per wave
  static_assert(MB % kWR == 0 && MB <= 4 * kWaves, "row blocks");
  static constexpr int kChunks = NC / 8;                        // 16-byte chunks per B row
  static constexpr int kRowsPerDma = 1024 / (NC * 2);           // B rows per 1 KB load
  static constexpr int kBDma = 8 / kRowsPerDma;                 // B loads per wave per k-step
  static constexpr int kBStageBytes = kKStep * NC * 2;          // 8 or 16 KB
  static constexpr int kAStageBytes = 16 * MB * kKStep * 2;     // MB KB: rows x 64 B
  static constexpr int kStageBytes = kBStageBytes + kAStageBytes;
  static constexpr int kStages = (159 * 1024) / kStageBytes < 8 ? (159 * 1024) / kStageBytes : 8;
  static constexpr int kLdsBytes = kStages * kStageBytes;
  static constexpr int kWaveCols = NC / kWC;                   // 32, 64 or 128
  static constexpr int kColBlocks = kWaveCols / 16;             // per wave
  static_assert(kStages >= 4, "pipeline depth");
  static constexpr int kMaxADma = (MB + kWaves - 1) / kWaves;  // A loads per wave per k-step
  static_assert((kStages - 1) * (kBDma + kMaxADma) <= 63, "vmcnt range");
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
// A rows are 64 B = 4 chunks; a fragment read (ds_read_b128) names rows
// lane % 16, chunk lane / 16.  gfx950 serves a ds_read_b128 in 4 passes of
// 16 lanes: lanes l and l' share a pass when l / 32 = l' / 32 and bits 2-4 of
// l and l' have the same parity, and two lanes of a pass that name the same
// 16-byte slot of the 256 bytes of banks (address / 16 mod 16) at different
// addresses cost a cycle (measured on MI355X with a probe of lane pairs and
// whole-wave patterns under SQ_LDS_BANK_CONFLICT).  chunk ^ (row / 2) % 4
// gives every pass 16 distinct slots; chunk ^ (row / 4) % 4, which spreads
// 16 consecutive lanes, cost 4 conflict cycles per read (a quarter of the
// kernel's LDS cycles at M = 16).
__host__ __device__ constexpr int swz_a64(int row) { return (row >> 1) & 3; }

// 128-column blocks: measured at 16 x 8192 x 8192, NC = 128 with K split 4
// ways took 24.3 us, NC = 256 with K split 8 ways 28.1 us (the larger
// k-split costs more in the final reduction than the wider rows gain).
int pick_nc(size_t) { return 128; }

// Counters of the split-K hand-off, one per (column block, wave).
constexpr size_t kCounterBytes = 4096;

// Number of workgroups sharing a column block's K range (pieces of K / 32
// steps, as equal as the steps allow): the largest power of two up to 8 that
// keeps the grid to one workgroup per CU with at least 4 steps per piece,
// while the counters fit.  Measured (us per launch, K split 1/2/4/8 ways):
// 128 x 28672 x 8192 (224 column blocks): 118 / 133 / 154 / 192; 128 x
// 11008 x 4096 (86): 46 / 29 / 37 / 52; 32 x 14336 x 4096 (112): 23 / 21 /
// 25 / 36; 128 x 8192 x 8192 (64): 86 / 49 / 33 / 54 -- a second round of
// workgroups costs more than the longer k range of each.  Counts between
// the powers of two fill more CUs and lose (5120 x 4096 at M = 1 / 16 / 64 /
// 128 with 6 pieces instead of 4: 13.3 / 13.5 / 16.6 / 21.8 against 11.2 /
// 11.2 / 14.4 / 20.3; 4608 x 4096 with 7: 12.2 / 12.8 / 18.2 / 22.4 against
// 10.3 / 10.5 / 13.6 / 19.9): their partials and longer sums cost more.
// Unequal pieces split K that 32 ks does not divide (128 x 8192 x 4064 in
// 4: 23.4 against 36.0 unsplit).
int pick_ks(size_t n, size_t k, int num_cus) {
  const size_t ncb = (n + pick_nc(n) - 1) / pick_nc(n);
  if (ncb * kWaves * sizeof(unsigned) > kCounterBytes) return 1;
  int ks = 1;
  while (ks < 8 && ncb * ks * 2 <= (size_t)num_cus && k / kKStep / (ks * 2) >= 4) ks *= 2;
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
#if VK_TIMELINE
  const unsigned long long tl0 = __builtin_amdgcn_s_memrealtime();
  unsigned long long tl1 = 0;
#endif
  const int n0 = cb * NC;
  // Piece kp of the K / 32 steps: steps floor(kp T / ks) .. floor((kp + 1) T / ks) - 1.
  const int tsteps = K / kKStep;
  const int sbeg = (int)((long long)kp * tsteps / ks_count);
  const int kbeg = sbeg * kKStep;
  const int nsteps = (int)((long long)(kp + 1) * tsteps / ks_count) - sbeg;
#if VK_TIMELINE
  auto tl_record = [&]() {
    if (threadIdx.x == 0 && cid < kSkTimelineGroups) {
      unsigned xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      unsigned long long* r = vk_timeline_sk + cid * 6;
      r[0] = tl0; r[1] = tl1; r[2] = __builtin_amdgcn_s_memrealtime(); r[3] = xcc & 15u;
      r[4] = (unsigned long long)nsteps; r[5] = (unsigned long long)kp;
    }
  };
#else
  auto tl_record = []() {};
#endif

  // Direct-to-LDS duty per k-step.  B: load i covers k-rows 8w + i*R .. +R-1
  // (R = 1024 / (2 NC) rows of NC/8 chunks; lane l: row l / (NC/8), slot
  // l % (NC/8)).  A: wave w covers the 16-row blocks w + 4j < MB (4 chunks
  // per row; lane l: row l/4, slot l%4; the swizzle of row r + 64 is that of
  // row r); a row past M loads row M - 1 instead (valid memory; the rows
  // past M are never stored).
  // In a last column block that N cuts short (N a multiple of 8), a lane
  // whose chunk lies past N loads the block's last chunk of the same row
  // instead: valid memory, and the columns past N are never stored.
  const int cvalid = min(NC, N - n0) / 8;
  uint32_t offB[G::kBDma];
#pragma unroll
  for (int i = 0; i < G::kBDma; i++) {
    const int krow = 8 * wave + i * G::kRowsPerDma + lane / G::kChunks;
    const int c = min((lane % G::kChunks) ^ swz_bk<NC>(krow), cvalid - 1);
    offB[i] = (uint32_t)(((size_t)krow * N + c * 8) * 2);
  }
  const int arow = 16 * wave + (lane >> 2);
  uint32_t offA[G::kMaxADma];
#pragma unroll
  for (int j = 0; j < G::kMaxADma; j++) {
    const int row = min(arow + 64 * j, M - 1);
    offA[j] = (uint32_t)(((size_t)row * K + (((lane & 3) ^ swz_a64(arow)) * 8)) * 2);
  }
  const char* gB = reinterpret_cast<const char*>(B) + ((size_t)kbeg * N + n0) * 2;
  const char* gA = reinterpret_cast<const char*>(A) + (size_t)kbeg * 2;
  const uint32_t lbase = lds_addr32(lds);
  int na = 0;  // A loads of this wave per k-step (wave-uniform)
#pragma unroll
  for (int j = 0; j < G::kMaxADma; j++) na += wave + kWaves * j < MB;

  // NA = this wave's A loads per k-step (blocks wave + 4j < MB are j < NA).
  auto issue = [&](auto nac, int stage, int step) {
    constexpr int NA = decltype(nac)::value;
    const uint32_t s = lbase + stage * G::kStageBytes;
    const size_t kb = (size_t)step * kKStep;
#pragma unroll
    for (int i = 0; i < G::kBDma; i++) dma16(gB + kb * N * 2, offB[i], s + (8 * wave + i * G::kRowsPerDma) * NC * 2);
#pragma unroll
    for (int j = 0; j < NA; j++) dma16(gA + kb * 2, offA[j], s + G::kBStageBytes + (wave + kWaves * j) * 1024);
  };
  // This wave's row and column group (compile-time 0 and `wave` when the
  // waves do not split the rows, so the fragment offsets stay immediates).
  const int rg = G::kWR == 1 ? 0 : wave / G::kWC;
  const int cg = G::kWR == 1 ? wave : wave % G::kWC;

  // Fragment addresses inside a stage.
  // B (MFMA B operand, 16x16x32): lane 16g + 4jj + q names k-row
  // 8g + 4h + jj, columns w*NC/4 + 16c + 4q .. +3; the transpose read hands
  // lane 16g + i the 4 k of column 16c + i.
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  const int krow0 = 8 * g + jj;  // plus 4h: bits 0, 1, 3 unchanged
  uint32_t boff[G::kColBlocks];
#pragma unroll
  for (int c = 0; c < G::kColBlocks; c++) {
    const int chunk = (G::kWaveCols / 8) * cg + 2 * c + (q >> 1);
    boff[c] = (uint32_t)(krow0 * NC * 2 + 16 * (chunk ^ swz_bk<NC>(krow0)) + 8 * (q & 1));
  }
  // A (MFMA A operand): lane l holds A[l%16][8*(l/16) .. +7]: row l%16,
  // chunk l/16 of that row.
  const int ar = lane & 15;
  const uint32_t aoff = (uint32_t)(G::kBStageBytes + ar * 64 + 16 * ((lane >> 4) ^ swz_a64(ar))) +
                        (uint32_t)(rg * G::kMBW * 1024);  // this wave's first row block

  constexpr int MBW = G::kMBW;
  float4v acc[MBW][G::kColBlocks];
#pragma unroll
  for (int r = 0; r < MBW; r++)
#pragma unroll
    for (int c = 0; c < G::kColBlocks; c++) acc[r][c] = float4v{0.f, 0.f, 0.f, 0.f};

  // Fragments of one k-step: B for this wave's column blocks, A for its rows.
  struct Frags {
    half8 b[G::kColBlocks];
    half8 a[MBW];
  };
  auto read_frags = [&](Frags& f, int stage) {
    const uint32_t sb = lbase + stage * G::kStageBytes;
#pragma unroll
    for (int c = 0; c < G::kColBlocks; c++) {
      const half4 lo = lds_read_tr16_at(sb + boff[c]);
      const half4 hi = lds_read_tr16_at(sb + boff[c] + 4 * NC * 2);
      f.b[c] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int r = 0; r < MBW; r++) f.a[r] = lds_read_h8(sb + aoff + r * 1024);
  };
  // Software pipeline over a ring of S stages: iteration `step` multiplies
  // the fragments of `step` (read during the previous iteration) while the
  // fragments of step + 1 are read, so the LDS reads of one k-step overlap
  // the MFMAs of the one before; the stage of `step` is refilled with step
  // + S once every wave's reads of it are done (barrier).  Clamped refills
  // of a short k range land in stages whose contents are never used.  The
  // loop is instantiated per count of A loads (NA, fixed for a wave), so a
  // k-step waits with a constant count and issues without branches (a
  // cascade of tests on the count cost ~2 us per launch at M = 128).
  auto pipeline = [&](auto nac) {
    constexpr int LOADS = G::kBDma + decltype(nac)::value;  // this wave's loads per k-step
#pragma unroll
    for (int st = 0; st < S; st++) issue(nac, st, min(st, nsteps - 1));
    Frags f[2];
    wait_vmcnt<(S - 1) * LOADS>();
    lds_barrier();
    read_frags(f[0], 0);
    auto iteration = [&](int step, Frags& cur, Frags& next) {
      // This wave's loads of step + 1 landed, then everyone's (barrier); the
      // barrier also ends every wave's reads of `step`'s stage.
      wait_vmcnt<(S - 2) * LOADS>();
      wait_lgkmcnt0();  // as the barrier's own wait, but visible to the compiler:
                        // it then knows `cur` has landed and waits for no read
                        // of `next` before the MFMAs
      lds_barrier();
      issue(nac, step % S, min(step + S, nsteps - 1));
      read_frags(next, (step + 1) % S);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 0; r < MBW; r++)
#pragma unroll
        for (int c = 0; c < G::kColBlocks; c++) acc[r][c] = mfma16x16x32(cur.a[r], cur.b[c], acc[r][c]);
    };
    for (int step = 0; step < nsteps; step += 2) {
      iteration(step, f[0], f[1]);
      if (step + 1 < nsteps) iteration(step + 1, f[1], f[0]);
    }
  };
  // A wave loads MB / 4 or MB / 4 + 1 blocks (0 or 1 below 4).
  constexpr int kNaHi = G::kMaxADma, kNaLo = MB / kWaves;
  if constexpr (kNaHi == kNaLo)
    pipeline(std::integral_constant<int, kNaHi>{});
  else if (na == kNaHi)
    pipeline(std::integral_constant<int, kNaHi>{});
  else
    pipeline(std::integral_constant<int, kNaLo>{});
  wait_vmcnt<0>();  // clamped tail refills
#if VK_TIMELINE
  tl1 = __builtin_amdgcn_s_memrealtime();
#endif

  // Epilogue.  D layout: lane l, register e of block (r, c) -> row
  // 16 r + 4 (l / 16) + e, column kWaveCols * w + 16 c + l % 16 of the block.
  constexpr int NB = MBW * G::kColBlocks;  // 16 x 16 blocks per wave
  const int col0 = n0 + G::kWaveCols * cg + (lane & 15);
  OutT* Cw = C + col0;
  const int rq = 16 * rg * MBW + 4 * (lane >> 4);
  auto store_c = [&](int b, const float4v& v) {
    const int r = b / G::kColBlocks, c = b % G::kColBlocks;
    if (col0 + 16 * c >= N) return;  // past N (a last column block cut short)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int row = 16 * r + rq + e;
      if (row < M) Cw[(size_t)row * N + 16 * c] = convert_out<OutT>(v[e]);
    }
  };
  if (ks_count == 1) {
#pragma unroll
    for (int b = 0; b < NB; b++) store_c(b, acc[b / G::kColBlocks][b % G::kColBlocks]);
    tl_record();
    return;
  }

  // Split K.  The partial of (column block cb, k part q) is slot cb * KS + q;
  // wave w's region of a slot holds its NB blocks x 64 lanes x 16 bytes, so
  // every partial access is a coalesced 1 KB row.  Each wave hands off on its
  // own counter (cb, w): it first reads the counter, and if every other part
  // has arrived it is the last and skips its store; otherwise it stores its
  // partial, waits for the stores to complete, and increments the counter.
  // The last arrival sums the KS parts in k order, its own from registers --
  // the same sum whichever part arrives last -- writes C and resets the
  // counter for the next call.
  constexpr uint32_t kWaveRegion = NB * 1024;
  constexpr uint32_t kSlotBytes = kWaves * kWaveRegion;
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      part, 0, (int)((uint32_t)((N + NC - 1) / NC) * (uint32_t)ks_count * kSlotBytes), kBufferWord3);
  auto soff = [&](int q) { return (uint32_t)(cb * ks_count + q) * kSlotBytes + (uint32_t)wave * kWaveRegion; };
  const uint32_t vlane = (uint32_t)lane * 16;
  unsigned* cnt = counters + cb * kWaves + wave;
  const unsigned seen =
      __builtin_amdgcn_readfirstlane(__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  if (seen != (unsigned)(ks_count - 1)) {
#pragma unroll
    for (int b = 0; b < NB; b++) store_partial(prs, vlane + b * 1024, soff(kp), acc[b / G::kColBlocks][b % G::kColBlocks]);
    wait_vmcnt0_ordered();  // the partial is in memory before the counter moves
    unsigned old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_amdgcn_readfirstlane(old) != (unsigned)(ks_count - 1)) {
      tl_record();
      return;
    }
  }
  // The counter read that made this wave the last stays before the reads of
  // the other parts.
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
            if (b0 + i < NB) x[q][i] = acc[(b0 + i) / G::kColBlocks][(b0 + i) % G::kColBlocks];
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
  tl_record();
}

constexpr int kMaxRows = 256;

// Row blocks of the instance that serves M rows (even from 8 on: 2 x 2 waves).
int pick_mb(size_t m) {
  const int mb = (int)((m + 15) / 16);
  return mb > 8 ? (mb + 1) & ~1 : mb;
}

// Workspace: a fixed 4 KB of (column block, wave) counters, then the
// partials.  K is split only while the counters fit (pick_ks); they sit at
// the same place for every shape, which keeps the library workspace clean
// (all counters zero) from one call to the next whatever the shapes.
// Unsplit shapes need no workspace.
size_t sk_workspace(size_t m, size_t n, size_t k, int num_cus) {
  const int ks = pick_ks(n, k, num_cus);
  if (ks == 1) return 0;
  const size_t ncb = (n + pick_nc(n) - 1) / pick_nc(n);
  return kCounterBytes + (size_t)ks * ncb * pick_nc(n) * 16 * pick_mb(m) * sizeof(float);
}

template <int NC, int MB, typename OutT>
hipError_t launch_sk_t(const GemmArgs& a) {
  using G = SkCfg<NC, MB>;
  static std::atomic<uint64_t> done{0};
  auto kfn = f16_skinny_sk_kernel<NC, MB, OutT>;
  hipError_t e = ensure_lds_attr(kfn, G::kLdsBytes, a.device, done);
  if (e != hipSuccess) return e;
  const int ks = pick_ks(a.n, a.k, a.num_cus);
  unsigned* counters = nullptr;
  float* part = nullptr;
  if (ks > 1) {
    if (((a.n + NC - 1) / NC) * kWaves * sizeof(unsigned) > kCounterBytes) return hipErrorInvalidValue;
    counters = static_cast<unsigned*>(a.workspace);
    part = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + kCounterBytes);
    if (!a.workspace_clean) {
      e = zero_words(counters, kCounterBytes / 4, a.stream);
      if (e != hipSuccess) return e;
    }
  }
  const unsigned grid = (unsigned)(((a.n + NC - 1) / NC) * ks);
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
  switch (pick_mb(a.m)) {
    case 1: return launch_mb<NC, 1>(a);
    case 2: return launch_mb<NC, 2>(a);
    case 3: return launch_mb<NC, 3>(a);
    case 4: return launch_mb<NC, 4>(a);
    case 5: return launch_mb<NC, 5>(a);
    case 6: return launch_mb<NC, 6>(a);
    case 7: return launch_mb<NC, 7>(a);
    case 8: return launch_mb<NC, 8>(a);
    case 10: return launch_mb<NC, 10>(a);
    case 12: return launch_mb<NC, 12>(a);
    case 14: return launch_mb<NC, 14>(a);
    default: return launch_mb<NC, 16>(a);
  }
}

hipError_t launch_sk(const GemmArgs& a) { return launch_nc<128>(a); }

// Any M up to 256 (measured at N = K = 8192, µs per launch, this kernel
// against the 256-row tiles of versions 10 / 9: M = 200 49.1 / 54.6, 224
// 48.6 / 55.0, 256 53.2 / 54.7); N a multiple of 8; K a multiple of 32; the
// 32-bit lane byte offsets into A (up to 256 rows) and B (32 rows) must not
// overflow.
bool sk_shape_ok(size_t m, size_t n, size_t k) {
  return m >= 1 && m <= kMaxRows && (size_t)256 * k * 2 < (1ull << 31) && (size_t)32 * n * 2 < (1ull << 31) &&
         ((n + 127) / 128) * 8 < (1ull << 31);
}

}  // namespace

void register_f16_skinny_sk() {
  KernelEntry e{};
  e.version = 8;
  e.in_dtype = VK_DTYPE_F16;
  e.name = "f16_v8_skinny_splitk";
  e.caps = make_caps(8, VK_DTYPE_F16, kOutF16 | kOutF32, 1, 8, kKStep, 16, 256, 128, kKStep, kThreads,
                     SkCfg<128, 16>::kLdsBytes, 0, 1, kMaxRows);
  e.launch = launch_sk;
  e.workspace = sk_workspace;
  e.shape_ok = sk_shape_ok;
  register_kernel(e);
}

}  // namespace vk
