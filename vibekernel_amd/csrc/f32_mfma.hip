// f32_mfma.hip -- fp32 GEMM on the matrix cores (versions 2 and 3 for fp32).
//
// Same operator as fp32 version 1 (f32_valu.hip: the harness's fp32 path,
// results/naive_cycle4/include/playground/system.hpp:35-41, ground truth
// matmul_f32_v0_cblas.cpp:8-12), computed with v_mfma_f32_32x32x2_f32.
// Measured on MI355X with random operands on all CUs (harness/mfma_stream):
// that instruction over 8 accumulators in rotation sustains 153.3-154.1
// TFLOP/s (0.983-0.986 of the 157.3 dense fp32 figure at the measured
// 2.38 GHz) with two waves per SIMD and 153.8 (0.984) with one; fp32 MFMAs
// stay below the board's power limit, so cycles are time.  The 16x16x4 form
// reaches 152.7 / 150.9 and a 16x16x4 version of this kernel measured
// slower.  An fp32 MFMA does 64 FLOP per clock per SIMD -- 16x fewer than
// the fp16 form -- so the operand traffic per cycle is small and no
// ping-pong is needed.  Common to both kernels below:
//  * 256x256 tiles; BK-deep k-tiles (A 256xBK and B BKx256 fp32) in an LDS
//    ring filled by direct-to-LDS loads, one barrier per k-tile;
//  * fragments: the MFMA takes lane l's A value as X[l%32][l/32] and its B
//    value as Y[l/32][l%32] (2 k per instruction).  Step s of a k-tile pairs
//    k = s (lanes 0..31) with k = BK/2 + s (lanes 32..63), so a lane's A
//    values for the BK/2 steps are BK/2 consecutive k of one row (16-byte
//    reads) and its B values one column of BK/2 k-rows.  Result: lane l,
//    register r holds D[8*(r/4) + 4*(l/32) + r%4][l%32] of the block;
//  * per element the sum runs over the steps in ascending order, k-tile by
//    k-tile, so the two kernels give the same bits.
// Versions 2 and 3 on 256x256 tiles with K % 32 == 0 run the four-wave
// kernel (f32_mfma4_kernel: one wave per SIMD owning a 128x128 quarter,
// 32-deep k-tiles in 2 stages of 64 KB; for version 3 with buffer loads and
// bounded stores); other K on 256x256 tiles run the eight-wave kernel
// (f32_mfma_kernel: wave w owns rows 128*(w/4) and columns 64*(w%4) onward,
// 4x2 blocks of 32x32; version 2 with K % 32 == 16: BK = 16 in 4 stages of
// 32 KB; version 3: BK = 32 in 2 stages, the last k-tile masked per lane).
// Grids of few 256x256 tiles take the four-wave kernel on 128x128 or 64x64
// tiles for any K (below).  Interleaved on one box, the
// four-wave form measured 0.8-1.4 % faster at 4096^3 (0.8 % at 4096 x 4096
// x 8192) and with edges 1.1 % at 4000^3 and 0.7 % at 1000 x 3000 x 2048;
// with the last k-tile's per-lane masking as well (64-bit mask shifts
// between the MFMAs) it was 0.6-1.0 % slower than the eight-wave form.
// LDS swizzles (physical 16-byte chunk = logical ^ f(row)):
//  * A rows are 4*BK bytes: f = (row / 4) % 4 for 64-byte rows, (row / 2) % 8
//    for 128-byte rows, so 16 consecutive rows reading one logical chunk hit
//    16 distinct slots of the 256-byte bank space;
//  * B k-rows are 1 KB (64 chunks): f = 8 for the k-rows lanes 32..63 read,
//    so the two lane halves (same columns) use opposite halves of the banks.
// The k-order of the sum differs from the oracle's sequential chain (pairs
// of products per step), so parity is the fp32 accumulation bound, not bit
// equality.
#include "vk_device.hpp"
#include "vk_internal.hpp"
#include "vk_splittail.hpp"
#include "vk_tile.hpp"

#include <atomic>

namespace vk {
namespace {

constexpr int kBM = 256, kBN = 256;
constexpr int kThreads = 512;  // the eight-wave kernel

// k-tile depth BK (fp32): 16 with a 4-stage ring or 32 with 2 stages (128 KB
// of LDS either way).
template <int BK>
struct F32Cfg {
  static constexpr int kNS = BK == 16 ? 4 : 2;
  static constexpr int kABytes = kBM * BK * 4;  // 256 rows x 4*BK bytes
  static constexpr int kBBytes = BK * kBN * 4;  // BK k-rows x 1 KB
  static constexpr int kStageBytes = kABytes + kBBytes;
  static constexpr int kLdsBytes = kNS * kStageBytes;
  static constexpr int kRowChunks = BK / 4;     // 16-byte chunks per A row
  static constexpr int kDmaA = BK / 8;          // A instructions per wave per k-tile (eight waves)
  static constexpr int kDmaB = BK / 8;          // B instructions per wave per k-tile (eight waves)
  static constexpr int kDma = kDmaA + kDmaB;
  static constexpr int kSteps = BK / 2;         // MFMA k-steps per k-tile
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
  static_assert(BK == 16 || BK == 32, "k-tile depth");
};

typedef float float16v_ __attribute__((ext_vector_type(16)));

// A: 64-byte rows (BK 16): chunk ^ (row / 4) % 4; 128-byte rows (BK 32):
// chunk ^ (row / 2) % 8 -- 16 consecutive rows reading one logical chunk hit
// 16 distinct 16-byte slots of the 256-byte bank space.  B: chunk ^ 8 for the
// k-rows read by lanes 32..63 (bit log2(BK/2) of the k-row).
template <int BK>
__host__ __device__ constexpr int swz_a32(int row) {
  return BK == 16 ? (row >> 2) & 3 : (row >> 1) & 7;
}
template <int BK>
__host__ __device__ constexpr int swz_b32(int krow) {
  return ((krow / (BK / 2)) & 1) << 3;
}

__device__ __forceinline__ float lds_read_f32(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) float*>(addr);
}
__device__ __forceinline__ float4v lds_read_f4(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) float4v*>(addr);
}

// Eight-wave kernel: per k-tile each wave reads its fragments (BK/2
// ds_read_b128 of A, BK ds_read_b32 of B) and issues 4*BK MFMAs of 64
// cycles, with its loads of a later k-tile going out one after each of the
// first MFMA steps.
// kEdge (version 3): the tiles may reach past M rows or N columns and the
// last k-tile past K (any M; N, K multiples of 4).  The loads then go through
// buffer resources over the whole matrices, the k-tile's offset in the
// scalar offset: a lane past the end of a matrix reads zeros (A rows at or
// below M, B k-rows at or below K); B columns past N are in range (the next
// row's) but only feed C columns that are not stored; A's k past K on the
// last k-tile (the next row's values, which must not meet B's zero rows: an
// infinity would make a NaN) is masked by giving those lanes the matrix size
// as their offset.  C elements outside M x N are not stored.
template <int BK, bool kEdge>
__global__ __launch_bounds__(kThreads) void f32_mfma_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                            float* __restrict__ C, int M, int N, int K) {
  using G = F32Cfg<BK>;
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, gw = wave & 3;
  int tm, tn;
  tile_of(blockIdx.x, (M + (kEdge ? kBM - 1 : 0)) / kBM, (N + (kEdge ? kBN - 1 : 0)) / kBN, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  // ---- direct-to-LDS duty per k-tile: A instructions kDmaA*w + d (1 KB =
  // 1024 / (4 BK) rows each), B instructions kDmaB*w + d (k-row of that
  // number, 1 KB) ----
  constexpr int kRowsPerDma = 1024 / (4 * BK);
  uint32_t voffA[G::kDmaA], voffB[G::kDmaB];
  uint32_t akin = 0;  // kEdge: bits 5d..5d+4 = first k of the lane's A chunk of instruction d
#pragma unroll
  for (int d = 0; d < G::kDmaA; d++) {
    const int i = G::kDmaA * wave + d;
    const int row = kRowsPerDma * i + lane / G::kRowChunks;
    const int ca = (lane % G::kRowChunks) ^ swz_a32<BK>(row);
    voffA[d] = (uint32_t)(((size_t)row * K + ca * 4) * 4);
    if constexpr (kEdge) akin |= (uint32_t)(ca * 4) << (5 * d);
  }
#pragma unroll
  for (int d = 0; d < G::kDmaB; d++) {
    const int i = G::kDmaB * wave + d;
    const int cb = lane ^ swz_b32<BK>(i);
    voffB[d] = (uint32_t)(((size_t)i * N + cb * 4) * 4);
  }
  const char* gA = reinterpret_cast<const char*>(A) + (size_t)m0 * K * 4;
  const char* gB = reinterpret_cast<const char*>(B) + (size_t)n0 * 4;
  const uint32_t sizeA = kEdge ? (uint32_t)M * (uint32_t)K * 4u : 0u;
  const uint32_t sizeB = kEdge ? (uint32_t)K * (uint32_t)N * 4u : 0u;
  const __amdgpu_buffer_rsrc_t rsrcA =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), 0, (int)sizeA, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rsrcB =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), 0, (int)sizeB, kBufferWord3);
  auto issue = [&](int kt, int slot) {
    const uint32_t s = lds_base + slot * G::kStageBytes;
    if constexpr (kEdge) {
      const uint32_t kleft = (uint32_t)(K - kt * BK);  // k from this k-tile's start to K (> 0)
      const uint32_t soffA = (uint32_t)(m0 * K + kt * BK) * 4u;
      const uint32_t soffB = (uint32_t)(kt * BK * N + n0) * 4u;
#pragma unroll
      for (int d = 0; d < G::kDmaA; d++) {
        const uint32_t off = ((akin >> (5 * d)) & 31u) < kleft ? voffA[d] : sizeA;  // sizeA: zeros
        dma16_buf(rsrcA, off, soffA, s + (G::kDmaA * wave + d) * 1024);
      }
#pragma unroll
      for (int d = 0; d < G::kDmaB; d++) dma16_buf(rsrcB, voffB[d], soffB, s + G::kABytes + (G::kDmaB * wave + d) * 1024);
    } else {
#pragma unroll
      for (int d = 0; d < G::kDmaA; d++)
        dma16(gA + (size_t)kt * BK * 4, voffA[d], s + (G::kDmaA * wave + d) * 1024);
#pragma unroll
      for (int d = 0; d < G::kDmaB; d++)
        dma16(gB + (size_t)kt * BK * N * 4, voffB[d], s + G::kABytes + (G::kDmaB * wave + d) * 1024);
    }
  };
  // Load d of the k-tile (A loads first, then B), one at a time: inside the
  // k-loop the loads of a later k-tile go out one after each MFMA step
  // instead of in a burst after the barrier (measured +1.1 % at 4096^3,
  // +1.6 % on version 3 at 4000^3: a wave stalled behind its burst of loads
  // issues no MFMA).
  auto issue_one = [&](int kt, int slot, int d) {
    const uint32_t s = lds_base + slot * G::kStageBytes;
    if constexpr (kEdge) {
      const uint32_t kleft = (uint32_t)(K - kt * BK);
      const uint32_t soffA = (uint32_t)(m0 * K + kt * BK) * 4u;
      const uint32_t soffB = (uint32_t)(kt * BK * N + n0) * 4u;
      if (d < G::kDmaA) {
        const uint32_t off = ((akin >> (5 * d)) & 31u) < kleft ? voffA[d] : sizeA;
        dma16_buf(rsrcA, off, soffA, s + (G::kDmaA * wave + d) * 1024);
      } else {
        const int e = d - G::kDmaA;
        dma16_buf(rsrcB, voffB[e], soffB, s + G::kABytes + (G::kDmaB * wave + e) * 1024);
      }
    } else {
      if (d < G::kDmaA) {
        dma16(gA + (size_t)kt * BK * 4, voffA[d], s + (G::kDmaA * wave + d) * 1024);
      } else {
        const int e = d - G::kDmaA;
        dma16(gB + (size_t)kt * BK * N * 4, voffB[e], s + G::kABytes + (G::kDmaB * wave + e) * 1024);
      }
    }
  };

  // ---- fragment addresses inside a stage: lane half h takes k = (BK/2) h
  // + s at step s ----
  const int h = lane >> 5;
  constexpr int kChunksPerHalf = G::kSteps / 4;  // A chunks a lane reads per block
  uint32_t aoff[4][kChunksPerHalf];
#pragma unroll
  for (int bi = 0; bi < 4; bi++) {
    const int row = grp * 128 + bi * 32 + (lane & 31);
#pragma unroll
    for (int c = 0; c < kChunksPerHalf; c++)
      aoff[bi][c] = row * (4 * BK) + 16 * ((kChunksPerHalf * h + c) ^ swz_a32<BK>(row));
  }
  uint32_t boff[2];
#pragma unroll
  for (int bj = 0; bj < 2; bj++) {
    const int col = gw * 64 + bj * 32 + (lane & 31);
    // k-row (BK/2) h + s: the swizzle bit is h for every step
    boff[bj] = G::kABytes + G::kSteps * h * 1024 + 16 * ((col >> 2) ^ (h << 3)) + 4 * (col & 3);
  }

  float16v_ acc[4][2];
#pragma unroll
  for (int bi = 0; bi < 4; bi++)
#pragma unroll
    for (int bj = 0; bj < 2; bj++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[bi][bj][r] = 0.0f;
  prefer_agpr_accumulators();

  const int nk = (K + (kEdge ? BK - 1 : 0)) / BK;
#pragma unroll
  for (int st = 0; st < G::kNS - 1; st++) issue(min(st, nk - 1), st);

  for (int t = 0; t < nk; t++) {
    // This wave's loads of k-tile t are in; then everyone's (barrier), which
    // also ends every wave's reads of the slot the next issue refills.
    wait_vmcnt<(G::kNS - 2) * G::kDma>();
    lds_barrier();
    const int kt_next = min(t + G::kNS - 1, nk - 1), slot_next = (t + G::kNS - 1) % G::kNS;
    const uint32_t s = lds_base + (t % G::kNS) * G::kStageBytes;
    float a[4][G::kSteps], b[2][G::kSteps];
#pragma unroll
    for (int bi = 0; bi < 4; bi++)
#pragma unroll
      for (int c = 0; c < kChunksPerHalf; c++) {
        const float4v v = lds_read_f4(s + aoff[bi][c]);
#pragma unroll
        for (int q = 0; q < 4; q++) a[bi][4 * c + q] = v[q];
      }
#pragma unroll
    for (int bj = 0; bj < 2; bj++)
#pragma unroll
      for (int st = 0; st < G::kSteps; st++) b[bj][st] = lds_read_f32(s + boff[bj] + st * 1024);
    static_assert(G::kDma <= G::kSteps, "one load per MFMA step");
#pragma unroll
    for (int st = 0; st < G::kSteps; st++) {
#pragma unroll
      for (int bi = 0; bi < 4; bi++)
#pragma unroll
        for (int bj = 0; bj < 2; bj++)
          acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[bi][st], b[bj][st], acc[bi][bj], 0, 0, 0);
      if (st < G::kDma) {
        __builtin_amdgcn_sched_barrier(0);
        issue_one(kt_next, slot_next, st);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  wait_vmcnt<0>();  // clamped refills past the last k-tile

  // ---- epilogue: lane l, register r of block (bi, bj) ->
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32: 128-byte row segments ----
  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int row0 = m0 + grp * 128, col0 = n0 + gw * 64;
#pragma unroll
  for (int bi = 0; bi < 4; bi++)
#pragma unroll
    for (int bj = 0; bj < 2; bj++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = row0 + bi * 32 + 8 * (r >> 2) + 4 * (lane_e >> 5) + (r & 3);
        const int col = col0 + bj * 32 + (lane_e & 31);
        if (!kEdge || (row < M && col < N)) C[(size_t)row * N + col] = acc[bi][bj][r];
      }
}

// Timeline build (make timeline -> libvk_gemm_timeline.so, VK_TIMELINE=1):
// every wave of the first 1024 workgroups of the four-wave kernel records
// the 100 MHz real-time clock at entry, at the start and end of its k-loop
// and after its C stores complete, its XCD, and in shader clock cycles the
// k-loop's length and the part of it spent from the last group's first
// MFMA step to the end of the k-tile barrier (waits for this wave's LDS reads
// and loads, and the barrier); vk_timeline_f32_read() copies them out.  The
// product library is built with VK_TIMELINE=0 and records nothing.
#ifndef VK_TIMELINE
#define VK_TIMELINE 0
#endif
#if VK_TIMELINE
constexpr int kF32TimelineWaves = 1024 * 4;
__device__ unsigned long long vk_timeline_f32[kF32TimelineWaves * 8];
extern "C" int vk_timeline_f32_read(unsigned long long* host, int waves) {
  if (waves < 0 || waves > kF32TimelineWaves) return -3;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(vk_timeline_f32), sizeof(unsigned long long) * 8 * waves, 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : -7;
}
#endif

// Four-wave kernel (versions 2 and 3, K % 32 == 0): the eight-wave kernel's
// 32-deep k-tiles, LDS layout, loads and per-element k order on tiles of
// 64 kNB x 64 kNB, one wave per SIMD owning a quarter of 32 kNB x 32 kNB
// (kNB x kNB blocks of 32x32); wave w owns rows 32 kNB (w / 2) and columns
// 32 kNB (w % 2) onward.
//  * kNB = 4, 256x256 tiles (256 fp32 accumulators per lane in AGPRs), where
//    those tiles fill the CUs in as few waves as 128x128 ones: per k-tile a
//    wave reads 16 KB of A and
//    16 KB of B fragments (the eight-wave kernel's waves 16 + 8 KB each, two
//    per SIMD), a third less LDS data per MFMA.  Measured per k-tile
//    (timeline build, 4096^3): 17,113 shader cycles against the 16,384 its
//    MFMAs need on every XCD (0.957); instrumented copies without the
//    fragment reads took 16,420 (the A reads' 16 ds_read_b128 cost ~510
//    cycles, the B reads' 32 ds_read2st64_b32 ~225), without the loads
//    16,988, without the barrier 17,090.
//  * kNB = 2, 128x128 tiles (64 accumulators per lane) everywhere else:
//    four times as many tiles, for grids whose 256x256 tiles would leave
//    CUs idle (1024^3: 16 of them on 256 CUs) or fill a last wave in part
//    (4096 x 4352: 272); where even the 128x128 tiles fill at most half of
//    the CUs, K is split over the idle ones (kSplit, below).  An fp32 MFMA
//    takes 64 cycles, so a wave's 128x128x32 k-tile is 4096 cycles of MFMA
//    against 16 KB of fragment reads and 8 KB of loads: the smaller tile
//    costs the matrix cores next to nothing (measured at 4096^3, 2 rounds on
//    one box: 943.8 / 945.3 us per launch against 939.9 / 941.7 with
//    256x256 tiles; 4096 x 4352 x 4096 1188 / 1193 against 1873 / 1861;
//    6144 x 4096 x 4096 1416 / 1417 against 1900 / 1881); with a part-empty
//    last round split (below): 4096 x 4352 x 4096 1063, 3072^3 430.5
//    against 535.6, 2304 x 2048 x 2048 168.4 against 237.1.
//  * kNB = 1, 64x64 tiles (one 32x32 block per wave, 16 accumulators) where
//    the 128x128 tiles are fewer than the CUs: per k-tile 16 MFMAs of
//    the one block, 3 fragment reads per group and 4 loads per wave.
//    Measured against 128x128 tiles (2 rounds, one box, us per launch):
//    512^3 9.35 against 15.75, 1024^3 20.4 / 25.9, 1024 x 1024 x 512 11.5 /
//    17.9, 768 x 512 x 256 6.8 / 12.5, v3 1000^3 22.5 / 27.2, 1280^3 42.3 /
//    48.5.
// A wave's fragments are read one group of 4 steps ahead into a second
// register set: the next group's kReads reads (kNB A reads of 16 bytes, 2 kNB
// pairs of B values) one after each of the first kReads MFMAs from the
// group's second step on.  The k-tile's one barrier sits after the first
// step of its last group (whose fragments are already in registers),
// followed by the next k-tile's first group of reads and, one after every
// kLoadEvery-th MFMA of the last three steps, the kD loads that refill the
// slot just freed with k-tile t + 2 (clamped to the last k-tile: a refill
// past the end rewrites the last k-tile's data into a slot nobody reads).
template <int kNB>
struct F32W4 {
  static constexpr int BK = 32;
  static constexpr int kT = 64 * kNB;                    // tile side
  static constexpr int kQ = 32 * kNB;                    // a wave's quarter
  static constexpr int kABytes = kT * BK * 4;            // kT rows of 128 B
  static constexpr int kBRow = kT * 4;                   // bytes of a B k-row
  static constexpr int kStageBytes = kABytes + BK * kBRow;
  static constexpr int kLdsBytes = 2 * kStageBytes;      // 128 or 64 KB
  static constexpr int kRowChunks = BK / 4;              // 16-byte chunks per A row
  static constexpr int kSteps = BK / 2;                  // MFMA k-steps per k-tile
  static constexpr int kDA = kT / 32;                    // A loads per wave per k-tile (8 rows each)
  static constexpr int kBRowsPerDma = 1024 / kBRow;      // B k-rows per 1 KB load
  static constexpr int kDB = BK / kBRowsPerDma / 4;      // B loads per wave per k-tile
  static constexpr int kD = kDA + kDB;
  static constexpr int kReads = 3 * kNB;                 // fragment reads per group of 4 steps
  // MFMAs per load in the last 3 steps; 0 (64x64 tiles: 4 loads, 3 MFMAs):
  // load m after MFMA m, the last two after the last MFMA
  static constexpr int kLoadEvery = 3 * kNB * kNB / kD;
  static_assert(kLdsBytes <= 160 * 1024 && (kLoadEvery >= 1 || kNB == 1) && kD * kLoadEvery <= 3 * kNB * kNB,
                "schedule");
  // loads [load_begin(m), load_begin(m + 1)) go out after MFMA m of the last 3 steps
  static constexpr int load_begin(int m) {
    return kLoadEvery >= 1 ? (m + kLoadEvery - 1) / kLoadEvery < kD ? (m + kLoadEvery - 1) / kLoadEvery : kD
                           : m < 3 * kNB * kNB ? m : kD;
  }
  static_assert(kReads <= 3 * kNB * kNB, "a group's reads fit its last three steps");
};

// ---- split K (kNB = 2): for grids whose 128x128 tiles fill at most half of
// the CUs, sk_plan_fill's pieces of every tile (at least kF32MinIters
// k-tiles each, the last one k-tile longer); otherwise sk_plan's split tail
// (the tiles of a part-empty last round of the CUs cut into k-slices, the
// others whole, as the fp16 version 9).  The pieces of a tile meet as in
// the fp16 128x128 kernel: per (tile, wave) an arrival counter; a finishing wave that
// finds every other piece in memory is the last and writes nothing,
// otherwise it writes its 16 KB fp32 partial with sc1 stores, waits for them
// and increments the counter, and the one that sees np - 1 is the last.  The
// last sums P0 + P1 + ... in k order (its own piece from registers), so C
// does not depend on the arrival order, stores C and resets the counter.
// A piece of 2 k-tiles is ~3.5 us of MFMA at the board's clock.  Measured
// against pieces of at least 4 (2 rounds, one box, us per launch): 512^3
// 15.5 against 16.7, 512 x 512 x 256 12.8 against 15.0, 256 x 512 x 512
// 15.2 against 16.6.
constexpr int kF32MinIters = 2;
// One tile's fp32 partial, and a wave's quarter of it.
constexpr size_t f32_slot_bytes(int nb) { return (size_t)(64 * nb) * (64 * nb) * sizeof(float); }
constexpr uint32_t f32_wave_bytes(int nb) { return (uint32_t)(32 * nb) * (32 * nb) * sizeof(float); }

__host__ __device__ inline int64_t f32_tiles(size_t m, size_t n, size_t t) {
  return (int64_t)((m + t - 1) / t) * (int64_t)((n + t - 1) / t);
}
// 128x128 tiles unless the 256x256 ones, each four times the work, fill the
// CUs in as few rounds (4096^3: 256 tiles in one round against 1024 in four).
inline bool f32_small_tiles(size_t m, size_t n, int num_cus) {
  const int64_t c = num_cus > 0 ? num_cus : 1;
  return 4 * ((f32_tiles(m, n, 256) + c - 1) / c) > (f32_tiles(m, n, 128) + c - 1) / c;
}
// Blocks of 32x32 per wave side off the 256x256 tiles: 2 (128x128 tiles), or
// 1 (64x64) where the 128x128 tiles are fewer than the CUs (several 64x64
// workgroups share a CU: 32 KB of LDS and at most 136 registers each).
// Measured against 128x128 tiles (2 rounds, one box, us per launch): 1536^3
// (144 tiles of 128x128) 58.6 against 96.3; where the 128x128 tiles fill
// whole rounds they win: 3072^3 409 against 452, 2048^3 128 / 126.
inline int f32_small_nb(size_t m, size_t n, int num_cus) {
  return f32_tiles(m, n, 128) < (num_cus > 0 ? num_cus : 1) ? 1 : 2;
}
inline SkPlan f32_plan(size_t m, size_t n, size_t k, int num_cus, int nb) {
  const int64_t T = f32_tiles(m, n, 64 * (size_t)nb), I = (int64_t)((k + 31) / 32);
  const SkPlan fill = sk_plan_fill(T, I, num_cus, kF32MinIters);
  return fill.units > 0 ? fill : sk_plan(T, I, num_cus);
}
// Extra k-tiles of a split tile's last piece: one in a fill plan (no whole
// tiles), sk_plan's own number in a tail plan.
inline int f32_last_extra(const SkPlan& p) { return p.dp > 0 ? kSkLastExtra : kFillLastExtra; }

// Vector v of a wave's accumulators: block (v / 4kNB, (v / 4) % kNB),
// registers 4 (v % 4) .. + 3.  In a partial, vector v of every lane sits at
// v * 1024 + lane * 16 of the wave's region: each store a coalesced 1 KB.
template <int kNB>
__device__ __forceinline__ float4v acc_vec(const float16v_ (&acc)[kNB][kNB], int v) {
  const float16v_& x = acc[v / (4 * kNB)][(v / 4) % kNB];
  const int r = 4 * (v % 4);
  return float4v{x[r], x[r + 1], x[r + 2], x[r + 3]};
}

// This wave holds piece p of np of its quarter; part_off(q): byte offset of
// the wave's region of piece q's slot.  Returns whether this wave arrived
// last.  Only the last piece, which usually arrives last, reads the counter
// first; the others publish their partial at once.
template <int kNB, typename PartOff>
__device__ __forceinline__ bool f32_split_arrive(const float16v_ (&acc)[kNB][kNB], int np, int p, int lane,
                                                 __amdgpu_buffer_rsrc_t part, PartOff part_off, unsigned* cnt) {
  if (p == np - 1) {
    const unsigned seen =
        __builtin_amdgcn_readfirstlane(__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if (seen == (unsigned)(np - 1)) return true;  // every other piece is in memory
  }
  const uint32_t soff = part_off(p);
#pragma unroll
  for (int v = 0; v < 4 * kNB * kNB; v++) store_partial(part, (uint32_t)lane * 16 + v * 1024, soff, acc_vec(acc, v));
  wait_vmcnt0_ordered();  // the partial is in memory before the counter moves
  unsigned old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_amdgcn_readfirstlane(old) == (unsigned)(np - 1);
}

// The last arrival: acc <- P0 + P1 + ... + P(NP-1), left to right, with
// P(p) = acc.  Every piece's vectors are loaded kB at a time (NP x kB loads
// in flight, at most 64 registers, which keeps the 128x128 split instance at
// 216 registers: two workgroups per CU, where batches of twice the size
// needed 288 -- measured 3072^3 411.1 against 431.7 us, 2304 x 2048 x 2048
// 160.7 against 168.3), the own piece's slot too (not used; it always lies
// inside the workspace, so no branch is needed).
template <int kNB, int NP, typename PartOff>
__device__ __forceinline__ void f32_split_sum_n(float16v_ (&acc)[kNB][kNB], int p, int lane,
                                                __amdgpu_buffer_rsrc_t part, PartOff part_off) {
  constexpr int kV = 4 * kNB * kNB;
  constexpr int kB = (NP <= 4 ? 4 : 2) < kV ? (NP <= 4 ? 4 : 2) : kV;
  static_assert(kV % kB == 0, "whole batches");
#pragma unroll
  for (int v0 = 0; v0 < kV; v0 += kB) {
    float4v x[NP][kB];
#pragma unroll
    for (int q = 0; q < NP; q++) {
      const uint32_t soff = part_off(q);
#pragma unroll
      for (int b = 0; b < kB; b++) x[q][b] = load_partial(part, (uint32_t)lane * 16 + (v0 + b) * 1024, soff);
    }
#pragma unroll
    for (int b = 0; b < kB; b++) {
      const int v = v0 + b;
      const uint4v own = __builtin_bit_cast(uint4v, acc_vec(acc, v));
      float4v t;
#pragma unroll
      for (int q = 0; q < NP; q++) {
        // piece q's term: the own registers where q == p, picked by a mask
        // the compiler cannot see through (no branch in the sum)
        uint32_t mine = q == p ? ~0u : 0u;
        asm volatile("" : "+v"(mine));
        const float4v term =
            __builtin_bit_cast(float4v, (__builtin_bit_cast(uint4v, x[q][b]) & ~mine) | (own & mine));
        t = q == 0 ? term : t + term;
      }
      float16v_& dst = acc[v / (4 * kNB)][(v / 4) % kNB];
      const int r = 4 * (v % 4);
#pragma unroll
      for (int e = 0; e < 4; e++) dst[r + e] = t[e];
    }
  }
}

template <int kNB, typename PartOff>
__device__ __forceinline__ void f32_split_sum(float16v_ (&acc)[kNB][kNB], int np, int p, int lane,
                                              __amdgpu_buffer_rsrc_t part, PartOff part_off) {
  // The counter read that made this wave the last stays before these reads.
  asm volatile("" ::: "memory");
  static_assert(kFillMaxPieces == 8, "one case per piece count");
  switch (np) {
    case 2: f32_split_sum_n<kNB, 2>(acc, p, lane, part, part_off); break;
    case 3: f32_split_sum_n<kNB, 3>(acc, p, lane, part, part_off); break;
    case 4: f32_split_sum_n<kNB, 4>(acc, p, lane, part, part_off); break;
    case 5: f32_split_sum_n<kNB, 5>(acc, p, lane, part, part_off); break;
    case 6: f32_split_sum_n<kNB, 6>(acc, p, lane, part, part_off); break;
    case 7: f32_split_sum_n<kNB, 7>(acc, p, lane, part, part_off); break;
    default: f32_split_sum_n<kNB, 8>(acc, p, lane, part, part_off); break;
  }
}

// kSplit: this workgroup is number blockIdx.x of the split plan {dp, units,
// pieces, chunks} (the last piece of a split tile `extra` k-tiles longer);
// part and counters are the workspace.  kKMask (with kEdge,
// for K % 32 != 0): the last k-tile reaches past K.  B's k-rows past K read
// zeros (the buffer range); A's k past K in memory are the next row's
// values, which must not meet those zeros (an infinity would make a NaN), so
// an A load whose chunk starts at or past K takes the matrix size as its
// offset and reads zeros (K % 4 == 0: a 16-byte chunk lies wholly on one
// side).
template <int kNB, bool kEdge, bool kSplit, bool kKMask = false>
__global__ __launch_bounds__(256) void f32_mfma4_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                        float* __restrict__ C, int M, int N, int K, int dp,
                                                        int units, int pieces, int chunks, int extra,
                                                        float* __restrict__ part, unsigned* __restrict__ counters) {
  using W = F32W4<kNB>;
  constexpr int BK = W::BK, kT = W::kT, kQ = W::kQ;
  constexpr int kDA = W::kDA, kDB = W::kDB, kD = W::kD;
  static_assert(!kSplit || kNB <= 2, "K is split on the 128x128 and 64x64 tiles only");
  static_assert(!kKMask || (kEdge && kNB <= 2), "the k mask is for the 128x128 and 64x64 edge tiles");
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = wave >> 1, wc = wave & 1;
  const int tiles_m = (M + (kEdge ? kT - 1 : 0)) / kT, tiles_n = (N + (kEdge ? kT - 1 : 0)) / kT;
  const int iters = (K + (kKMask ? BK - 1 : 0)) / BK;
  int tm, tn, kb = 0, nk = iters;
  SkWork w{};
  if constexpr (kSplit) {
    w = sk_work(blockIdx.x, tiles_m * tiles_n, iters, SkPlan{dp, units, pieces, chunks}, extra);
    raster_tile(w.cid, tiles_m, tiles_n, tm, tn);
    kb = w.kb;
    nk = w.ke - w.kb;
  } else {
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  }
  const int m0 = tm * kT, n0 = tn * kT;
  const uint32_t lds_base = lds_addr32(lds);

#if VK_TIMELINE
  const unsigned long long tl_entry = __builtin_amdgcn_s_memrealtime();
  unsigned long long tl_bar = 0;
#endif
  // Load d < kDA of a wave is A instruction kDA w + d (8 rows of 128 bytes),
  // load kDA + e its B instruction kDB w + e (kBRowsPerDma k-rows, 1 KB).
  constexpr int kRowsPerDma = 1024 / (4 * BK);
  constexpr int kBLanesPerRow = 64 / W::kBRowsPerDma;
  uint32_t voffA[kDA], voffB[kDB];
  uint32_t achunk = 0;  // kKMask: bits 3d .. 3d + 2, the k-chunk A load d fetches
#pragma unroll
  for (int d = 0; d < kDA; d++) {
    const int i = kDA * wave + d;
    const int row = kRowsPerDma * i + lane / W::kRowChunks;
    const int ca = (lane % W::kRowChunks) ^ swz_a32<BK>(row);
    voffA[d] = (uint32_t)(((size_t)row * K + ca * 4) * 4);
    achunk |= (uint32_t)ca << (3 * d);
  }
#pragma unroll
  for (int d = 0; d < kDB; d++) {
    const int krow = W::kBRowsPerDma * (kDB * wave + d) + lane / kBLanesPerRow;
    const int cb = (lane % kBLanesPerRow) ^ swz_b32<BK>(krow);
    voffB[d] = (uint32_t)(((size_t)krow * N + cb * 4) * 4);
  }
  const char* gA = reinterpret_cast<const char*>(A) + ((size_t)m0 * K + (size_t)kb * BK) * 4;
  const char* gB = reinterpret_cast<const char*>(B) + ((size_t)kb * BK * N + n0) * 4;
  const uint32_t sizeA = kEdge ? (uint32_t)M * (uint32_t)K * 4u : 0u;
  const uint32_t sizeB = kEdge ? (uint32_t)K * (uint32_t)N * 4u : 0u;
  const __amdgpu_buffer_rsrc_t rsrcA =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), 0, (int)sizeA, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rsrcB =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), 0, (int)sizeB, kBufferWord3);
  auto issue_one = [&](int kt, int slot, int d) {
    const uint32_t s = lds_base + slot * W::kStageBytes;
    if constexpr (kEdge) {
      // rows past M and k-rows past K read zeros (the buffer ranges); B
      // columns past N read the next row's, feeding only C columns that are
      // not stored
      if (d < kDA) {
        uint32_t off = voffA[d];
        if constexpr (kKMask) {
          const int kleft = K - (kb + kt) * BK;
          off = 4 * (int)((achunk >> (3 * d)) & 7u) < kleft ? off : sizeA;  // sizeA: zeros
        }
        dma16_buf(rsrcA, off, (uint32_t)(m0 * K + (kb + kt) * BK) * 4u, s + (kDA * wave + d) * 1024);
      } else
        dma16_buf(rsrcB, voffB[d - kDA], (uint32_t)((kb + kt) * BK * N + n0) * 4u,
                  s + W::kABytes + (kDB * wave + d - kDA) * 1024);
    } else {
      if (d < kDA)
        dma16(gA + (size_t)kt * BK * 4, voffA[d], s + (kDA * wave + d) * 1024);
      else
        dma16(gB + (size_t)kt * BK * N * 4, voffB[d - kDA], s + W::kABytes + (kDB * wave + d - kDA) * 1024);
    }
  };

  const int h = lane >> 5;
  uint32_t aoff[kNB][4];
#pragma unroll
  for (int bi = 0; bi < kNB; bi++) {
    const int row = wr * kQ + bi * 32 + (lane & 31);
#pragma unroll
    for (int c = 0; c < 4; c++) aoff[bi][c] = row * (4 * BK) + 16 * ((4 * h + c) ^ swz_a32<BK>(row));
  }
  uint32_t boff[kNB];
#pragma unroll
  for (int bj = 0; bj < kNB; bj++) {
    const int col = wc * kQ + bj * 32 + (lane & 31);
    boff[bj] = W::kABytes + W::kSteps * h * W::kBRow + 16 * ((col >> 2) ^ (h << 3)) + 4 * (col & 3);
  }

  float16v_ acc[kNB][kNB];
#pragma unroll
  for (int bi = 0; bi < kNB; bi++)
#pragma unroll
    for (int bj = 0; bj < kNB; bj++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[bi][bj][r] = 0.0f;
  prefer_agpr_accumulators();

  struct Frag {
    float a[kNB][4];  // [block][step of the group]
    float b[kNB][4];
  };
  Frag f[2];
  auto read_group = [&](Frag& fr, uint32_t s, auto gc) {
    constexpr int g = decltype(gc)::value;
#pragma unroll
    for (int bi = 0; bi < kNB; bi++) {
      const float4v v = lds_read_f4(s + aoff[bi][g]);
#pragma unroll
      for (int q = 0; q < 4; q++) fr.a[bi][q] = v[q];
    }
#pragma unroll
    for (int bj = 0; bj < kNB; bj++)
#pragma unroll
      for (int q = 0; q < 4; q++) fr.b[bj][q] = lds_read_f32(s + boff[bj] + (4 * g + q) * W::kBRow);
  };
  // Read i of a group (0 .. kReads - 1): the 16-byte A read of block i
  // (i < kNB), else the two B values of block (i - kNB) / 2, steps
  // 2 ((i - kNB) % 2) and + 1.
  auto read_one = [&](Frag& fr, uint32_t s, int g, int i) {
    if (i < kNB) {
      const float4v v = lds_read_f4(s + aoff[i][g]);
#pragma unroll
      for (int q = 0; q < 4; q++) fr.a[i][q] = v[q];
    } else {
      const int bj = (i - kNB) >> 1, q = 2 * ((i - kNB) & 1);
      fr.b[bj][q] = lds_read_f32(s + boff[bj] + (4 * g + q) * W::kBRow);
      fr.b[bj][q + 1] = lds_read_f32(s + boff[bj] + (4 * g + q + 1) * W::kBRow);
    }
  };
  auto mfma_step = [&](const Frag& fr, int q) {
#pragma unroll
    for (int bi = 0; bi < kNB; bi++)
#pragma unroll
      for (int bj = 0; bj < kNB; bj++)
        acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(fr.a[bi][q], fr.b[bj][q], acc[bi][bj], 0, 0, 0);
  };

  // Prologue: k-tiles 0 and 1 (clamped) in flight, k-tile 0 waited for.
#pragma unroll
  for (int d = 0; d < kD; d++) issue_one(0, 0, d);
#pragma unroll
  for (int d = 0; d < kD; d++) issue_one(min(1, nk - 1), 1, d);
  wait_vmcnt<kD>();
  lds_barrier();
  read_group(f[0], lds_base, std::integral_constant<int, 0>{});
#if VK_TIMELINE
  const unsigned long long tl_loop_rt = __builtin_amdgcn_s_memrealtime();
  const unsigned long long tl_loop_c = __builtin_amdgcn_s_memtime();
#endif

  for (int t = 0; t < nk; t++) {
    const uint32_t s = lds_base + (t & 1) * W::kStageBytes;
    static_for<4>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
#if VK_TIMELINE
      unsigned long long tl_b0 = 0;
      if constexpr (g == 3) tl_b0 = __builtin_amdgcn_s_memtime();
#endif
      __builtin_amdgcn_sched_barrier(0);
      mfma_step(f[g & 1], 0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (g < 3) {
        // steps 1..3, the next group's reads one after each of the first
        // kReads MFMAs
        static_for<3>([&](auto qc) {
          constexpr int q = decltype(qc)::value + 1;
          if constexpr ((q - 1) * kNB * kNB < W::kReads) {
#pragma unroll
            for (int bi = 0; bi < kNB; bi++)
#pragma unroll
              for (int bj = 0; bj < kNB; bj++) {
                const int m = (q - 1) * kNB * kNB + kNB * bi + bj;
                acc[bi][bj] =
                    __builtin_amdgcn_mfma_f32_32x32x2f32(f[g & 1].a[bi][q], f[g & 1].b[bj][q], acc[bi][bj], 0, 0, 0);
                if (m < W::kReads) {
                  __builtin_amdgcn_sched_barrier(0);
                  read_one(f[(g + 1) & 1], s, g + 1, m);
                }
                __builtin_amdgcn_sched_barrier(0);
              }
          } else {
            __builtin_amdgcn_sched_barrier(0);
            mfma_step(f[g & 1], q);
          }
        });
      } else {
        wait_lgkmcnt0();
        wait_vmcnt<0>();  // this wave's loads of k-tile t + 1
        lds_barrier();    // everyone's; also ends every read of slot t & 1
#if VK_TIMELINE
        tl_bar += __builtin_amdgcn_s_memtime() - tl_b0;
#endif
        const uint32_t s_next = lds_base + ((t + 1) & 1) * W::kStageBytes;
        const int kt_next = min(t + 2, nk - 1);
        // steps 1..3: the next k-tile's first kReads reads after the first
        // kReads MFMAs, a load after every kLoadEvery-th, A and B alternating
#pragma unroll
        for (int q = 1; q < 4; q++)
#pragma unroll
          for (int bi = 0; bi < kNB; bi++)
#pragma unroll
            for (int bj = 0; bj < kNB; bj++) {
              const int m = kNB * kNB * (q - 1) + kNB * bi + bj;
              __builtin_amdgcn_sched_barrier(0);
              acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(f[1].a[bi][q], f[1].b[bj][q], acc[bi][bj], 0, 0, 0);
              if (m < W::kReads) {
                __builtin_amdgcn_sched_barrier(0);
                read_one(f[0], s_next, 0, m);
              }
#pragma unroll
              for (int d = W::load_begin(m); d < W::load_begin(m + 1); d++) {
                __builtin_amdgcn_sched_barrier(0);
                issue_one(kt_next, t & 1, (d & 1) ? kDA + (d >> 1) : (d >> 1));
              }
            }
      }
    });
  }
  wait_vmcnt<0>();  // clamped refills past the last k-tile
#if VK_TIMELINE
  const unsigned long long tl_end_c = __builtin_amdgcn_s_memtime();
  const unsigned long long tl_end_rt = __builtin_amdgcn_s_memrealtime();
#endif

  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  unsigned* cnt = nullptr;
  const bool split = kSplit && w.np > 1;  // whole tiles of a tail plan store at once
  if (split) {
    const __amdgpu_buffer_rsrc_t prsrc =
        __builtin_amdgcn_make_buffer_rsrc(part, 0, (int)((size_t)units * f32_slot_bytes(kNB)), kBufferWord3);
    const SkPlan plan{dp, units, pieces, chunks};
    const int T = tiles_m * tiles_n;
    auto part_off = [&](int q) {
      return (uint32_t)((size_t)sk_unit_of(plan, T, w.tile, q) * f32_slot_bytes(kNB)) +
             (uint32_t)wave * f32_wave_bytes(kNB);
    };
    cnt = counters + (size_t)w.tile * kSkWaves + wave;
    if (!f32_split_arrive(acc, w.np, w.p, lane_e, prsrc, part_off, cnt)) return;
    f32_split_sum(acc, w.np, w.p, lane_e, prsrc, part_off);
  }
  const int row0 = m0 + wr * kQ, col0 = n0 + wc * kQ;
#pragma unroll
  for (int bi = 0; bi < kNB; bi++)
#pragma unroll
    for (int bj = 0; bj < kNB; bj++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = row0 + bi * 32 + 8 * (r >> 2) + 4 * (lane_e >> 5) + (r & 3);
        const int col = col0 + bj * 32 + (lane_e & 31);
        if (!kEdge || (row < M && col < N)) C[(size_t)row * N + col] = acc[bi][bj][r];
      }
  if (split && lane_e == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#if VK_TIMELINE
  wait_vmcnt0_ordered();
  const unsigned long long tl_exit = __builtin_amdgcn_s_memrealtime();
  const int rec = (int)blockIdx.x * 4 + wave;
  if (lane == 0 && rec < kF32TimelineWaves) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    unsigned long long* r = vk_timeline_f32 + rec * 8;
    r[0] = tl_entry; r[1] = tl_loop_rt; r[2] = tl_end_rt; r[3] = tl_exit; r[4] = xcc & 15u;
    r[5] = tl_end_c - tl_loop_c; r[6] = tl_bar; r[7] = (unsigned long long)nk;
  }
#endif
}

template <int kNB, bool kEdge, bool kSplit, bool kKMask = false>
hipError_t launch_w4(const GemmArgs& a, const SkPlan& p) {
  using W = F32W4<kNB>;
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f32_mfma4_kernel<kNB, kEdge, kSplit, kKMask>;
  hipError_t e = ensure_lds_attr(kfn, W::kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  unsigned* counters = nullptr;
  float* part = nullptr;
  if constexpr (kSplit) {
    counters = static_cast<unsigned*>(a.workspace);
    part = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + kSkCounterBytes);
    if (!a.workspace_clean) {
      e = zero_words(counters, kSkCounterBytes / sizeof(unsigned), a.stream);
      if (e != hipSuccess) return e;
    }
  }
  const int grid = kSplit ? p.dp + p.units : (int)f32_tiles(a.m, a.n, W::kT);
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(256), W::kLdsBytes, a.stream, static_cast<const float*>(a.A),
                     static_cast<const float*>(a.B), static_cast<float*>(a.C), (int)a.m, (int)a.n, (int)a.k, p.dp,
                     p.units, p.pieces, p.chunks, f32_last_extra(p), part, counters);
  return hipGetLastError();
}

bool f32_mfma_edge_shape_ok(size_t m, size_t n, size_t k);

// The 128x128 or 64x64 tiles (f32_small_tiles, f32_small_nb), K split
// where they fill at most half of the CUs or leave the last round part
// empty; K % 32 != 0 through the edge kernel with the k mask (also on
// version 2's grid, whose 16-deep eight-wave kernel has 256x256 tiles only;
// the caller checks the edge kernel's size limits).
template <int kNB, bool kEdge>
hipError_t launch_f32_small_nb(const GemmArgs& a) {
  const SkPlan p = f32_plan(a.m, a.n, a.k, a.num_cus, kNB);
  if (a.k % 32 != 0)
    return p.units > 0 ? launch_w4<kNB, true, true, true>(a, p) : launch_w4<kNB, true, false, true>(a, p);
  return p.units > 0 ? launch_w4<kNB, kEdge, true>(a, p) : launch_w4<kNB, kEdge, false>(a, p);
}
template <bool kEdge>
hipError_t launch_f32_small(const GemmArgs& a) {
  return f32_small_nb(a.m, a.n, a.num_cus) == 1 ? launch_f32_small_nb<1, kEdge>(a) : launch_f32_small_nb<2, kEdge>(a);
}

// Workspace of versions 2 and 3: the split's counters and partials.
size_t f32_workspace(size_t m, size_t n, size_t k, int num_cus) {
  if (!f32_small_tiles(m, n, num_cus) || (k % 32 != 0 && !f32_mfma_edge_shape_ok(m, n, k))) return 0;
  const int nb = f32_small_nb(m, n, num_cus);
  const SkPlan p = f32_plan(m, n, k, num_cus, nb);
  return p.units > 0 ? kSkCounterBytes + (size_t)p.units * f32_slot_bytes(nb) : 0;
}

// 32-deep k-tiles when K allows (one barrier per 128 MFMAs of a wave:
// measured 141.2 against 139.6 TFLOP/s at 4096^3), else 16-deep.
template <int BK, bool kEdge = false>
hipError_t launch_bk(const GemmArgs& a) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f32_mfma_kernel<BK, kEdge>;
  hipError_t e = ensure_lds_attr(kfn, F32Cfg<BK>::kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  const int tiles = kEdge ? (int)(((a.m + kBM - 1) / kBM) * ((a.n + kBN - 1) / kBN)) : (int)((a.m / kBM) * (a.n / kBN));
  hipLaunchKernelGGL(kfn, dim3(tiles), dim3(kThreads), F32Cfg<BK>::kLdsBytes, a.stream,
                     static_cast<const float*>(a.A), static_cast<const float*>(a.B), static_cast<float*>(a.C),
                     (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

// 256x256 tiles where they take as few rounds of the CUs as 128x128 ones
// (the four-wave kernel when K % 32 == 0, else the eight-wave one with
// 16-deep k-tiles), otherwise the 128x128 tiles.
hipError_t launch_f32_mfma(const GemmArgs& a) {
  if (f32_small_tiles(a.m, a.n, a.num_cus) && (a.k % 32 == 0 || f32_mfma_edge_shape_ok(a.m, a.n, a.k)))
    return launch_f32_small<false>(a);
  return a.k % 32 == 0 ? launch_w4<4, false, false>(a, SkPlan{0, 0, 1, 1}) : launch_bk<16>(a);
}

// 32-bit lane offsets: the rows of A one instruction covers span less than
// 256 * K floats beyond the k-tile base and the k-rows of B 32 * N floats;
// the per-k-tile and per-tile steps are 64-bit scalar bases.
bool f32_mfma_shape_ok(size_t m, size_t n, size_t k) {
  return (size_t)256 * k * 4 < (1ull << 31) && (size_t)32 * n * 4 < (1ull << 31) &&
         (m / kBM) * (n / kBN) < (1ull << 31);
}

// Version 3 (any M; N, K multiples of 4): 32-deep k-tiles (the last one
// masked where K % 32 != 0); each operand below 2^31 bytes (buffer sizes and
// offsets).
hipError_t launch_f32_mfma_edge(const GemmArgs& a) {
  if (f32_small_tiles(a.m, a.n, a.num_cus)) return launch_f32_small<true>(a);
  return a.k % 32 == 0 ? launch_w4<4, true, false>(a, SkPlan{0, 0, 1, 1}) : launch_bk<32, true>(a);
}

bool f32_mfma_edge_shape_ok(size_t m, size_t n, size_t k) {
  return m >= 1 && n >= 4 && k >= 4 && m * k * 4 < (1ull << 31) && k * n * 4 < (1ull << 31) &&
         f32_mfma_shape_ok(((m + kBM - 1) / kBM) * kBM, ((n + kBN - 1) / kBN) * kBN, k);
}

}  // namespace

void register_f32_mfma() {
  KernelEntry e{};
  e.version = 2;
  e.in_dtype = VK_DTYPE_F32;
  e.name = "f32_v2_mfma256";
  e.caps = make_caps(2, VK_DTYPE_F32, kOutF32, kBM, kBN, 16, 16, kBM, kBN, 32, 256, F32Cfg<32>::kLdsBytes, 0, 0);
  e.caps.uses_workspace = 1;  // K split on grids of few tiles
  e.launch = launch_f32_mfma;
  e.workspace = f32_workspace;
  e.shape_ok = f32_mfma_shape_ok;
  register_kernel(e);

  KernelEntry e3 = e;
  e3.version = 3;
  e3.name = "f32_v3_mfma256_edge";
  e3.caps = make_caps(3, VK_DTYPE_F32, kOutF32, 1, 4, 4, 16, kBM, kBN, 32, 256, F32Cfg<32>::kLdsBytes, 0, 0);
  e3.caps.uses_workspace = 1;
  e3.launch = launch_f32_mfma_edge;
  e3.shape_ok = f32_mfma_edge_shape_ok;
  register_kernel(e3);
}

}  // namespace vk
