// f16_pingpong.hip -- fp16 GEMM, version 5: 256x256 tile, 8 waves in two
// phase-shifted groups ("ping-pong").
//
// Same job and tile as version 3 (f16_dma.hip; the reference's champion is
// results/ralph_loop_fable/src/matmul_f16/matmul_f16_v42_shfl2.cu:104-490),
// but with two waves per SIMD instead of one.  A 512-thread workgroup places
// waves w and w + 4 on the same SIMD, so the waves form two groups, P = waves
// 0..3 and Q = waves 4..7, one wave of each per SIMD:
//
//  * P computes rows 0..127 of the tile, Q rows 128..255; wave g of a group
//    owns columns 64g..64g+63, i.e. a 128x64 block = 4x2 MFMA 32x32x16 blocks
//    (128 fp32 accumulators per lane).
//  * The k-loop alternates two phases separated by workgroup barriers:
//      memory phase:  issue this wave's share of a future k-tile's
//                     global->LDS loads and read the current k-tile's
//                     fragments from LDS into registers;
//      compute phase: 16 MFMAs on those fragments, nothing else.
//    Q starts one phase later than P (one extra barrier at the start, P takes
//    one at the end), so in every phase one wave of each SIMD issues only
//    MFMAs while its partner reads LDS and issues loads: the matrix pipe is
//    never left waiting on LDS latency, and a barrier costs only its own
//    latency, hidden behind the MFMAs already issued.
//  * LDS: a 4-stage ring of (A 256x32, B 32x256) k-tiles, 32 KB per stage,
//    same swizzles as version 3.  P loads the B half of each k-tile and Q the
//    A half, 4 direct-to-LDS instructions per wave per k-tile.
//
// Timeline (phase f = the interval between barriers f and f+1 after the
// prologue barrier; t = k-tile):
//    P: memory(t) in phase 2t,   compute(t) in phase 2t+1
//    Q: memory(t) in phase 2t+1, compute(t) in phase 2t+2
// Stage t % 4 is read in phases 2t (P) and 2t+1 (Q), so it is free from phase
// 2t+2 on; memory(t) refills stage (t-1) % 4 with k-tile t+3.  Every wave
// makes its loads of k-tile t+1 complete (vmcnt) before barrier 2t+2, the
// first phase that reads that tile: P after compute(t), Q after memory(t).
// Both groups pass the same number of barriers: 1 + 1 + 2 nk + 1.
#include "vk_device.hpp"
#include "vk_internal.hpp"
#include "vk_splittail.hpp"
#include "vk_tile.hpp"

#include <algorithm>
#include <atomic>
#include <type_traits>

// Timeline build (make timeline -> libvk_gemm_timeline.so, VK_TIMELINE=1):
// version 7's kernel also records, for waves 0 and 4 of each workgroup (one
// per group), its XCD and the 100 MHz real-time clock at entry, after the
// prologue (the first MFMA), after the k-loop, after the epilogue's stores
// are issued and after they complete; vk_timeline_read() copies them out.
// The product library is built with VK_TIMELINE=0 and records nothing.
#ifndef VK_TIMELINE
#define VK_TIMELINE 0
#endif
#if VK_TIMELINE
constexpr int kTimelineGroups = 4096;  // workgroups recorded (the first 4096 of a launch)
__device__ unsigned long long vk_timeline[kTimelineGroups * 2 * 8];
extern "C" int vk_timeline_read(unsigned long long* host, int records) {
  if (records < 0 || records > kTimelineGroups * 2) return -3;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(vk_timeline), sizeof(unsigned long long) * 8 * records, 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : -7;
}
#endif

namespace vk {
namespace {

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 32;
constexpr int kNS = 4;  // LDS ring stages
constexpr int kThreads = 512;
constexpr int kABytes = kBM * kBK * 2;          // 16 KB
constexpr int kBBytes = kBK * kBN * 2;          // 16 KB
constexpr int kStageBytes = kABytes + kBBytes;  // 32 KB
constexpr int kLdsBytes = kNS * kStageBytes;    // 128 KB
constexpr int kDma = 4;                         // direct-to-LDS instructions per wave per k-tile
// Outstanding loads allowed when k-tile t+1 must have landed: k-tiles t+2 ..
// t+kNS-1 of this wave.
constexpr int kVmWait = (kNS - 2) * kDma;
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(kLdsBytes >= 8 * 128 * 64 * 2, "fp16 epilogue staging: 16 KB per wave");

// fp16 output block of one wave (128 x 64) staged in LDS: row pitch 128 B =
// 16 units of 8 B (4 halves); unit u of row r sits at unit u ^ (r % 16).
// The MFMA lanes that write together hold the same 8-byte unit of 16
// consecutive rows, which this spreads over all 16 unit positions of the
// 128-byte row: measured on MI355X, the writes have no bank conflicts (the
// previous layout, 16-byte chunks XOR (r / 2) % 8, cost 4 conflict cycles per
// write instruction: all 262,144 of the 4096^3 kernel's conflict cycles).
__device__ __forceinline__ uint32_t epi16_unit_addr(uint32_t base, int row, int unit) {
  return base + row * 128 + 8 * (unit ^ (row & 15));
}
// The 16 bytes of units 2ch and 2ch+1 of a row: one 16-byte read at unit
// pair ch ^ (r / 2) % 8, whose two halves come swapped when r is odd.  (Also
// conflict-free, measured: 8 rows x 8 pairs per instruction.)
__device__ __forceinline__ uint4v epi16_read_pair(uint32_t base, int row, int ch) {
  const uint4v v = lds_read16(base + row * 128 + 16 * (ch ^ ((row >> 1) & 7)));
  const bool odd = row & 1;
  return uint4v{odd ? v[2] : v[0], odd ? v[3] : v[1], odd ? v[0] : v[2], odd ? v[1] : v[3]};
}

template <typename OutT>
__device__ __forceinline__ typename std::enable_if<std::is_same<OutT, half_t>::value>::type
epilogue_store(float16v (&acc)[4][2], uint32_t wbase, OutT* Cw, int N, int lane) {
  // MFMA output of block (i, j) (C^T form, see the k-loop): lane l, register
  // 4*g4 + e holds C[i*32 + l%32][j*32 + 8*g4 + 4*(l/32) + e].
  const int r0 = lane & 31, hsel = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const int row = i * 32 + r0;
        half4 h = {(half_t)acc[i][j][4 * g4 + 0], (half_t)acc[i][j][4 * g4 + 1],
                   (half_t)acc[i][j][4 * g4 + 2], (half_t)acc[i][j][4 * g4 + 3]};
        lds_write8(epi16_unit_addr(wbase, row, 2 * (4 * j + g4) + hsel), h);
      }
  // Read back 8 rows x 8 chunks per instruction: each row a full 128-byte line.
  const int rsub = lane >> 3, ch = lane & 7;
#pragma unroll
  for (int q = 0; q < 16; q++) {
    const int row = 8 * q + rsub;
    const uint4v v = epi16_read_pair(wbase, row, ch);
    *reinterpret_cast<uint4v*>(Cw + (size_t)row * N + ch * 8) = v;
  }
}

// fp32 output: two passes of 64 rows (16 KB per wave each), row pitch 256 B =
// 16 chunks, physical chunk = chunk ^ (row % 16); 4 rows per read.
template <typename OutT>
__device__ __forceinline__ typename std::enable_if<std::is_same<OutT, float>::value>::type
epilogue_store(float16v (&acc)[4][2], uint32_t wbase, OutT* Cw, int N, int lane) {
  const int r0 = lane & 31, hsel = lane >> 5;
#pragma unroll
  for (int pass = 0; pass < 2; pass++) {
#pragma unroll
    for (int ii = 0; ii < 2; ii++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          const int i = 2 * pass + ii;
          const int row = ii * 32 + r0;  // row within this pass
          const int chunk = 8 * j + 2 * g4 + hsel;
          float4v f = {acc[i][j][4 * g4 + 0], acc[i][j][4 * g4 + 1], acc[i][j][4 * g4 + 2],
                       acc[i][j][4 * g4 + 3]};
          lds_write16(wbase + row * 256 + 16 * (chunk ^ (row & 15)), f);
        }
    const int rsub = lane >> 4, ch = lane & 15;
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const int row = 4 * q + rsub;
      const uint4v v = lds_read16(wbase + row * 256 + 16 * (ch ^ (row & 15)));
      *reinterpret_cast<uint4v*>(Cw + (size_t)(pass * 64 + row) * N + ch * 4) = v;
    }
    if (pass == 0) wait_lgkmcnt0();  // this wave's region is rewritten by the next pass
  }
}

template <typename OutT>
__global__ __launch_bounds__(kThreads) void f16_pp_kernel(const half_t* __restrict__ A,
                                                          const half_t* __restrict__ B,
                                                          OutT* __restrict__ C, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;  // 0 = P, 1 = Q; waves w and w+4 share a SIMD
  const int gw = wave & 3;

  int tm, tn;
  tile_of(blockIdx.x, M / kBM, N / kBN, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  // ---- this wave's direct-to-LDS duty: P the B k-tile, Q the A k-tile ----
  // A: instruction i covers rows gw*64 + i*16 .. +15 (4 chunks of 16 B each);
  // B: instruction i covers k-rows gw*8 + 2i, +1 (32 chunks each).  Either way
  // it lands at stage offset (grp ? 0 : kABytes) + (gw*4 + i) * 1024.
  uint32_t doff[kDma];
  const char* gsrc;
  size_t gstep;  // bytes between consecutive k-tiles of the source
  if (grp) {
#pragma unroll
    for (int i = 0; i < kDma; i++) {
      const int row = gw * 64 + i * 16 + (lane >> 2);
      const int c = (lane & 3) ^ swz_a<kBK>(row);
      doff[i] = (uint32_t)(((size_t)row * K + c * 8) * 2);
    }
    gsrc = reinterpret_cast<const char*>(A) + (size_t)m0 * K * 2;
    gstep = (size_t)kBK * 2;
  } else {
#pragma unroll
    for (int i = 0; i < kDma; i++) {
      const int krow = gw * 8 + i * 2 + (lane >> 5);
      const int c = (lane & 31) ^ swz_b(krow);
      doff[i] = (uint32_t)(((size_t)krow * N + c * 8) * 2);
    }
    gsrc = reinterpret_cast<const char*>(B) + (size_t)n0 * 2;
    gstep = (size_t)kBK * N * 2;
  }
  const uint32_t ddst = (grp ? 0u : (uint32_t)kABytes) + gw * 4 * 1024;

  // ---- fragment addresses (bytes inside a stage) ----
  // A block i, k-step ks: row grp*128 + i*32 + lane%32, chunk 2*ks + lane/32.
  const int arow = grp * 128 + (lane & 31);
  uint32_t aoff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ks++) aoff[ks] = arow * (kBK * 2) + 16 * ((2 * ks + (lane >> 5)) ^ swz_a<kBK>(arow));
  // B block j, k-step ks, half h: lane 16g + 4jj + q names k-row
  // ks*16 + 8*(g/2) + 4h + jj, columns gw*64 + j*32 + 16*(g%2) + 4q .. +3; the
  // transpose read hands lane 16g + i the 4 k of column 16*(g%2) + i.
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  uint32_t boff[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int krow0 = 8 * (g >> 1) + jj;  // plus ks*16 + 4h: krow0 % 4 is unchanged
    const int c = gw * 8 + j * 4 + 2 * (g & 1) + (q >> 1);
    boff[j] = kABytes + krow0 * (kBN * 2) + 16 * (c ^ swz_b(krow0)) + 8 * (q & 1);
  }

  float16v acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  half8 fa[2][4], fb[2][2];
  const int nk = K / kBK;
  prefer_agpr_accumulators();

  auto issue = [&](int stage, int kt) {
    const uint32_t dst = lds_base + stage * kStageBytes + ddst;
    const char* src = gsrc + (size_t)kt * gstep;
#pragma unroll
    for (int i = 0; i < kDma; i++) dma16(src, doff[i], dst + i * 1024);
  };
  auto read_frags = [&](int stage) {
    const uint32_t sb = lds_base + stage * kStageBytes;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
#pragma unroll
      for (int i = 0; i < 4; i++) fa[ks][i] = lds_read_h8(sb + aoff[ks] + i * 32 * kBK * 2);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const uint32_t p = sb + boff[j] + ks * 16 * kBN * 2;
        const half4 lo = lds_read_tr16_at(p);
        const half4 hi = lds_read_tr16_at(p + 4 * kBN * 2);
        fb[ks][j] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  };
  // The B fragment is the MFMA's first operand, so each block computes C^T:
  // lane l then holds 4 consecutive columns of row l % 32 (see the epilogue).
  auto compute = [&]() {
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = mfma32x32x16(fb[ks][j], fa[ks][i], acc[i][j]);
  };

  // Prologue: k-tiles 0..kNS-2 in flight; tile 0 landed everywhere after the
  // barrier.  Then Q takes one extra barrier so that it runs one phase behind.
#pragma unroll
  for (int s = 0; s < kNS - 1; s++) issue(s, min(s, nk - 1));
  wait_vmcnt<kVmWait>();
  lds_barrier();
  if (grp) lds_barrier();

  // Every iteration runs the same code for both groups; refills past the last
  // k-tile are clamped to it and land in a stage that is never read again,
  // which keeps the vmcnt bookkeeping constant.
  for (int t = 0; t < nk; t++) {
    __builtin_amdgcn_sched_barrier(0);
    issue((t + kNS - 1) % kNS, min(t + kNS - 1, nk - 1));
    read_frags(t % kNS);
    if (grp) wait_vmcnt<kVmWait>();  // Q: k-tile t+1 landed before barrier 2t+2
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    compute();
    if (!grp) wait_vmcnt<kVmWait>();  // P: k-tile t+1 landed before barrier 2t+2
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!grp) lds_barrier();
  // Drain the clamped tail refills before any wave reuses the ring for the
  // epilogue (and before the workgroup can exit).
  wait_vmcnt<0>();
  lds_barrier();

  epilogue_store<OutT>(acc, lds_base + wave * (128 * 64 * 2),
                       C + (size_t)(m0 + grp * 128) * N + n0 + gw * 64, N, lane);
}

template <typename OutT>
hipError_t launch_pp_t(const GemmArgs& a) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp_kernel<OutT>;
  hipError_t e = ensure_lds_attr(kfn, kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  const int tiles = (int)((a.m / kBM) * (a.n / kBN));
  hipLaunchKernelGGL(kfn, dim3(tiles), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B),
                     static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

hipError_t launch_pp(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_pp_t<half_t>(a) : launch_pp_t<float>(a);
}

// 32-bit byte offsets inside one 256-row panel of A and one 32-row slab of B
// must not overflow; the grid is 1-D.
bool pp_shape_ok(size_t m, size_t n, size_t k) {
  return (size_t)kBM * k * 2 < (1ull << 31) && (size_t)kBK * n * 2 < (1ull << 31) &&
         (m / kBM) * (n / kBN) < (1ull << 31);
}


// ---------------------------------------------------------------------------
// Version 6: the same ping-pong with 64-deep k-tiles, so each phase holds 32
// MFMAs (1024 matrix-core cycles) and the barrier pair costs half as much per
// FLOP, and with the global->LDS loads moved out of the memory phase.
//
// Measured on version 5 and on a first 64-deep variant: a wave that issues its
// direct-to-LDS loads at the start of its memory phase stalls on them (the
// texture unit accepts one 1 KB load instruction about every 16 cycles per
// CU), and its LDS reads queue behind them.  Here the memory phase holds only
// the LDS fragment reads, and each wave issues its 8 loads of a k-tile during
// its compute phase, one after every 4 MFMAs, where the wait costs nothing.
//
// LDS ring, split by reader (160 KB):
//    A-top  rows   0..127 of the A k-tile, read by P     2 slots x 16 KB
//    A-bot  rows 128..255,                   read by Q     2 slots x 16 KB
//    B      64 x 256,                        read by both  3 slots x 32 KB
//
// Phases as in version 5 (P: memory(t) in phase 2t, compute(t) in 2t+1; Q one
// phase later).  During compute(t):
//    P loads B(t+2)                 -> B slot (t+2)%3 (B(t-1), read by phase 2t-1)
//    Q loads A-top(t+2), A-bot(t+2) -> slot t%2 (A-top(t) read in phase 2t,
//                                      A-bot(t) in phase 2t+1)
// and the waits that make a k-tile land before the first barrier that opens a
// phase reading it are:
//    P after compute(t):  vmcnt(8)  B(t+1)                   (barrier 2t+2)
//    Q after memory(t):   vmcnt(4)  A-top(t+1)               (barrier 2t+2)
//    Q after compute(t):  vmcnt(8)  A-top(t+1), A-bot(t+1)   (barrier 2t+3)
// Refills past the last k-tile are clamped to it and land in slots that are
// never read again.
namespace pp64 {

constexpr int kBK = 64;
constexpr int kHalfBytes = 128 * kBK * 2;  // 16 KB: one A half-tile
constexpr int kBBytes = kBK * kBN * 2;     // 32 KB
constexpr int kATop = 0;                   // 2 slots
constexpr int kABot = 2 * kHalfBytes;      // 2 slots
constexpr int kBOff = 4 * kHalfBytes;      // 3 slots
constexpr int kBSlots = 3;
constexpr int kLdsBytes = kBOff + kBSlots * kBBytes;  // 160 KB
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(kLdsBytes >= 8 * 128 * 64 * 2, "fp16 epilogue staging: 16 KB per wave");

template <typename OutT>
__global__ __launch_bounds__(kThreads) void f16_pp64_kernel(const half_t* __restrict__ A,
                                                            const half_t* __restrict__ B,
                                                            OutT* __restrict__ C, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;  // 0 = P, 1 = Q; waves w and w+4 share a SIMD
  const int gw = wave & 3;

  int tm, tn;
  tile_of(blockIdx.x, M / kBM, N / kBN, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  // ---- direct-to-LDS duty: 8 instructions (8 KB) per wave per k-tile ----
  // Instruction d = 4h + i (h = 0, 1; i = 0..3) uses lane offset voff[i]; the
  // h step and the slot are wave-uniform address terms, so both groups run the
  // same branch-free code with different scalars.
  // Q, A: rows gw*32 + 8i .. +7 of the A-top (h = 0) or A-bot (h = 1) half (8
  //   chunks of 16 B per row), landing at half offset (gw*4 + i) * 1024.
  // P, B: k-rows gw*16 + 2i + 8h, +1 (32 chunks each), landing at B offset
  //   (gw*8 + 4h + i) * 1024; +8 k-rows keep the swizzle.
  uint32_t voff[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (grp) {
      const int row = gw * 32 + i * 8 + (lane >> 3);
      const int c = (lane & 7) ^ swz_a<kBK>(row);
      voff[i] = (uint32_t)(((size_t)row * K + c * 8) * 2);
    } else {
      const int krow = gw * 16 + i * 2 + (lane >> 5);
      const int c = (lane & 31) ^ swz_b(krow);
      voff[i] = (uint32_t)(((size_t)krow * N + c * 8) * 2);
    }
  }
  const char* a_top = reinterpret_cast<const char*>(A) + (size_t)m0 * K * 2;
  const char* b_src = reinterpret_cast<const char*>(B) + (size_t)n0 * 2;
  const char* g_base = grp ? a_top : b_src;
  const size_t g_kt = grp ? (size_t)kBK * 2 : (size_t)kBK * N * 2;    // per k-tile
  const size_t g_h = grp ? (size_t)128 * K * 2 : (size_t)8 * N * 2;   // per h
  const uint32_t l_base = lds_base + (grp ? (uint32_t)kATop + gw * 4 * 1024 : (uint32_t)kBOff + gw * 8 * 1024);
  const uint32_t l_slot = grp ? (uint32_t)kHalfBytes : (uint32_t)kBBytes;  // per slot
  const uint32_t l_h = grp ? (uint32_t)(kABot - kATop) : 4096u;           // per h

  // Load instruction d (0..7) of k-tile kt into slot `slot` (P: a B slot, Q:
  // an A slot).
  auto dma = [&](int d, int kt, int slot) {
    const char* g = g_base + (size_t)kt * g_kt + (d >> 2) * g_h;
    dma16(g, voff[d & 3], l_base + slot * l_slot + (d >> 2) * l_h + (d & 3) * 1024);
  };

  // ---- fragment addresses ----
  // A block i, k-step ks: half-row i*32 + lane%32, chunk 2*ks + lane/32.
  const int arow = lane & 31;
  const uint32_t a_half = grp ? kABot : kATop;
  uint32_t aoff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ks++)
    aoff[ks] = a_half + arow * (kBK * 2) + 16 * ((2 * ks + (lane >> 5)) ^ swz_a<kBK>(arow));
  // B block j, k-step ks, half h: as version 5 (k-row ks*16 + 8*(g/2) + 4h + jj).
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  uint32_t boff[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int krow0 = 8 * (g >> 1) + jj;
    const int c = gw * 8 + j * 4 + 2 * (g & 1) + (q >> 1);
    boff[j] = kBOff + krow0 * (kBN * 2) + 16 * (c ^ swz_b(krow0)) + 8 * (q & 1);
  }

  float16v acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  half8 fa[4][4], fb[4][2];
  const int nk = K / kBK;
  prefer_agpr_accumulators();

  auto read_frags = [&](int aslot, int bslot) {
    const uint32_t sa = lds_base + aslot * kHalfBytes;
    const uint32_t sb = lds_base + bslot * kBBytes;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
#pragma unroll
      for (int i = 0; i < 4; i++) fa[ks][i] = lds_read_h8(sa + aoff[ks] + i * 32 * kBK * 2);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const uint32_t p = sb + boff[j] + ks * 16 * kBN * 2;
        const half4 lo = lds_read_tr16_at(p);
        const half4 hi = lds_read_tr16_at(p + 4 * kBN * 2);
        fb[ks][j] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  };
  // 32 MFMAs with the 8 loads of k-tile kt interleaved, one after every 4.
  auto compute_and_load = [&](int kt, int slot) {
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = mfma32x32x16(fb[ks][j], fa[ks][i], acc[i][j]);
        if (i & 1) {
          __builtin_amdgcn_sched_barrier(0);
          dma(2 * ks + (i >> 1), kt, slot);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
  };

  // Prologue: P loads B(0), B(1); Q loads A-top(0), A-bot(0), A-top(1),
  // A-bot(1).  Barrier 0 needs A-top(0) and B(0); Q's extra barrier 1 needs
  // A-bot(0).  The rest is covered by the loop's own waits.
  const int kt1 = min(1, nk - 1);
#pragma unroll
  for (int d = 0; d < 8; d++) dma(d, 0, 0);
#pragma unroll
  for (int d = 0; d < 8; d++) dma(d, kt1, 1);
  if (grp)
    wait_vmcnt<12>();
  else
    wait_vmcnt<8>();
  lds_barrier();
  if (grp) {
    wait_vmcnt<8>();
    lds_barrier();
  }

  for (int t = 0; t < nk; t++) {
    const int aslot = t & 1;
    const int bslot = t % kBSlots;
    const int kt2 = min(t + 2, nk - 1);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(aslot, bslot);
    if (grp) wait_vmcnt<4>();  // Q: A-top(t+1) landed before barrier 2t+2
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    compute_and_load(kt2, grp ? aslot : (t + 2) % kBSlots);
    wait_vmcnt<8>();  // P: B(t+1); Q: A-top(t+1), A-bot(t+1)
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!grp) lds_barrier();
  wait_vmcnt<0>();
  lds_barrier();

  epilogue_store<OutT>(acc, lds_base + wave * (128 * 64 * 2),
                       C + (size_t)(m0 + grp * 128) * N + n0 + gw * 64, N, lane);
}

template <typename OutT>
hipError_t launch_t(const GemmArgs& a) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp64_kernel<OutT>;
  hipError_t e = ensure_lds_attr(kfn, kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  const int tiles = (int)((a.m / kBM) * (a.n / kBN));
  hipLaunchKernelGGL(kfn, dim3(tiles), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B),
                     static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

hipError_t launch(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_t<half_t>(a) : launch_t<float>(a);
}

// 32-bit lane offsets: 128 rows of A and 64 k-rows of B (the 4-row steps of B
// and the A-top -> A-bot step are folded into the 64-bit scalar base) must
// stay below 2^31 bytes.
bool shape_ok(size_t m, size_t n, size_t k) {
  return (size_t)128 * k * 2 < (1ull << 31) && (size_t)kBK * n * 2 < (1ull << 31) &&
         (m / kBM) * (n / kBN) < (1ull << 31);
}

}  // namespace pp64

// ---------------------------------------------------------------------------
// Version 7: version 6 with v_mfma_f32_16x16x32_f16 instead of the 32x32x16
// MFMA.  Same LDS bytes, loads, phases and waits; each wave's 128x64 block is
// 8x4 blocks of 16x16, 64 MFMAs of 16 cycles per 64-deep k-tile.
//
// Why: MI355X runs a sustained GEMM at its power limit, so FLOPs per joule set
// the clock.  Measured on a pure MFMA stream (random fp16 operands, 2 waves
// per SIMD, ~97% of issue slots busy): the 16x16x32 form holds ~1.84 GHz where
// the 32x32x16 form holds ~1.60 GHz.  Per multiply-add the 16x16x32 form moves
// half the accumulator data (256 outputs per 32-deep instruction instead of
// 1024 per 16-deep) for twice the operand data, 20% fewer register bytes.
//
// Layouts for the 16x16x32 shape (lane l):
//   A operand (the B fragment here, as in version 5): lane l holds 8
//     consecutive k of column l % 16, k = 8 * (l / 16) + e;
//   B operand (the A fragment): 8 consecutive k of row l % 16;
//   D: lane l, register r holds C^T[4 * (l / 16) + r][l % 16], i.e.
//     C[row l % 16][column 4 * (l / 16) + r].
// LDS swizzles, chosen for 16-lane (and 32-lane) access phases:
//   A rows (128 B = 8 chunks): chunk ^ ((row / 2) % 8): the 16 rows of one
//     fragment read fill the 16 16-byte slots of the 256-byte bank space;
//   B k-rows: version 5's chunk ^ {0, 6, 12, 10}[k % 4], additionally ^ 2 for
//     k-rows with bit 3 set, so the two 16-lane groups of a 32-lane phase
//     (k-rows 8 apart, same columns) use distinct slots.
namespace pp16 {

using pp64::kBK;
using pp64::kHalfBytes;
using pp64::kBBytes;
using pp64::kATop;
using pp64::kABot;
using pp64::kBOff;
using pp64::kBSlots;
using pp64::kLdsBytes;

__host__ __device__ constexpr int swz_a16(int row) { return (row >> 1) & 7; }
__host__ __device__ constexpr int swz_b16(int krow) { return swz_b(krow) ^ (((krow >> 3) & 1) << 1); }

// Leave-one-out instances of version 7 (versions 71-77): each turns off one
// ingredient of the k-loop or the tile order and keeps everything else, so
// that a kernel trace and counters show what that ingredient buys.  All of
// them compute every element in the same order as version 7 (bitwise equal
// results); none is ever picked.
constexpr int kAblNoSwzA = 1;      // A k-tile rows stored unswizzled (chunk c at slot c)
constexpr int kAblNoSwzB = 2;      // B k-rows stored unswizzled
constexpr int kAblRegStage = 4;    // global -> VGPR -> ds_write_b128 instead of direct-to-LDS loads
constexpr int kAblB2 = 8;          // B ring of 2 slots: B(t+1) loaded during compute(t) (prefetch 1 ahead)
constexpr int kAblNoPingPong = 16; // both groups in phase: all 8 waves read, then all compute
constexpr int kAblNoXcd = 32;      // grouped raster without the XCD remap
constexpr int kAblNoChain = 64;    // MFMAs rotate over the 32 accumulators (each one's first k-step for all, then the second)

template <int kAbl>
constexpr int lds_bytes_of() {
  return (kAbl & kAblB2) ? kBOff + 2 * kBBytes : kLdsBytes;
}
static_assert(lds_bytes_of<kAblB2>() >= 8 * 128 * 64 * 2, "fp16 epilogue staging: 16 KB per wave");

// Store of a wave's 128x64 block of C through its 16 KB LDS staging region,
// in two halves of 64 rows: stage() the 16 MFMA blocks (i, j) of a half, then
// flush() it.  Block (i, j), register r, lane l holds
// C[i*16 + l%16][j*16 + 4*(l/16) + r].
template <typename OutT>
struct Epi16;

// fp16: the whole 128x64 block fits the region (row pitch 128 B, see
// epi16_unit_addr), so only the second flush() stores, 8 rows x 8 chunks per
// read.
template <>
struct Epi16<half_t> {
  static __device__ __forceinline__ void stage(uint32_t wbase, int lane, int i, int j, const float4v& v) {
    const int r0 = lane & 15, g = lane >> 4;
    half4 h = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
    lds_write8(epi16_unit_addr(wbase, i * 16 + r0, 4 * j + g), h);
  }
  static __device__ __forceinline__ void flush(uint32_t wbase, half_t* Cw, int N, int lane, int half) {
    if (half == 0) return;
    const int rsub = lane >> 3, ch = lane & 7;
    const __amdgpu_buffer_rsrc_t cr = out_rsrc(Cw);  // 128 rows: offsets below 256 N <= 2^32
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const int row = 8 * q + rsub;
      const uint4v v = epi16_read_pair(wbase, row, ch);
      store_out16(cr, (uint32_t)(row * N + ch * 8) * 2u, v);
    }
  }
  // The same for a block at (row0, col0) of C that may reach past M rows or
  // N columns (N a multiple of 8): chunks outside are not stored.
  static __device__ __forceinline__ void flush_edge(uint32_t wbase, half_t* C, int M, int N, int row0, int col0,
                                                    int lane, int half) {
    if (half == 0) return;
    const int rsub = lane >> 3, ch = lane & 7;
    const bool col_in = col0 + ch * 8 < N;
    // Plain stores on the edge paths (version 10, the split tails with
    // edges): the sc1 stores that help the whole tiles made the 128 x 128
    // kernel's edge path slower at 1000^3.
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const int row = 8 * q + rsub;
      const uint4v v = epi16_read_pair(wbase, row, ch);
      if (col_in && row0 + row < M) *reinterpret_cast<uint4v*>(C + (size_t)(row0 + row) * N + col0 + ch * 8) = v;
    }
  }
};

// fp32: 64 rows per half (row pitch 256 B = 16 chunks, physical chunk =
// chunk ^ (row % 16)), 4 rows per read.
template <>
struct Epi16<float> {
  static __device__ __forceinline__ void stage(uint32_t wbase, int lane, int i, int j, const float4v& v) {
    const int row = (i & 3) * 16 + (lane & 15);  // row within the half
    const int chunk = 4 * j + (lane >> 4);
    lds_write16(wbase + row * 256 + 16 * (chunk ^ (row & 15)), v);
  }
  static __device__ __forceinline__ void flush(uint32_t wbase, float* Cw, int N, int lane, int half) {
    const int rsub = lane >> 4, ch = lane & 15;
    const __amdgpu_buffer_rsrc_t cr = out_rsrc(Cw + (size_t)(half * 64) * N);  // 64 rows: below 256 N
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const int row = 4 * q + rsub;
      const uint4v v = lds_read16(wbase + row * 256 + 16 * (ch ^ (row & 15)));
      store_out16(cr, (uint32_t)(row * N + ch * 4) * 4u, v);
    }
    if (half == 0) wait_lgkmcnt0();  // the region is rewritten by the second half
  }
  static __device__ __forceinline__ void flush_edge(uint32_t wbase, float* C, int M, int N, int row0, int col0,
                                                    int lane, int half) {
    const int rsub = lane >> 4, ch = lane & 15;
    const bool col_in = col0 + ch * 4 < N;
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const int row = 4 * q + rsub;
      const uint4v v = lds_read16(wbase + row * 256 + 16 * (ch ^ (row & 15)));
      const int r = row0 + half * 64 + row;
      if (col_in && r < M) *reinterpret_cast<uint4v*>(C + (size_t)r * N + col0 + ch * 4) = v;
    }
    if (half == 0) wait_lgkmcnt0();
  }
};

template <typename OutT>
__device__ __forceinline__ void epilogue16(float4v (&acc)[8][4], uint32_t wbase, OutT* Cw, int N, int lane) {
#pragma unroll
  for (int half = 0; half < 2; half++) {
#pragma unroll
    for (int i = 4 * half; i < 4 * half + 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) Epi16<OutT>::stage(wbase, lane, i, j, acc[i][j]);
    Epi16<OutT>::flush(wbase, Cw, N, lane, half);
  }
}

template <typename OutT>
__device__ __forceinline__ void epilogue16_edge(float4v (&acc)[8][4], uint32_t wbase, OutT* C, int M, int N,
                                                int row0, int col0, int lane) {
#pragma unroll
  for (int half = 0; half < 2; half++) {
#pragma unroll
    for (int i = 4 * half; i < 4 * half + 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) Epi16<OutT>::stage(wbase, lane, i, j, acc[i][j]);
    Epi16<OutT>::flush_edge(wbase, C, M, N, row0, col0, lane, half);
  }
}

// The k-loop of one 256x256 tile over k-tiles kb .. kb + nk - 1 (nk >= 1):
// zeroes `acc`, runs the prologue, the two-phase loop and the closing
// barriers, and leaves the wave's 128x64 block of C in `acc` with the LDS ring
// idle.  A and B point at the whole matrices; m0, n0 name the tile.  kEdge
// (version 10): the tile may reach past M rows, N columns or K (M any; N, K
// multiples of 8); what lies outside the matrices is loaded as zeros.
//
// kAbl (versions 71-77, whole tiles only): the kAbl* ingredients turned off.
template <bool kEdge = false, int kAbl = 0>
__device__ __forceinline__ void pp16_mainloop(const half_t* __restrict__ A, const half_t* __restrict__ B, int N,
                                              int K, int m0, int n0, int kb, int nk, uint32_t lds_base, int grp,
                                              int gw, int lane, float4v (&acc)[8][4], int M = 0,
                                              unsigned long long* t_first = nullptr) {
  static_assert(!(kEdge && kAbl), "the leave-one-out instances take whole tiles only");
  constexpr bool kSwzA = !(kAbl & kAblNoSwzA), kSwzB = !(kAbl & kAblNoSwzB);
  constexpr bool kDma = !(kAbl & kAblRegStage), kPP = !(kAbl & kAblNoPingPong);
  constexpr bool kB2 = kAbl & kAblB2, kChain = !(kAbl & kAblNoChain);
  constexpr int kNB = kB2 ? 2 : kBSlots;  // B slots
  auto sa = [](int row) { return kSwzA ? swz_a16(row) : 0; };
  auto sb = [](int krow) { return kSwzB ? swz_b16(krow) : 0; };
  // ---- direct-to-LDS duty: instruction d = 4h + i (8 per wave per k-tile) ----
  // Q, A: rows gw*32 + 8i .. +7 of the A-top (h = 0) or A-bot (h = 1) half,
  //   landing at half offset (gw*4 + i) * 1024.
  // P, B: k-rows gw*16 + 2*(i&1) + 8*(i>>1) + 4h, +1, landing at their own
  //   row offset (512 B per k-row).  h moves 4 k-rows (bit 2), which the B
  //   swizzle ignores, so voff[i] serves both h.
  uint32_t voff[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (grp) {
      const int row = gw * 32 + i * 8 + (lane >> 3);
      const int c = (lane & 7) ^ sa(row);
      voff[i] = (uint32_t)(((size_t)row * K + c * 8) * 2);
    } else {
      const int krow = gw * 16 + 2 * (i & 1) + 8 * (i >> 1) + (lane >> 5);
      const int c = (lane & 31) ^ sb(krow);
      voff[i] = (uint32_t)(((size_t)krow * N + c * 8) * 2);
    }
  }
  const char* a_top = reinterpret_cast<const char*>(A) + ((size_t)m0 * K + (size_t)kb * kBK) * 2;
  const char* b_src = reinterpret_cast<const char*>(B) + ((size_t)kb * kBK * N + n0) * 2;
  const char* g_base = grp ? a_top : b_src;
  const size_t g_kt = grp ? (size_t)kBK * 2 : (size_t)kBK * N * 2;   // per k-tile
  const size_t g_h = grp ? (size_t)128 * K * 2 : (size_t)4 * N * 2;  // per h
  const uint32_t l_base = lds_base + (grp ? (uint32_t)kATop + gw * 4 * 1024 : (uint32_t)kBOff + gw * 16 * 512);
  const uint32_t l_slot = grp ? (uint32_t)kHalfBytes : (uint32_t)kBBytes;  // per slot
  const uint32_t l_h = grp ? (uint32_t)(kABot - kATop) : 4u * 512u;       // per h

  // Edges: the same loads through a buffer resource over the whole matrix
  // (each operand below 2^31 bytes), the k-tile's offset from the matrix
  // start in the scalar offset and the lane's within the k-tile as before,
  // so a lane past the end of the matrix reads zeros: A rows at or below M,
  // B k-rows at or below K.  B columns past N (in range: the next row's) only
  // feed C columns that are not stored.  What remains is A's k past K on the
  // last k-tile (the next row's values, which must not meet B's zero rows:
  // an infinity there would make a NaN): such lanes get the matrix size as
  // their offset.  Bits 6i..6i+5 of akin: the first k of the lane's A chunk
  // of instruction i within a k-tile (a select, not a branch, inside the
  // MFMA sequence: a branch there made the fp32-output kernel spill).
  uint32_t akin = 0;
  if constexpr (kEdge) {
    if (grp) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = gw * 32 + i * 8 + (lane >> 3);
        akin |= (uint32_t)(((lane & 7) ^ sa(row)) * 8) << (6 * i);
      }
    }
  }
  const char* g_start = grp ? reinterpret_cast<const char*>(A) : reinterpret_cast<const char*>(B);
  const uint32_t g_size = kEdge ? (uint32_t)(grp ? M * K * 2 : K * N * 2) : 0u;
  const __amdgpu_buffer_rsrc_t g_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(g_start), 0, (int)g_size, kBufferWord3);
  const uint32_t g_off0 = (uint32_t)(g_base - g_start);  // the tile's first k-tile (kEdge: below 2^31)

  // LDS offset of load i within its (slot, h) region.
  uint32_t l_i[4];
#pragma unroll
  for (int i = 0; i < 4; i++) l_i[i] = grp ? (uint32_t)i * 1024 : (uint32_t)((i & 1) * 1024 + (i >> 1) * 4096);

  // Scalar operands of the 8 loads of one k-tile.  The loop computes them in
  // the memory phase, before the phase barrier, so that the compute phase
  // issues each load as three instructions (M0, its wait state and the load)
  // between two MFMAs: a wave issues at most one instruction every 4 cycles, so the ~10
  // scalar instructions of an address computation in front of a load leave
  // the matrix pipe idle for most of their length (measured: compute phases
  // of 1180 cycles for 1024 cycles of MFMA issue).
  struct DmaOps {
    const char* g[2];  // global base of half h (kEdge: unused)
    uint32_t soff[2];  // kEdge: the buffer's scalar offset of half h
    uint32_t kleft;    // kEdge: k from the k-tile's start to K (Q), 64 (P)
    uint32_t l[8];     // LDS destination of load d
  };
  auto dma_ops = [&](int kt, int slot) {
    DmaOps o;
    const uint32_t ls = l_base + slot * l_slot;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      if constexpr (kEdge)
        o.soff[h] = g_off0 + (uint32_t)kt * (uint32_t)g_kt + (uint32_t)h * (uint32_t)g_h;
      else
        o.g[h] = g_base + (size_t)kt * g_kt + h * g_h;
#pragma unroll
      for (int i = 0; i < 4; i++) o.l[4 * h + i] = ls + h * l_h + l_i[i];
    }
    // B's lanes are never masked here; A's k past K read zeros
    o.kleft = kEdge && grp ? (uint32_t)(K - (kb + kt) * kBK) : 64u;
    return o;
  };
  // Makes the compiler materialise the operands here (in scalar registers).
  auto pin_ops = [&](const DmaOps& o) {
    if constexpr (kEdge)
      asm volatile("" ::"s"(o.soff[0]), "s"(o.soff[1]), "s"(o.kleft));
    else
      asm volatile("" ::"s"(o.g[0]), "s"(o.g[1]));
    asm volatile("" ::"s"(o.l[0]), "s"(o.l[1]), "s"(o.l[2]), "s"(o.l[3]), "s"(o.l[4]), "s"(o.l[5]), "s"(o.l[6]),
                 "s"(o.l[7]));
  };
  auto dma_with = [&](int d, const DmaOps& o) {
    const int i = d & 3, h = d >> 2;
    if constexpr (kEdge) {
      const uint32_t off = ((akin >> (6 * i)) & 63u) < o.kleft ? voff[i] : g_size;  // g_size: zeros
      dma16_buf(g_rsrc, off, o.soff[h], o.l[d]);
    } else {
      dma16(o.g[h], voff[i], o.l[d]);
    }
  };
  auto dma = [&](int d, int kt, int slot) { dma_with(d, dma_ops(kt, slot)); };
  // kAblRegStage: the same 16 bytes per lane through a VGPR and a ds_write
  // to the address the direct-to-LDS load would have filled.
  const uint32_t lane16 = (uint32_t)lane * 16;
  auto gload = [&](int d, const DmaOps& o) -> uint4v {
    return *reinterpret_cast<const uint4v*>(o.g[d >> 2] + voff[d & 3]);
  };
  auto swrite = [&](int d, const DmaOps& o, const uint4v& v) {
    lds_write16(o.l[d] + lane16, __builtin_bit_cast(float4v, v));
  };
  // All 8 loads of one k-tile, written as they land (prologue).
  auto stage_tile = [&](int kt, int slot) {
    if constexpr (kDma) {
#pragma unroll
      for (int d = 0; d < 8; d++) dma(d, kt, slot);
    } else {
      const DmaOps o = dma_ops(kt, slot);
      uint4v v[8];
#pragma unroll
      for (int d = 0; d < 8; d++) v[d] = gload(d, o);
#pragma unroll
      for (int d = 0; d < 8; d++) swrite(d, o, v[d]);
    }
  };

  // ---- fragment addresses ----
  // A block i, k-step s: half-row i*16 + l%16, chunk 4s + l/16.
  const int arow = lane & 15;
  const uint32_t a_half = grp ? kABot : kATop;
  uint32_t aoff[2];
#pragma unroll
  for (int s2 = 0; s2 < 2; s2++)
    aoff[s2] = a_half + arow * (kBK * 2) + 16 * ((4 * s2 + (lane >> 4)) ^ sa(arow));
  // B block j, k-step s, half h: lane 16g + 4jj + q names k-row
  // 32s + 8g + 4h + jj, columns gw*64 + 16j + 4q .. +3; the transpose read
  // hands lane 16g + c the 4 k of column 16j + c.
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  const int krow0 = 8 * g + jj;  // plus 32s + 4h: bits 0, 1, 3 unchanged
  uint32_t boff[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int c = gw * 8 + 2 * j + (q >> 1);
    boff[j] = kBOff + krow0 * (kBN * 2) + 16 * (c ^ sb(krow0)) + 8 * (q & 1);
  }

#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  half8 fa[2][8], fb[2][4];
  // Accumulators stay in VGPRs (128 of them; 235-239 VGPRs in all, no
  // spills): at the power limit, v7 at 4096^3 ran 93.6 us per launch against
  // 94.8 with AGPR accumulators (interleaved A/B on one box, 3 pairs).

  // One per-lane base address per A k-step and per B block (6 VALU adds per
  // phase); the block, k-step and half offsets (< 64 KB) go into the reads'
  // immediate offset fields.
  auto read_frags = [&](int aslot, int bslot) {
    const uint32_t sa = lds_base + aslot * kHalfBytes;
    const uint32_t sb = lds_base + bslot * kBBytes;
    uint32_t va[2], vb[4];
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) va[s2] = sa + aoff[s2];
#pragma unroll
    for (int j = 0; j < 4; j++) vb[j] = sb + boff[j];
    static_for<2>([&](auto s2c) {
      constexpr int s2 = decltype(s2c)::value;
      static_for<8>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        fa[s2][i] = lds_read_h8_off<i * 16 * kBK * 2>(va[s2]);
      });
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const half4 lo = lds_read_tr16_off<s2 * 32 * kBN * 2>(vb[j]);
        const half4 hi = lds_read_tr16_off<s2 * 32 * kBN * 2 + 4 * kBN * 2>(vb[j]);
        fb[s2][j] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    });
  };
  // 64 MFMAs with the 8 loads described by `o` interleaved, one after every 8.
  // Each accumulator takes its two k-steps back to back (the second MFMA's
  // accumulator input is the first one's result): measured on MI355X with a
  // pure 16x16x32 stream at the power limit, such chains of 2 raise the
  // sustained clock by ~4% over rotating through the accumulators, at the
  // same issue rate.  The chains run along each row of blocks and back along
  // the next (j = 3 .. 0 on odd i), and accumulator (i, j) takes k-step
  // (i ^ j) & 1 first, so every chain starts on the operand register the one
  // before ended on (A fragment within a row, B at a row change): fewer
  // operand bits toggle, and at 4096^3, 8192^3 and 4096 x 4096 x 11008 the
  // board held its power limit 10-11 MHz higher for the same cycles per
  // launch (+0.5-0.7 %, 5 interleaved pairs on one box).  The scheduling
  // barriers keep the pairs adjacent.
  // Load d of the k-tile described by `o`: direct-to-LDS, or (kAblRegStage)
  // into stg[d], written to LDS four loads later (the compiler waits for
  // that load alone: vmcnt(3)), the last four after the MFMAs.
  uint4v stg[8];
  auto load_step = [&](int d, const DmaOps& o) {
    if constexpr (kDma) {
      dma_with(d, o);
    } else {
      if (d >= 4) swrite(d - 4, o, stg[d - 4]);
      stg[d] = gload(d, o);
    }
  };
  auto compute_and_load = [&](const DmaOps& o) {
    if constexpr (kChain) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const int j = (i & 1) ? 3 - jj : jj;
          const int k0 = (i ^ j) & 1;
          acc[i][j] = mfma16x16x32(fb[k0][j], fa[k0][i], acc[i][j]);
          __builtin_amdgcn_sched_barrier(0);
          acc[i][j] = mfma16x16x32(fb[k0 ^ 1][j], fa[k0 ^ 1][i], acc[i][j]);
          __builtin_amdgcn_sched_barrier(0);
        }
        load_step(i, o);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
        for (int i = 0; i < 8; i++) {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int k = s2 ^ ((i ^ j) & 1);  // the chained form's per-element order
            acc[i][j] = mfma16x16x32(fb[k][j], fa[k][i], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
          }
          if (i & 1) {
            load_step(4 * s2 + (i >> 1), o);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
    }
    if constexpr (!kDma) {
#pragma unroll
      for (int d = 4; d < 8; d++) swrite(d, o, stg[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Prologue and loop: exactly as version 6.  kAblB2: P keeps B one k-tile
  // ahead (B(t+1) in compute(t), waited for at its end); kAblNoPingPong: no
  // extra barrier for Q at the start or for P at the end, and every wave
  // waits for k-tile t+1 after compute(t).
  const int kt1 = min(1, nk - 1);
  stage_tile(0, 0);
  if (!kB2 || grp) stage_tile(kt1, 1);
  if (grp)
    wait_vmcnt<kPP ? 12 : 8>();
  else
    wait_vmcnt<kB2 ? 0 : 8>();
  lds_barrier();
  if (kPP && grp) {
    wait_vmcnt<8>();
    lds_barrier();
  }
  if constexpr (VK_TIMELINE != 0) *t_first = __builtin_amdgcn_s_memrealtime();

  for (int t = 0; t < nk; t++) {
    const int aslot = t & 1;
    const int bslot = t % kNB;
    const int kt2 = min(t + 2, nk - 1);
    const int ktp = kB2 && !grp ? min(t + 1, nk - 1) : kt2;  // this wave's loads
    __builtin_amdgcn_sched_barrier(0);
    read_frags(aslot, bslot);
    __builtin_amdgcn_sched_barrier(0);  // the reads go out first
    const DmaOps ops = dma_ops(ktp, grp ? aslot : (t + (kB2 ? 1 : 2)) % kNB);
    pin_ops(ops);
    if (kPP && grp) wait_vmcnt<4>();  // Q: A-top(t+1) landed before barrier 2t+2
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    compute_and_load(ops);
    if (kB2 && !grp)
      wait_vmcnt<0>();  // P: B(t+1)
    else
      wait_vmcnt<8>();  // P: B(t+1); Q: A-top(t+1), A-bot(t+1)
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  }
  __builtin_amdgcn_sched_barrier(0);
  if (kPP && !grp) lds_barrier();
  wait_vmcnt<0>();
  lds_barrier();
}

// Lane index recomputed from the exec mask, so that no register has to carry
// threadIdx.x across the k-loop.
__device__ __forceinline__ int lane_from_exec() {
  return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

template <typename OutT>
__global__ __launch_bounds__(kThreads) void f16_pp16_kernel(const half_t* __restrict__ A,
                                                            const half_t* __restrict__ B,
                                                            OutT* __restrict__ C, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;  // 0 = P, 1 = Q; waves w and w+4 share a SIMD
  const int gw = wave & 3;

  int tm, tn;
  tile_of(blockIdx.x, M / kBM, N / kBN, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  float4v acc[8][4];
#if VK_TIMELINE
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  unsigned long long t1 = 0;
  pp16_mainloop(A, B, N, K, m0, n0, 0, K / kBK, lds_base, grp, gw, lane, acc, 0, &t1);
  const unsigned long long t2 = __builtin_amdgcn_s_memrealtime();
  epilogue16<OutT>(acc, lds_base + wave * (128 * 64 * 2), C + (size_t)(m0 + grp * 128) * N + n0 + gw * 64, N,
                   lane_from_exec());
  const unsigned long long t3 = __builtin_amdgcn_s_memrealtime();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const unsigned long long t4 = __builtin_amdgcn_s_memrealtime();
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  if (lane_from_exec() == 0 && gw == 0 && blockIdx.x < kTimelineGroups) {
    unsigned long long* r = vk_timeline + (blockIdx.x * 2 + grp) * 8;
    r[0] = t0; r[1] = t1; r[2] = t2; r[3] = t3; r[4] = t4; r[5] = xcc & 15u; r[6] = tm; r[7] = tn;
  }
#else
  pp16_mainloop(A, B, N, K, m0, n0, 0, K / kBK, lds_base, grp, gw, lane, acc);
  epilogue16<OutT>(acc, lds_base + wave * (128 * 64 * 2), C + (size_t)(m0 + grp * 128) * N + n0 + gw * 64, N,
                   lane_from_exec());
#endif
}

template <typename OutT>
hipError_t launch_t(const GemmArgs& a) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp16_kernel<OutT>;
  hipError_t e = ensure_lds_attr(kfn, kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  const int tiles = (int)((a.m / kBM) * (a.n / kBN));
  hipLaunchKernelGGL(kfn, dim3(tiles), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B),
                     static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

hipError_t launch(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_t<half_t>(a) : launch_t<float>(a);
}

// Versions 71-77: version 7 with one ingredient off (kAbl, see kAblNoSwzA).
template <typename OutT, int kAbl>
__global__ __launch_bounds__(kThreads) void f16_pp16_abl_kernel(const half_t* __restrict__ A,
                                                                const half_t* __restrict__ B,
                                                                OutT* __restrict__ C, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;
  const int gw = wave & 3;

  int tm, tn;
  if constexpr ((kAbl & kAblNoXcd) != 0)
    raster_tile(blockIdx.x, M / kBM, N / kBN, tm, tn);
  else
    tile_of(blockIdx.x, M / kBM, N / kBN, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  float4v acc[8][4];
  pp16_mainloop<false, kAbl>(A, B, N, K, m0, n0, 0, K / kBK, lds_base, grp, gw, lane, acc);
  epilogue16<OutT>(acc, lds_base + wave * (128 * 64 * 2), C + (size_t)(m0 + grp * 128) * N + n0 + gw * 64, N,
                   lane_from_exec());
}

template <typename OutT, int kAbl>
hipError_t launch_abl_t(const GemmArgs& a) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp16_abl_kernel<OutT, kAbl>;
  hipError_t e = ensure_lds_attr(kfn, lds_bytes_of<kAbl>(), a.device, attr_done);
  if (e != hipSuccess) return e;
  const int tiles = (int)((a.m / kBM) * (a.n / kBN));
  hipLaunchKernelGGL(kfn, dim3(tiles), dim3(kThreads), lds_bytes_of<kAbl>(), a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B),
                     static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

template <int kAbl>
hipError_t launch_abl(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_abl_t<half_t, kAbl>(a) : launch_abl_t<float, kAbl>(a);
}

// ---------------------------------------------------------------------------
// Version 10: version 7 for shapes off its 256 x 256 x 64 grid -- any M, N and
// K multiples of 8 (16-byte rows).  Same tiles, schedule and kernel body; the
// tiles on the right and bottom edges and the last k-tile reach past the
// matrices: their loads go through buffer resources that return zeros past
// the end of a matrix, the A chunks past K are masked, and the C stores skip
// the chunks outside.  The reference's kernels would launch no blocks for
// such shapes (matmul_f16_v42_shfl2.cu:124, :520-527).
template <typename OutT>
__global__ __launch_bounds__(kThreads) void f16_pp16_edge_kernel(const half_t* __restrict__ A,
                                                                 const half_t* __restrict__ B,
                                                                 OutT* __restrict__ C, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;
  const int gw = wave & 3;

  int tm, tn;
  tile_of(blockIdx.x, (M + kBM - 1) / kBM, (N + kBN - 1) / kBN, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  float4v acc[8][4];
  pp16_mainloop<true>(A, B, N, K, m0, n0, 0, (K + kBK - 1) / kBK, lds_base, grp, gw, lane, acc, M);
  epilogue16_edge<OutT>(acc, lds_base + wave * (128 * 64 * 2), C, M, N, m0 + grp * 128, n0 + gw * 64,
                        lane_from_exec());
}

template <typename OutT>
hipError_t launch_edge_t(const GemmArgs& a) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp16_edge_kernel<OutT>;
  hipError_t e = ensure_lds_attr(kfn, kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  const int tiles = (int)(((a.m + kBM - 1) / kBM) * ((a.n + kBN - 1) / kBN));
  hipLaunchKernelGGL(kfn, dim3(tiles), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B),
                     static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

hipError_t launch_edge(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_edge_t<half_t>(a) : launch_edge_t<float>(a);
}

// Each operand below 2^31 bytes (buffer sizes), and version 7's 32-bit lane
// offsets (128 rows of A, 64 k-rows of B) and tile count.
bool edge_shape_ok(size_t m, size_t n, size_t k) {
  return m >= 1 && n >= 8 && k >= 8 && m * k * 2 < (1ull << 31) && k * n * 2 < (1ull << 31) &&
         pp64::shape_ok(((m + kBM - 1) / kBM) * kBM, ((n + kBN - 1) / kBN) * kBN, k);
}

// ---------------------------------------------------------------------------
// Version 9: version 7's tile loop with a split tail, for grids whose last
// wave of 256x256 tiles would leave compute units idle (the reference's
// answer to the same problem is stream-K, results/naive_fable_cycle2/src/
// matmul_f16/matmul_f16_v9_streamk.cu:383-448, and the tail lesson of
// matmul_f16_v42_shfl2.cu:182-189).  The schedule (vk_splittail.hpp): whole
// tiles first, in version 7's order, then each tail tile cut into s aligned
// k-slices computed by s workgroups at once.  The pieces of a split tile are
// summed by whichever of them finishes last:
//  * each wave handles its own 128x64 block of the tile on its own, with one
//    arrival counter per (tile, wave), so the hand-off needs no workgroup
//    barrier;
//  * a finishing wave first reads the counter: if every other piece has
//    already arrived it is the last and skips writing its partial; otherwise
//    it writes its fp32 partial (stores that do not stay dirty in the XCD's
//    L2), waits for them to complete, and increments the counter; the one that
//    sees count == pieces - 1 is the last;
//  * the last one sums the pieces in k order, P0 + P1 + ..., its own piece
//    taken from registers, so the result does not depend on arrival order,
//    stores C and resets the counter to 0 for the next call.
// When the schedule splits nothing every tile runs whole, as version 7.
constexpr size_t kSkSlotBytes = (size_t)kBM * kBN * sizeof(float);  // one tile's fp32 partial

size_t sk_workspace(size_t m, size_t n, size_t k, int num_cus) {
  const SkPlan p = sk_plan((int64_t)((m / kBM) * (n / kBN)), (int64_t)(k / kBK), num_cus);
  return p.units ? kSkCounterBytes + (size_t)p.units * kSkSlotBytes : 0;
}

// Partial slots are read and written with store_partial / load_partial (sc1
// buffer accesses).

// Hand-off of one wave's block of a tile split into np pieces; this wave holds
// piece p.  part_off(q) is the byte offset of the wave's region of piece q's
// partial slot: 32 blocks (i, j) x 64 lanes x 16 bytes, so every access is a
// 1 KB coalesced row.  Returns whether this wave is the last to arrive.
template <typename PartOff>
__device__ __forceinline__ bool sk_arrive(float4v (&acc)[8][4], int np, int p, __amdgpu_buffer_rsrc_t part,
                                          PartOff part_off, unsigned* cnt) {
  const int lane = lane_from_exec();
  const unsigned seen =
      __builtin_amdgcn_readfirstlane(__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  if (seen == (unsigned)(np - 1)) return true;  // every other piece is in memory
  const uint32_t soff = part_off(p);
#pragma unroll
  for (int b = 0; b < 32; b++) store_partial(part, (uint32_t)lane * 16 + b * 1024, soff, acc[b >> 2][b & 3]);
  wait_vmcnt0_ordered();  // the partial is in memory before the counter moves
  unsigned old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_amdgcn_readfirstlane(old) == (unsigned)(np - 1);
}

// Store of the wave's block of C: acc alone for a whole tile (np = 1); for a
// split tile, the last arrival's sum of all pieces, after which the counter is
// reset for the next call.  The block starts at row row0, column col0 of C;
// kEdge: it may reach past M rows or N columns, which are not stored.
template <typename OutT, bool kEdge, typename PartOff>
__device__ __forceinline__ void sk_write_c(float4v (&acc)[8][4], int np, int p, __amdgpu_buffer_rsrc_t part,
                                           PartOff part_off, unsigned* cnt, uint32_t wstage, OutT* C, int M,
                                           int N, int row0, int col0) {
  const int lane = lane_from_exec();
  const uint32_t vlane = (uint32_t)lane * 16;
  // The counter read that made this wave the last stays before the reads of
  // the other pieces' partials.
  asm volatile("" ::: "memory");
  // C = P0 + P1 + ... + P(np-1), left to right, with P(p) = acc, summed 8
  // blocks at a time (the 8 loads of a piece issued together) and staged for
  // the store as each batch completes.
#pragma unroll
  for (int half = 0; half < 2; half++) {
#pragma unroll
    for (int bb = 2 * half; bb < 2 * half + 2; bb++) {
      float4v t[8], x[8];
      for (int q = 0; q < p; q++) {
        const uint32_t soff = part_off(q);
#pragma unroll
        for (int b = 0; b < 8; b++) x[b] = load_partial(part, vlane + (8 * bb + b) * 1024, soff);
#pragma unroll
        for (int b = 0; b < 8; b++) t[b] = q == 0 ? x[b] : t[b] + x[b];
      }
#pragma unroll
      for (int b = 0; b < 8; b++) t[b] = p == 0 ? acc[2 * bb + (b >> 2)][b & 3] : t[b] + acc[2 * bb + (b >> 2)][b & 3];
      for (int q = p + 1; q < np; q++) {
        const uint32_t soff = part_off(q);
#pragma unroll
        for (int b = 0; b < 8; b++) x[b] = load_partial(part, vlane + (8 * bb + b) * 1024, soff);
#pragma unroll
        for (int b = 0; b < 8; b++) t[b] += x[b];
      }
#pragma unroll
      for (int b = 0; b < 8; b++) Epi16<OutT>::stage(wstage, lane, 2 * bb + (b >> 2), b & 3, t[b]);
    }
    if constexpr (kEdge)
      Epi16<OutT>::flush_edge(wstage, C, M, N, row0, col0, lane, half);
    else
      Epi16<OutT>::flush(wstage, C + (size_t)row0 * N + col0, N, lane, half);
  }
  if (np > 1 && lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename OutT, bool kEdge>
__global__ __launch_bounds__(kThreads) void f16_pp16_sk_kernel(const half_t* __restrict__ A,
                                                               const half_t* __restrict__ B,
                                                               OutT* __restrict__ C, int M, int N, int K, int dp,
                                                               int units, int pieces, int chunks,
                                                               float* __restrict__ part,
                                                               unsigned* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;
  const int gw = wave & 3;
  // kEdge (version 10's split tails): the tiles and k-tiles that reach past
  // M, N or K count as whole ones, as in f16_pp16_edge_kernel.
  const int tiles_m = (M + (kEdge ? kBM - 1 : 0)) / kBM, tiles_n = (N + (kEdge ? kBN - 1 : 0)) / kBN;
  const int T = tiles_m * tiles_n;
  const int I = (K + (kEdge ? kBK - 1 : 0)) / kBK;
  const uint32_t lds_base = lds_addr32(lds);
  const uint32_t wstage = lds_base + wave * (128 * 64 * 2);
  const int bid = blockIdx.x;

  const SkPlan plan{dp, units, pieces, chunks};
  const SkWork w = sk_work(bid, T, I, plan);
  int tm, tn;
  raster_tile(w.cid, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  float4v acc[8][4];
  pp16_mainloop<kEdge>(A, B, N, K, m0, n0, w.kb, w.ke - w.kb, lds_base, grp, gw, lane, acc, M);
  // One partial slot per split-tail unit (at most 256: 64 MB, within 32-bit
  // offsets); piece q of this tile is in the slot of unit sk_unit_of(.., q).
  const __amdgpu_buffer_rsrc_t prsrc =
      __builtin_amdgcn_make_buffer_rsrc(part, 0, (int)(units * kSkSlotBytes), kBufferWord3);
  auto part_off = [&](int q) {
    return (uint32_t)(sk_unit_of(plan, T, w.tile, q) * kSkSlotBytes) + (uint32_t)wave * (128 * 64 * 4);
  };
  unsigned* cnt = counters + (size_t)w.tile * kSkWaves + wave;
  if (w.np == 1 || sk_arrive(acc, w.np, w.p, prsrc, part_off, cnt))
    sk_write_c<OutT, kEdge>(acc, w.np, w.p, prsrc, part_off, cnt, wstage, C, M, N, m0 + grp * 128, n0 + gw * 64);
}

// Split-tail plan of a shape: kEdge counts the tiles and k-tiles that reach
// past M, N or K.
template <bool kEdge>
SkPlan sk_plan_of(size_t m, size_t n, size_t k, int num_cus) {
  const size_t tm = kEdge ? (m + kBM - 1) / kBM : m / kBM, tn = kEdge ? (n + kBN - 1) / kBN : n / kBN;
  return sk_plan((int64_t)(tm * tn), (int64_t)(kEdge ? (k + kBK - 1) / kBK : k / kBK), num_cus);
}

template <typename OutT, bool kEdge>
hipError_t launch_sk_t(const GemmArgs& a) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp16_sk_kernel<OutT, kEdge>;
  hipError_t e = ensure_lds_attr(kfn, kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  const SkPlan p = sk_plan_of<kEdge>(a.m, a.n, a.k, a.num_cus);
  unsigned* counters = nullptr;
  float* part = nullptr;
  if (p.units > 0) {
    counters = static_cast<unsigned*>(a.workspace);
    part = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + kSkCounterBytes);
    if (!a.workspace_clean) {
      e = zero_words(counters, kSkCounterBytes / sizeof(unsigned), a.stream);
      if (e != hipSuccess) return e;
    }
  }
  hipLaunchKernelGGL(kfn, dim3((unsigned)(p.dp + p.units)), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B), static_cast<OutT*>(a.C),
                     (int)a.m, (int)a.n, (int)a.k, p.dp, p.units, p.pieces, p.chunks, part, counters);
  return hipGetLastError();
}

hipError_t launch_sk(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_sk_t<half_t, false>(a) : launch_sk_t<float, false>(a);
}

// Version 10: whole tiles with masked edges, or, where the split-tail plan
// splits (a part-empty last wave, e.g. 1000^3 = 16 tiles), version 9's
// schedule with the same edges.
hipError_t launch_edge_any(const GemmArgs& a) {
  if (sk_plan_of<true>(a.m, a.n, a.k, a.num_cus).units == 0) return launch_edge(a);
  return a.out_dtype == VK_DTYPE_F16 ? launch_sk_t<half_t, true>(a) : launch_sk_t<float, true>(a);
}

size_t sk_workspace_edge(size_t m, size_t n, size_t k, int num_cus) {
  const SkPlan p = sk_plan_of<true>(m, n, k, num_cus);
  return p.units ? kSkCounterBytes + (size_t)p.units * kSkSlotBytes : 0;
}

}  // namespace pp16
}  // namespace

void register_f16_pingpong() {
  KernelEntry e{};
  e.version = 5;
  e.in_dtype = VK_DTYPE_F16;
  e.name = "f16_v5_pp256_bk32x4";
  e.caps = make_caps(5, VK_DTYPE_F16, kOutF16 | kOutF32, kBM, kBN, kBK, 16, kBM, kBN, kBK, kThreads,
                     kLdsBytes, 0, 0);
  e.launch = launch_pp;
  e.workspace = nullptr;
  e.shape_ok = pp_shape_ok;
  register_kernel(e);

  KernelEntry e6{};
  e6.version = 6;
  e6.in_dtype = VK_DTYPE_F16;
  e6.name = "f16_v6_pp256_bk64_split";
  e6.caps = make_caps(6, VK_DTYPE_F16, kOutF16 | kOutF32, kBM, kBN, pp64::kBK, 16, kBM, kBN, pp64::kBK,
                      kThreads, pp64::kLdsBytes, 0, 0);
  e6.launch = pp64::launch;
  e6.workspace = nullptr;
  e6.shape_ok = pp64::shape_ok;
  register_kernel(e6);

  KernelEntry e7 = e6;
  e7.version = 7;
  e7.name = "f16_v7_pp256_bk64_m16";
  e7.caps.version = 7;
  e7.launch = pp16::launch;
  register_kernel(e7);

  // Leave-one-out instances of version 7 (never picked; bench.py --version N).
  struct Abl {
    int version;
    const char* name;
    LaunchFn launch;
    int lds;
  };
  const Abl abl[] = {
      {71, "f16_v71_v7_no_swizzle_a", pp16::launch_abl<pp16::kAblNoSwzA>, pp64::kLdsBytes},
      {72, "f16_v72_v7_no_swizzle_b", pp16::launch_abl<pp16::kAblNoSwzB>, pp64::kLdsBytes},
      {73, "f16_v73_v7_vgpr_staging", pp16::launch_abl<pp16::kAblRegStage>, pp64::kLdsBytes},
      {74, "f16_v74_v7_b_ring2", pp16::launch_abl<pp16::kAblB2>, pp16::lds_bytes_of<pp16::kAblB2>()},
      {75, "f16_v75_v7_no_pingpong", pp16::launch_abl<pp16::kAblNoPingPong>, pp64::kLdsBytes},
      {76, "f16_v76_v7_no_xcd_order", pp16::launch_abl<pp16::kAblNoXcd>, pp64::kLdsBytes},
      {77, "f16_v77_v7_no_mfma_chain", pp16::launch_abl<pp16::kAblNoChain>, pp64::kLdsBytes},
  };
  for (const Abl& x : abl) {
    KernelEntry ea = e7;
    ea.version = x.version;
    ea.name = x.name;
    ea.caps.version = x.version;
    ea.caps.lds_bytes = x.lds;
    ea.launch = x.launch;
    register_kernel(ea);
  }

  KernelEntry e10 = e7;
  e10.version = 10;
  e10.name = "f16_v10_pp256_edge";
  e10.caps = make_caps(10, VK_DTYPE_F16, kOutF16 | kOutF32, 1, 8, 8, 16, kBM, kBN, pp64::kBK, kThreads,
                       pp64::kLdsBytes, 0, 0);
  e10.caps.uses_workspace = 1;
  e10.launch = pp16::launch_edge_any;
  e10.workspace = pp16::sk_workspace_edge;
  e10.shape_ok = pp16::edge_shape_ok;
  register_kernel(e10);

  KernelEntry e9 = e7;
  e9.version = 9;
  e9.name = "f16_v9_pp256_splittail";
  e9.caps.version = 9;
  e9.caps.uses_workspace = 1;
  e9.launch = pp16::launch_sk;
  e9.workspace = pp16::sk_workspace;
  register_kernel(e9);
}

}  // namespace vk
