// f16_pp128.hip -- fp16 GEMM, version 11: version 7's ping-pong on 128x128
// tiles with 128-deep k-tiles, for grids that 256x256 tiles leave part empty.
//
// At 4096^3 a 256x256 tile per CU is the cheapest way to feed the matrix
// cores (f16_pingpong.hip).  A GEMM with few such tiles -- 1024 x 4096 x
// 4096 has 64 on 256 CUs -- must otherwise split K (version 9), and each
// split tile's pieces meet through fp32 partials that cost as much as the
// k-loop (measured: ~24 us of k-loop, 47.6 us per launch).  Here four times
// as many tiles fill the CUs instead, and no partial leaves a CU.  The price
// is twice the L2->LDS and LDS-read bytes per FLOP of the 256x256 tile.
//
// Same design as version 7 scaled down, with 128-deep k-tiles so that a
// phase still holds 512 matrix-core cycles:
//  * 512 threads = 8 waves: P = waves 0..3 own tile rows 0..63, Q = waves
//    4..7 rows 64..127; wave g of a group owns columns 32g..32g+31, a 64x32
//    block = 4x2 MFMA blocks of 16x16 (32 fp32 accumulators per lane);
//  * per k-tile each group runs a memory phase (this wave's 16 A-fragment
//    reads and 16 transposed B reads of the k-tile) and a compute phase (32
//    v_mfma_f32_16x16x32_f16, each accumulator's 4 k-steps back to back, and
//    this wave's 8 direct-to-LDS loads of k-tile t+2, one after each
//    accumulator's chain); Q runs one phase behind P;
//  * LDS ring (160 KB), the slot sizes of version 7's:
//      A-top  rows  0..63 of the A k-tile (64 x 128 k), read by P  2 x 16 KB
//      A-bot  rows 64..127,                               read by Q  2 x 16 KB
//      B      128 k x 128 columns,                        read by both 3 x 32 KB
//    Q loads A-top(t+2) and A-bot(t+2) into slot t % 2, P loads B(t+2) into
//    slot (t+2) % 3, with version 7's waits (vmcnt 4 and 8);
//  * A rows are 256 B = 16 chunks of 16 B, chunk ^ (row % 16): the 16 rows of
//    a fragment read sit in 16 distinct chunks; B k-rows are 256 B too,
//    chunk ^ 2 (k % 4) ^ 8 bit3(k) (the skinny kernel's transpose-read
//    swizzle for 16-chunk rows);
//  * the epilogue stages each wave's 64x32 block of C through LDS (8-byte
//    units XOR 2 ((row / 4) % 4) for fp16, 16-byte chunks XOR (row / 2) % 8
//    for fp32) and stores 16-byte pieces of full row segments.
// Shapes: any M, N and K multiples of 8.  Off the 128 x 128 x 128 grid the
// edge tiles and the last k-tile reach past the matrices (kEdge, version
// 10's treatment): the loads go through buffer resources over the whole
// matrices, which return zeros past a matrix's end (A rows at or below M, B
// k-rows at or below K); A's k past K on the last k-tile (the next row's
// values, which must not meet B's zero rows: an infinity would make a NaN)
// is masked by a select; B columns past N only feed C columns that are not
// stored; the C stores are bounds-checked.
// Where the tiles fill at most half of the CUs, K is split over the idle
// ones (kSplit, below), the pieces meeting through fp32 partials.
#include "vk_device.hpp"
#include "vk_internal.hpp"
#include "vk_splittail.hpp"
#include "vk_tile.hpp"

#include <atomic>

namespace vk {
namespace {
namespace pp128 {

constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kThreads = 512;
constexpr int kRowBytes = kBK * 2;                // 256: an A row of a k-tile
constexpr int kHalfBytes = 64 * kRowBytes;        // 16 KB: one A half-tile
constexpr int kBRowBytes = kBN * 2;               // 256: a B k-row of a tile
constexpr int kBBytes = kBK * kBRowBytes;         // 32 KB
constexpr int kATop = 0;                          // 2 slots
constexpr int kABot = 2 * kHalfBytes;             // 2 slots
constexpr int kBOff = 4 * kHalfBytes;             // 3 slots
constexpr int kBSlots = 3;
constexpr int kLdsBytes = kBOff + kBSlots * kBBytes;  // 160 KB
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(kLdsBytes >= 8 * 64 * 32 * 4, "fp32 epilogue staging: 8 KB per wave");

__host__ __device__ constexpr int swz_a(int row) { return row & 15; }
__host__ __device__ constexpr int swz_b(int krow) { return (2 * (krow & 3)) ^ (((krow >> 3) & 1) << 3); }

// Store of a wave's 64x32 block of C.  Block (i, j), register r, lane l
// holds C[16 i + l % 16][16 j + 4 (l / 16) + r].
template <typename OutT>
struct Epi;

// fp16: rows of 64 B = 8 units of 8 B (4 halves); unit u of row r at
// u ^ (r / 2) % 8.  gfx950 serves a ds_write_b64 in passes of 16 lanes over
// banks that repeat every 128 bytes (measured: two lanes of a pass whose
// addresses differ by a multiple of 128 B take two cycles).  A pass names 16
// consecutive rows of one unit column, two rows per 128 bytes: the XOR puts
// the 8 rows of each parity on 8 distinct units, one cycle per pass.  A read
// takes units 2c, 2c+1 (16 B) from the slot c ^ (r / 4) % 4, its two 8-byte
// halves swapped when (r / 2) is odd.
template <>
struct Epi<half_t> {
  static constexpr int kRegion = 64 * 64;
  static __device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }
  static __device__ __forceinline__ uint4v read_pair(uint32_t wbase, int row, int ch) {
    const uint4v v = lds_read16(wbase + row * 64 + 16 * (ch ^ (swz(row) >> 1)));
    const bool odd = swz(row) & 1;
    return uint4v{odd ? v[2] : v[0], odd ? v[3] : v[1], odd ? v[0] : v[2], odd ? v[1] : v[3]};
  }
  static __device__ __forceinline__ void stage(uint32_t wbase, int lane, int i, int j, const float4v& v) {
    const int row = 16 * i + (lane & 15), unit = 4 * j + (lane >> 4);
    half4 h = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
    lds_write8(wbase + row * 64 + 8 * (unit ^ swz(row)), h);
  }
  static __device__ __forceinline__ void store(uint32_t wbase, half_t* Cw, int N, int lane) {
    const int rsub = lane >> 2, ch = lane & 3;
    const __amdgpu_buffer_rsrc_t cr = out_rsrc(Cw);  // 64 rows, N < 2^23: offsets below 2^31
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int row = 16 * q + rsub;
      const uint4v v = read_pair(wbase, row, ch);
      store_out16(cr, (uint32_t)(row * N + ch * 8) * 2u, v);
    }
  }
  // The block at (row0, col0) of C may reach past M rows or N columns (N a
  // multiple of 8): chunks outside are not stored.
  static __device__ __forceinline__ void store_edge(uint32_t wbase, half_t* C, int M, int N, int row0, int col0,
                                                    int lane) {
    const int rsub = lane >> 2, ch = lane & 3;
    const bool col_in = col0 + ch * 8 < N;
    // Plain stores here: measured at 1000^3, the sc1 stores of the whole
    // tiles made this edge path slower (10.13 against 9.71 us per launch).
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int row = 16 * q + rsub;
      const uint4v v = read_pair(wbase, row, ch);
      if (col_in && row0 + row < M) *reinterpret_cast<uint4v*>(C + (size_t)(row0 + row) * N + col0 + ch * 8) = v;
    }
  }
};

// fp32: rows of 128 B = 8 chunks of 16 B (4 floats); chunk u of row r at
// u ^ r % 8.  A ds_write_b128 pass (8 lanes: 8 consecutive rows of one chunk
// column) then covers the 8 chunk positions of the 128-byte bank period, and
// a read (8 rows x 8 chunks) the 16 slots of each of its passes.
template <>
struct Epi<float> {
  static constexpr int kRegion = 64 * 128;
  static __device__ __forceinline__ void stage(uint32_t wbase, int lane, int i, int j, const float4v& v) {
    const int row = 16 * i + (lane & 15), chunk = 4 * j + (lane >> 4);
    lds_write16(wbase + row * 128 + 16 * (chunk ^ (row & 7)), v);
  }
  static __device__ __forceinline__ void store(uint32_t wbase, float* Cw, int N, int lane) {
    const int rsub = lane >> 3, ch = lane & 7;
    const __amdgpu_buffer_rsrc_t cr = out_rsrc(Cw);
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const int row = 8 * q + rsub;
      const uint4v v = lds_read16(wbase + row * 128 + 16 * (ch ^ (row & 7)));
      store_out16(cr, (uint32_t)(row * N + ch * 4) * 4u, v);
    }
  }
  static __device__ __forceinline__ void store_edge(uint32_t wbase, float* C, int M, int N, int row0, int col0,
                                                    int lane) {
    const int rsub = lane >> 3, ch = lane & 7;
    const bool col_in = col0 + ch * 4 < N;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const int row = 8 * q + rsub;
      const uint4v v = lds_read16(wbase + row * 128 + 16 * (ch ^ (row & 7)));
      if (col_in && row0 + row < M) *reinterpret_cast<uint4v*>(C + (size_t)(row0 + row) * N + col0 + ch * 4) = v;
    }
  }
};

// ---- split K for grids whose tiles fill at most half of the CUs ----
// With T tiles of I k-tiles on C CUs and 2T <= C, each tile is cut into
// s = min(8, C / T, I / 8) aligned k-slices (at least kFillMinIters = 8
// k-tiles each)
// computed by s workgroups at once (sk_plan_fill in vk_splittail.hpp: no
// whole tiles; the pieces of an XCD's share of the raster stay on it), and
// the pieces of a tile meet as in version 9: per (tile, wave) an arrival
// counter; a finishing wave that finds every other piece in memory is the
// last and writes nothing, otherwise it writes its 8 KB fp32 partial with
// sc1 stores, waits for them and increments the counter, and the one that
// sees s - 1 is the last.  The last sums P0 + P1 + ... in k order (its own
// piece from registers), so C does not depend on the arrival order, stores
// C and resets the counter.  The last piece is one k-tile longer than the
// others, so it usually arrives last and skips its store.
constexpr size_t kSlotBytes = (size_t)kBM * kBN * sizeof(float);  // one tile's fp32 partial
constexpr uint32_t kWaveSlotBytes = 64 * 32 * 4;                   // a wave's 64x32 block

// This wave holds piece p of np of its block.  part_off(q): byte offset of
// the wave's region of piece q's slot (8 blocks x 64 lanes x 16 bytes, each
// access a coalesced 1 KB row).  Returns whether this wave arrived last.
// Only the last piece, which usually arrives last, reads the counter first;
// the others publish their partial at once.
template <typename PartOff>
__device__ __forceinline__ bool split_arrive(const float4v (&acc)[4][2], int np, int p, int lane,
                                             __amdgpu_buffer_rsrc_t part, PartOff part_off, unsigned* cnt) {
  if (p == np - 1) {
    const unsigned seen =
        __builtin_amdgcn_readfirstlane(__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if (seen == (unsigned)(np - 1)) return true;  // every other piece is in memory
  }
  const uint32_t soff = part_off(p);
#pragma unroll
  for (int b = 0; b < 8; b++) store_partial(part, (uint32_t)lane * 16 + b * 1024, soff, acc[b >> 1][b & 1]);
  wait_vmcnt0_ordered();  // the partial is in memory before the counter moves
  unsigned old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_amdgcn_readfirstlane(old) == (unsigned)(np - 1);
}

// The last arrival: acc <- P0 + P1 + ... + P(NP-1), left to right, P(p) =
// acc.  The partials' loads go out together, kB blocks of every piece at a
// time (at most 32 loads in flight: 128 registers), so the wait is one
// memory round trip per batch (measured ~1.2 us each); the own piece's slot
// is loaded too and not used (no branch; the slot is always inside the
// workspace).
template <int NP, typename PartOff>
__device__ __forceinline__ void split_sum_n(float4v (&acc)[4][2], int p, int lane, __amdgpu_buffer_rsrc_t part,
                                            PartOff part_off) {
  constexpr int kB = NP <= 4 ? 8 : 4;  // blocks per batch
#pragma unroll
  for (int b0 = 0; b0 < 8; b0 += kB) {
    float4v x[NP][kB];
#pragma unroll
    for (int q = 0; q < NP; q++) {
      const uint32_t soff = part_off(q);
#pragma unroll
      for (int b = 0; b < kB; b++) x[q][b] = load_partial(part, (uint32_t)lane * 16 + (b0 + b) * 1024, soff);
    }
#pragma unroll
    for (int b = 0; b < kB; b++) {
      const uint4v own = __builtin_bit_cast(uint4v, acc[(b0 + b) >> 1][(b0 + b) & 1]);
      float4v t;
#pragma unroll
      for (int q = 0; q < NP; q++) {
        // Piece q's term: the own registers where q == p, chosen by a bit
        // mask (kept opaque, so no branch replaces it).
        uint32_t own_mask = q == p ? ~0u : 0u;
        asm volatile("" : "+v"(own_mask));
        const float4v term =
            __builtin_bit_cast(float4v, (__builtin_bit_cast(uint4v, x[q][b]) & ~own_mask) | (own & own_mask));
        t = q == 0 ? term : t + term;
      }
      acc[(b0 + b) >> 1][(b0 + b) & 1] = t;
    }
  }
}

template <typename PartOff>
__device__ __forceinline__ void split_sum(float4v (&acc)[4][2], int np, int p, int lane,
                                          __amdgpu_buffer_rsrc_t part, PartOff part_off) {
  // The counter read that made this wave the last stays before these reads.
  asm volatile("" ::: "memory");
  static_assert(kFillMaxPieces == 8, "one case per piece count");
  switch (np) {
    case 2: split_sum_n<2>(acc, p, lane, part, part_off); break;
    case 3: split_sum_n<3>(acc, p, lane, part, part_off); break;
    case 4: split_sum_n<4>(acc, p, lane, part, part_off); break;
    case 5: split_sum_n<5>(acc, p, lane, part, part_off); break;
    case 6: split_sum_n<6>(acc, p, lane, part, part_off); break;
    case 7: split_sum_n<7>(acc, p, lane, part, part_off); break;
    default: split_sum_n<8>(acc, p, lane, part, part_off); break;
  }
}

// kSplit: this workgroup is unit blockIdx.x of the split plan {0, units,
// pieces, chunks}; part and counters are the workspace.
template <typename OutT, bool kEdge, bool kSplit>
__global__ __launch_bounds__(kThreads) void f16_pp128_kernel(const half_t* __restrict__ A,
                                                             const half_t* __restrict__ B,
                                                             OutT* __restrict__ C, int M, int N, int K, int units,
                                                             int pieces, int chunks, float* __restrict__ part,
                                                             unsigned* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;  // 0 = P, 1 = Q; waves w and w+4 share a SIMD
  const int gw = wave & 3;
  constexpr int kR = kEdge ? 1 : 0;  // round the tile and k-tile counts up
  const int tiles_m = (M + kR * (kBM - 1)) / kBM, tiles_n = (N + kR * (kBN - 1)) / kBN;
  const int iters = (K + kR * (kBK - 1)) / kBK;
  int tm, tn, kb = 0, nk = iters;
  SkWork w{};
  if constexpr (kSplit) {
    w = sk_work(blockIdx.x, tiles_m * tiles_n, iters, SkPlan{0, units, pieces, chunks}, kFillLastExtra);
    raster_tile(w.cid, tiles_m, tiles_n, tm, tn);
    kb = w.kb;
    nk = w.ke - w.kb;
  } else {
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  }
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  // ---- direct-to-LDS duty: instruction d = 4h + i (8 per wave per k-tile) ----
  // Q, A: rows gw*16 + 4i + l/16 of the A-top (h = 0) or A-bot (h = 1) half
  //   (4 rows of 256 B per 1 KB instruction; lane l lands at chunk position
  //   l % 16, which holds chunk (l % 16) ^ swz_a(row)), at half offset
  //   (gw*16 + 4i) * 256.
  // P, B: k-rows gw*32 + 16h + 4i + l/16, landing at their own row offset;
  //   h moves 16 k-rows (bit 4), which the B swizzle ignores, so voff[i]
  //   serves both h.
  uint32_t voff[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (grp) {
      const int row = gw * 16 + 4 * i + (lane >> 4);
      const int c = (lane & 15) ^ swz_a(row);
      voff[i] = (uint32_t)(((size_t)row * K + c * 8) * 2);
    } else {
      const int krow = gw * 32 + 4 * i + (lane >> 4);
      const int c = (lane & 15) ^ swz_b(krow);
      voff[i] = (uint32_t)(((size_t)krow * N + c * 8) * 2);
    }
  }
  const size_t g_kt = grp ? (size_t)kBK * 2 : (size_t)kBK * N * 2;  // per k-tile
  const char* g_base = (grp ? reinterpret_cast<const char*>(A) + (size_t)m0 * K * 2
                            : reinterpret_cast<const char*>(B) + (size_t)n0 * 2) +
                       (size_t)kb * g_kt;  // k-tile kb: local k-tile 0
  const size_t g_h = grp ? (size_t)64 * K * 2 : (size_t)16 * N * 2;  // per h
  const uint32_t l_base = lds_base + (grp ? (uint32_t)kATop + gw * 16 * kRowBytes : (uint32_t)kBOff + gw * 32 * kBRowBytes);
  const uint32_t l_slot = grp ? (uint32_t)kHalfBytes : (uint32_t)kBBytes;  // per slot
  const uint32_t l_h = grp ? (uint32_t)(kABot - kATop) : 16u * kBRowBytes;  // per h

  // Edges: the same loads through a buffer resource over the whole matrix
  // (below 2^31 bytes), the k-tile's offset in the scalar offset and the
  // lane's within the k-tile in the VGPR, so a lane past the end of the
  // matrix reads zeros.  Byte 8i of akin (Q): the first k of the lane's A
  // chunk in instruction i within a k-tile; a chunk at or past K gets the
  // matrix size as its offset (zeros).
  uint32_t akin = 0;
  if constexpr (kEdge) {
    if (grp) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = gw * 16 + 4 * i + (lane >> 4);
        akin |= (uint32_t)(((lane & 15) ^ swz_a(row)) * 8) << (8 * i);
      }
    }
  }
  const char* g_start = grp ? reinterpret_cast<const char*>(A) : reinterpret_cast<const char*>(B);
  const uint32_t g_size = kEdge ? (uint32_t)(grp ? (size_t)M * K * 2 : (size_t)K * N * 2) : 0u;
  const __amdgpu_buffer_rsrc_t g_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(g_start), 0, (int)g_size, kBufferWord3);
  const uint32_t g_off0 = (uint32_t)(g_base - g_start);  // kEdge: below 2^31

  // Scalar operands of the 8 loads of one k-tile, computed in the memory
  // phase so that the compute phase issues each load as M0, its wait state
  // and the load between two MFMAs.
  struct DmaOps {
    const char* g[2];  // global base of half h (kEdge: unused)
    uint32_t soff[2];  // kEdge: the buffer's scalar offset of half h
    uint32_t kleft;    // kEdge: k from the k-tile's start to K (Q), 128 (P)
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
      for (int i = 0; i < 4; i++) o.l[4 * h + i] = ls + h * l_h + i * 1024;
    }
    o.kleft = kEdge && grp ? (uint32_t)(K - (kb + kt) * kBK) : (uint32_t)kBK;
    return o;
  };
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
      const uint32_t off = ((akin >> (8 * i)) & 255u) < o.kleft ? voff[i] : g_size;  // g_size: zeros
      dma16_buf(g_rsrc, off, o.soff[h], o.l[d]);
    } else {
      dma16(o.g[h], voff[i], o.l[d]);
    }
  };
  auto dma = [&](int d, int kt, int slot) { dma_with(d, dma_ops(kt, slot)); };

  // ---- fragment addresses ----
  // A block i, k-step s: half-row 16i + l%16, chunk 4s + l/16 (the row's
  // swizzle is that of l%16 for every i).
  const int arow = lane & 15;
  const uint32_t a_half = grp ? kABot : kATop;
  uint32_t aoff[4];
#pragma unroll
  for (int s = 0; s < 4; s++) aoff[s] = a_half + arow * kRowBytes + 16 * ((4 * s + (lane >> 4)) ^ swz_a(arow));
  // B block j, k-step s, half h: lane 16g + 4jj + q names k-row
  // 32s + 8g + 4h + jj, columns 32 gw + 16j + 4q .. +3; the transpose read
  // hands lane 16g + c the 4 k of column 16j + c.
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  const int krow0 = 8 * g + jj;  // plus 32s + 4h: bits 0, 1, 3 unchanged
  uint32_t boff[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int c = gw * 4 + 2 * j + (q >> 1);
    boff[j] = kBOff + krow0 * kBRowBytes + 16 * (c ^ swz_b(krow0)) + 8 * (q & 1);
  }

  float4v acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  half8 fa[4][4], fb[4][2];  // [k-step][block]
  auto read_frags = [&](int aslot, int bslot) {
    const uint32_t sa = lds_base + aslot * kHalfBytes;
    const uint32_t sb = lds_base + bslot * kBBytes;
    uint32_t va[4], vb[2];
#pragma unroll
    for (int s = 0; s < 4; s++) va[s] = sa + aoff[s];
#pragma unroll
    for (int j = 0; j < 2; j++) vb[j] = sb + boff[j];
    static_for<4>([&](auto sc) {
      constexpr int s = decltype(sc)::value;
      static_for<4>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        fa[s][i] = lds_read_h8_off<i * 16 * kRowBytes>(va[s]);
      });
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const half4 lo = lds_read_tr16_off<s * 32 * kBRowBytes>(vb[j]);
        const half4 hi = lds_read_tr16_off<s * 32 * kBRowBytes + 4 * kBRowBytes>(vb[j]);
        fb[s][j] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    });
  };
  // 32 MFMAs, each accumulator's 4 k-steps back to back, and the 8 loads
  // described by `o`, one after each accumulator.  Version 7's per-element
  // order: in each 64-deep half of the k-tile, block (i, j) takes k-step
  // (i ^ j) & 1 of the half first (the wave's block offsets are multiples of
  // 32, so i and j have the parity of the global 16-row and 16-column block
  // indices, as in version 7's 128 x 64 wave blocks).
  auto compute_and_load = [&](const DmaOps& o) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int j = 0; j < 2; j++) {
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
          const int s = s4 ^ ((i ^ j) & 1);
          acc[i][j] = mfma16x16x32(fb[s][j], fa[s][i], acc[i][j]);
          __builtin_amdgcn_sched_barrier(0);
        }
        dma_with(2 * i + j, o);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // Prologue and loop: version 7's phases and waits.
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
    __builtin_amdgcn_sched_barrier(0);  // the reads go out first
    const DmaOps ops = dma_ops(kt2, grp ? aslot : (t + 2) % kBSlots);
    pin_ops(ops);
    if (grp) wait_vmcnt<4>();  // Q: A-top(t+1) landed before barrier 2t+2
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    compute_and_load(ops);
    wait_vmcnt<8>();  // P: B(t+1); Q: A-top(t+1), A-bot(t+1)
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!grp) lds_barrier();
  wait_vmcnt<0>();
  lds_barrier();

  unsigned* cnt = nullptr;
  if constexpr (kSplit) {
    const __amdgpu_buffer_rsrc_t prsrc =
        __builtin_amdgcn_make_buffer_rsrc(part, 0, (int)((size_t)units * kSlotBytes), kBufferWord3);
    const SkPlan plan{0, units, pieces, chunks};
    auto part_off = [&](int q) {
      return (uint32_t)((size_t)sk_unit_of(plan, tiles_m * tiles_n, w.tile, q) * kSlotBytes) +
             (uint32_t)wave * kWaveSlotBytes;
    };
    cnt = counters + (size_t)w.tile * kSkWaves + wave;
    if (!split_arrive(acc, w.np, w.p, lane, prsrc, part_off, cnt)) return;
    split_sum(acc, w.np, w.p, lane, prsrc, part_off);
  }

  // ---- epilogue: the ring is idle; each wave stages its block in its own region ----
  const uint32_t wstage = lds_base + wave * Epi<OutT>::kRegion;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) Epi<OutT>::stage(wstage, lane, i, j, acc[i][j]);
  wait_lgkmcnt0();  // a wave reads back only its own region
  if constexpr (kEdge)
    Epi<OutT>::store_edge(wstage, C, M, N, m0 + grp * 64, n0 + gw * 32, lane);
  else
    Epi<OutT>::store(wstage, C + (size_t)(m0 + grp * 64) * N + n0 + gw * 32, N, lane);
  if constexpr (kSplit) {
    if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The split plan of a shape (tiles and k-tiles rounded up).
SkPlan plan_of(size_t m, size_t n, size_t k, int num_cus) {
  const int64_t tiles = (int64_t)(((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN));
  return sk_plan_fill(tiles, (int64_t)((k + kBK - 1) / kBK), num_cus);
}

size_t workspace(size_t m, size_t n, size_t k, int num_cus) {
  const SkPlan p = plan_of(m, n, k, num_cus);
  return p.units ? kSkCounterBytes + (size_t)p.units * kSlotBytes : 0;
}

template <typename OutT, bool kEdge, bool kSplit>
hipError_t launch_t(const GemmArgs& a, const SkPlan& p) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp128_kernel<OutT, kEdge, kSplit>;
  hipError_t e = ensure_lds_attr(kfn, kLdsBytes, a.device, attr_done);
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
  hipLaunchKernelGGL(kfn, dim3((unsigned)(kSplit ? p.units : p.dp)), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B), static_cast<OutT*>(a.C),
                     (int)a.m, (int)a.n, (int)a.k, p.units, p.pieces, p.chunks, part, counters);
  return hipGetLastError();
}

template <typename OutT>
hipError_t launch_out(const GemmArgs& a) {
  const SkPlan p = plan_of(a.m, a.n, a.k, a.num_cus);
  const bool grid = a.m % kBM == 0 && a.n % kBN == 0 && a.k % kBK == 0;
  if (p.units > 0) return grid ? launch_t<OutT, false, true>(a, p) : launch_t<OutT, true, true>(a, p);
  return grid ? launch_t<OutT, false, false>(a, p) : launch_t<OutT, true, false>(a, p);
}

// Shapes on the 128 x 128 x 128 grid run without the edge treatment.
hipError_t launch(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_out<half_t>(a) : launch_out<float>(a);
}

// 32-bit lane offsets (64 rows of A, 128 k-rows of B past the scalar base),
// each operand below 2^31 bytes with room for the last tile's rows and
// k-rows past it (buffer sizes; scalar plus lane offsets of the edge
// tiles), and the 1-D grid.
bool shape_ok(size_t m, size_t n, size_t k) {
  return m >= 1 && n >= 8 && k >= 8 && (size_t)kBM * k * 2 < (1ull << 31) && (size_t)kBK * n * 2 < (1ull << 31) &&
         (m + 2 * kBM) * k * 2 < (1ull << 31) && (k + 2 * kBK) * n * 2 < (1ull << 31) &&
         ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN) < (1ull << 31);
}

// ---------------------------------------------------------------------------
// Version 12: version 11's 128 x 128 tiles with 64 x 64 wave tiles.  In
// version 11 each wave computes a 64 x 32 block over every k-tile and reads
// 768 bytes of LDS fragments per MFMA; here each group of 4 waves takes
// alternate 64-deep k-tiles of the whole tile (P the even ones, Q the odd
// ones), each wave a 64 x 64 block (16 accumulators of 16 x 16), 512 bytes of
// fragments per MFMA, and the two groups' sums are added at the end.
//  * LDS ring: 5 slots of one k-tile (A 128 rows x 64 k, rows of 128 B with
//    chunk ^ (row / 2) % 8; B 64 k-rows x 128 columns, rows of 256 B with
//    version 11's transpose-read swizzle), 160 KB;
//  * phase p (one barrier each): group p % 2 computes k-tile p from
//    registers (32 MFMAs, each accumulator's 2 k-steps back to back) and
//    issues the 8 loads per wave of k-tile p + 5 into slot p % 5, which
//    k-tile p left; the other group reads k-tile p + 1's fragments and then
//    waits until its own loads of k-tile p + 2 (issued 2 of its compute
//    phases ago) have landed (vmcnt 8); each wave runs this as one loop over
//    its own k-tiles, memory phase then compute phase;
//  * afterwards P gives Q the right half of its block and Q gives P the left
//    half (through LDS), so each wave holds a 64 x 32 block of P + Q (the
//    sum of the even and of the odd k-tiles: fp32 addition commutes, so both
//    halves are the same sum) -- version 11's block shape, whose epilogue and
//    split hand-off are reused.
// Results differ from version 11's in the order of the k-sum (two chains
// added at the end) and are deterministic.  The split plan is version 11's,
// over 128-deep k-units, each piece taking the 64-deep k-tiles of its units.
namespace pp128w {

constexpr int kBK = 64;                             // k-tile
constexpr int kARow = kBK * 2;                      // 128 B: an A row of a k-tile
constexpr int kABytes = kBM * kARow;                // 16 KB
constexpr int kBRow = kBN * 2;                      // 256 B: a B k-row
constexpr int kSlot = kABytes + kBK * kBRow;        // 32 KB
constexpr int kSlots = 5;
constexpr int kLdsBytes = kSlots * kSlot;           // 160 KB
constexpr int kXchg = 64 * 1024;                    // the end's exchange regions: 8 x 8 KB
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(kXchg + 8 * 8192 <= kLdsBytes && 8 * Epi<float>::kRegion <= kXchg, "epilogue regions");

__host__ __device__ constexpr int swz_a8(int row) { return (row >> 1) & 7; }

template <typename OutT, bool kEdge, bool kSplit>
__global__ __launch_bounds__(kThreads) void f16_pp128w_kernel(const half_t* __restrict__ A,
                                                              const half_t* __restrict__ B,
                                                              OutT* __restrict__ C, int M, int N, int K, int units,
                                                              int pieces, int chunks, float* __restrict__ part,
                                                              unsigned* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;  // 0 = P (even k-tiles), 1 = Q (odd); waves w and w+4 share a SIMD
  const int gw = wave & 3;
  const int wr = gw >> 1, wc = gw & 1;  // the wave's 64 x 64 block of the tile
  constexpr int kR = kEdge ? 1 : 0;
  const int tiles_m = (M + kR * (kBM - 1)) / kBM, tiles_n = (N + kR * (kBN - 1)) / kBN;
  const int nk_all = (K + kR * (kBK - 1)) / kBK;
  int tm, tn, kb = 0, nk = nk_all;
  SkWork w{};
  if constexpr (kSplit) {
    w = sk_work(blockIdx.x, tiles_m * tiles_n, (nk_all + 1) / 2, SkPlan{0, units, pieces, chunks}, kFillLastExtra);
    raster_tile(w.cid, tiles_m, tiles_n, tm, tn);
    kb = 2 * w.kb;
    nk = min(2 * w.ke, nk_all) - kb;
  } else {
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  }
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  // ---- direct-to-LDS duty: 8 loads per wave per k-tile, issued by the group computing ----
  // A load i (0..3): rows 32 gw + 8 i + l / 8, lane l at chunk position l % 8,
  //   which holds chunk (l % 8) ^ swz_a8(row).
  // B load i (0..3): k-rows 16 gw + 4 i + l / 16, position l % 16, holding
  //   chunk (l % 16) ^ swz_b(krow).
  uint32_t voa[4], vob[4], akin = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = gw * 32 + 8 * i + (lane >> 3);
    const int ca = (lane & 7) ^ swz_a8(row);
    voa[i] = (uint32_t)(((size_t)row * K + ca * 8) * 2);
    akin |= (uint32_t)(ca * 8) << (8 * i);  // kEdge: the chunk's first k within the k-tile
    const int krow = gw * 16 + 4 * i + (lane >> 4);
    const int cb = (lane & 15) ^ swz_b(krow);
    vob[i] = (uint32_t)(((size_t)krow * N + cb * 8) * 2);
  }
  const char* ga0 = reinterpret_cast<const char*>(A) + ((size_t)m0 * K + (size_t)kb * kBK) * 2;
  const char* gb0 = reinterpret_cast<const char*>(B) + ((size_t)kb * kBK * N + n0) * 2;
  const uint32_t a_size = kEdge ? (uint32_t)((size_t)M * K * 2) : 0u;
  const uint32_t b_size = kEdge ? (uint32_t)((size_t)K * N * 2) : 0u;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(A), 0, (int)a_size, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(B), 0, (int)b_size, kBufferWord3);
  const uint32_t sa0 = (uint32_t)(ga0 - reinterpret_cast<const char*>(A));  // kEdge: below 2^31
  const uint32_t sb0 = (uint32_t)(gb0 - reinterpret_cast<const char*>(B));
  const uint32_t la0 = lds_base + (uint32_t)(gw * 32 * kARow);
  const uint32_t lb0 = lds_base + (uint32_t)(kABytes + gw * 16 * kBRow);

  struct Ops {
    const char* ga;
    const char* gb;
    uint32_t sa, sb;   // kEdge: scalar offsets into the buffers
    uint32_t kleft;    // kEdge: k from the k-tile's start to K
    uint32_t la, lb;   // LDS destination of load 0 (A, B)
  };
  auto ops_of = [&](int kt, int slot) {
    Ops o;
    o.ga = ga0 + (size_t)kt * kBK * 2;
    o.gb = gb0 + (size_t)kt * kBK * N * 2;
    o.sa = sa0 + (uint32_t)kt * (uint32_t)(kBK * 2);
    o.sb = sb0 + (uint32_t)kt * (uint32_t)(kBK * N * 2);
    o.kleft = kEdge ? (uint32_t)(K - (kb + kt) * kBK) : (uint32_t)kBK;
    o.la = la0 + (uint32_t)(slot * kSlot);
    o.lb = lb0 + (uint32_t)(slot * kSlot);
    return o;
  };
  auto pin = [&](const Ops& o) {
    if constexpr (kEdge)
      asm volatile("" ::"s"(o.sa), "s"(o.sb), "s"(o.kleft));
    else
      asm volatile("" ::"s"(o.ga), "s"(o.gb));
    asm volatile("" ::"s"(o.la), "s"(o.lb));
  };
  // load d: A for d < 4, B for d >= 4
  auto dma_with = [&](int d, const Ops& o) {
    const int i = d & 3;
    if (d < 4) {
      if constexpr (kEdge) {
        const uint32_t off = ((akin >> (8 * i)) & 255u) < o.kleft ? voa[i] : a_size;  // a_size: zeros
        dma16_buf(ra, off, o.sa, o.la + i * 1024);
      } else {
        dma16(o.ga, voa[i], o.la + i * 1024);
      }
    } else {
      if constexpr (kEdge)
        dma16_buf(rb, vob[i], o.sb, o.lb + i * 1024);
      else
        dma16(o.gb, vob[i], o.lb + i * 1024);
    }
  };
  auto dma_all = [&](int kt, int slot) {
    const Ops o = ops_of(kt, slot);
#pragma unroll
    for (int d = 0; d < 8; d++) dma_with(d, o);
  };

  // ---- fragment addresses ----
  // A block i (rows 64 wr + 16 i + l % 16), k-step s: chunk 4 s + l / 16,
  // swizzled by the row's bits 1..3 (= those of l % 16).
  const int arow = lane & 15;
  uint32_t aoff[2];
#pragma unroll
  for (int s = 0; s < 2; s++)
    aoff[s] = (uint32_t)((wr * 64 + arow) * kARow + 16 * ((4 * s + (lane >> 4)) ^ swz_a8(arow)));
  // B block j (columns 64 wc + 16 j ..), k-step s, half h: lane 16 g + 4 jj + q
  // names k-row 32 s + 8 g + 4 h + jj and the 8-byte half q % 2 of chunk
  // 8 wc + 2 j + q / 2 (as version 11).
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  const int krow0 = 8 * g + jj;
  uint32_t boff[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int c = wc * 8 + 2 * j + (q >> 1);
    boff[j] = (uint32_t)(kABytes + krow0 * kBRow + 16 * (c ^ swz_b(krow0)) + 8 * (q & 1));
  }

  float4v acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  half8 fa[2][4], fb[2][4];  // [k-step][block]
  auto read_frags = [&](int slot) {
    const uint32_t sl = lds_base + (uint32_t)(slot * kSlot);
    uint32_t va[2], vb[4];
#pragma unroll
    for (int s = 0; s < 2; s++) va[s] = sl + aoff[s];
#pragma unroll
    for (int j = 0; j < 4; j++) vb[j] = sl + boff[j];
    static_for<2>([&](auto sc) {
      constexpr int s = decltype(sc)::value;
      static_for<4>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        fa[s][i] = lds_read_h8_off<i * 16 * kARow>(va[s]);
      });
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const half4 lo = lds_read_tr16_off<s * 32 * kBRow>(vb[j]);
        const half4 hi = lds_read_tr16_off<s * 32 * kBRow + 4 * kBRow>(vb[j]);
        fb[s][j] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    });
  };
  // 32 MFMAs, each accumulator's 2 k-steps back to back, with the 8 loads of
  // `o` interleaved (one after every second accumulator).
  auto compute_and_load = [&](const Ops& o) {
#pragma unroll
    for (int x = 0; x < 16; x++) {
      const int i = x >> 2, j = x & 3;
      acc[i][j] = mfma16x16x32(fb[0][j], fa[0][i], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
      acc[i][j] = mfma16x16x32(fb[1][j], fa[1][i], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
      if (x & 1) {
        dma_with(x >> 1, o);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // ---- prologue: k-tiles 0..4 (Q loads the even ones, P the odd ones) ----
  // A k-tile past the last one is the last one again, into its own slot, so
  // every compute phase issues 8 loads and the waits stay fixed.
#pragma unroll
  for (int j = 0; j < kSlots; j++)
    if ((j & 1) != grp) dma_all(min(j, nk - 1), j);
  if (grp) wait_vmcnt<16>();  // Q: k-tile 0
  lds_barrier();
  // Every wave runs the same loop over its own k-tiles j = grp, grp + 2, ...:
  // a memory phase (phase j - 1: k-tile j's fragments, then the wait for this
  // group's loads of k-tile j + 1, issued two of its compute phases ago) and
  // a compute phase (phase j), one barrier after each.  Q starts one phase
  // later (phase -1 idle), and a group that computes no k-tile in the last
  // phase takes its barrier at the end, so every wave passes nk + 1 phase
  // barriers.  The fragments go from the reads to the MFMAs of the same
  // iteration, so they stay in their registers (their consumers come after
  // the barrier's lgkmcnt(0)).
  if (grp) lds_barrier();
  int phases = grp;
  for (int j = grp; j < nk; j += 2) {
    __builtin_amdgcn_sched_barrier(0);
    read_frags(j % kSlots);
    __builtin_amdgcn_sched_barrier(0);
    const Ops o = ops_of(min(j + kSlots, nk - 1), j % kSlots);
    pin(o);
    wait_vmcnt<8>();  // this group's loads of k-tile j + 1
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    compute_and_load(o);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    phases += 2;
  }
  __builtin_amdgcn_sched_barrier(0);
  if (phases < nk + 1) lds_barrier();
  wait_vmcnt<0>();
  lds_barrier();

  // ---- P + Q: P keeps columns 0..31 of the block (j = 0, 1), Q columns 32..63 ----
  {
    const uint32_t give = lds_base + (uint32_t)(kXchg + wave * 8192);
    const uint32_t take = lds_base + (uint32_t)(kXchg + (wave ^ 4) * 8192);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int h = 0; h < 2; h++) lds_write16(give + ((i * 2 + h) * 64 + lane) * 16, acc[i][grp ? h : 2 + h]);
    lds_barrier();
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const float4v o = __builtin_bit_cast(float4v, lds_read16(take + ((i * 2 + h) * 64 + lane) * 16));
        acc[i][h] = acc[i][grp ? 2 + h : h] + o;
      }
  }
  float4v blk[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int h = 0; h < 2; h++) blk[i][h] = acc[i][h];
  const int row0 = m0 + wr * 64, col0 = n0 + wc * 64 + grp * 32;

  unsigned* cnt = nullptr;
  if constexpr (kSplit) {
    const __amdgpu_buffer_rsrc_t prsrc =
        __builtin_amdgcn_make_buffer_rsrc(part, 0, (int)((size_t)units * kSlotBytes), kBufferWord3);
    const SkPlan plan{0, units, pieces, chunks};
    auto part_off = [&](int qq) {
      return (uint32_t)((size_t)sk_unit_of(plan, tiles_m * tiles_n, w.tile, qq) * kSlotBytes) +
             (uint32_t)wave * kWaveSlotBytes;
    };
    cnt = counters + (size_t)w.tile * kSkWaves + wave;
    if (!split_arrive(blk, w.np, w.p, lane, prsrc, part_off, cnt)) return;
    split_sum(blk, w.np, w.p, lane, prsrc, part_off);
  }

  // ---- epilogue: each wave stages its 64 x 32 block in its own region ----
  const uint32_t wstage = lds_base + wave * Epi<OutT>::kRegion;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int h = 0; h < 2; h++) Epi<OutT>::stage(wstage, lane, i, h, blk[i][h]);
  wait_lgkmcnt0();  // a wave reads back only its own region
  if constexpr (kEdge)
    Epi<OutT>::store_edge(wstage, C, M, N, row0, col0, lane);
  else
    Epi<OutT>::store(wstage, C + (size_t)row0 * N + col0, N, lane);
  if constexpr (kSplit) {
    if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <typename OutT, bool kEdge, bool kSplit>
hipError_t launch_t(const GemmArgs& a, const SkPlan& p) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp128w_kernel<OutT, kEdge, kSplit>;
  hipError_t e = ensure_lds_attr(kfn, kLdsBytes, a.device, attr_done);
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
  hipLaunchKernelGGL(kfn, dim3((unsigned)(kSplit ? p.units : p.dp)), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B), static_cast<OutT*>(a.C),
                     (int)a.m, (int)a.n, (int)a.k, p.units, p.pieces, p.chunks, part, counters);
  return hipGetLastError();
}

template <typename OutT>
hipError_t launch_out(const GemmArgs& a) {
  const SkPlan p = plan_of(a.m, a.n, a.k, a.num_cus);
  const bool grid = a.m % kBM == 0 && a.n % kBN == 0 && a.k % kBK == 0;
  if (p.units > 0) return grid ? launch_t<OutT, false, true>(a, p) : launch_t<OutT, true, true>(a, p);
  return grid ? launch_t<OutT, false, false>(a, p) : launch_t<OutT, true, false>(a, p);
}

hipError_t launch(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_out<half_t>(a) : launch_out<float>(a);
}

}  // namespace pp128w

// ---------------------------------------------------------------------------
// Version 13: version 11's tile and wave blocks (128 x 128 tiles, each wave a
// 64 x 32 block over every k-tile) without the ping-pong.  In version 11 one
// wave per SIMD reads fragments while the other computes, and a phase lasts
// as long as that one wave needs to get its 24 KB of LDS reads through
// (~820 cycles against ~580 of MFMA issue, measured): LDS serves a single
// reading wave per SIMD at ~142 B/clk/CU, two at ~222.  Here every wave
// computes its current 64-deep k-tile from registers while it reads the next
// k-tile's fragments into a second register set (one LDS read after each
// MFMA) and issues its 4 loads of the k-tile 4 ahead, so both waves of a SIMD
// read and compute at once; one barrier per k-tile.
//  * LDS ring: 5 slots of one k-tile, version 12's (A 128 rows x 64 k, rows
//    of 128 B, chunk ^ (row / 2) % 8; B 64 k-rows x 128 columns, rows of
//    256 B, version 11's transpose-read swizzle), 160 KB;
//  * step t: compute k-tile t (fragments read during step t - 1), read
//    k-tile t + 1's fragments, load k-tile t + 4 into slot (t + 4) % 5 (its
//    previous k-tile, t - 1, was read during step t - 2); then wait for this
//    wave's loads of k-tile t + 2 (vmcnt 8: the 4 loads of steps t - 1 and t
//    may still fly) and barrier;
//  * loads per step: wave w loads A rows 16 w .. 16 w + 15 (2 loads of 8
//    rows) and B k-rows 8 w .. 8 w + 7 (2 loads of 4 k-rows);
//  * each element is the same chain of MFMAs over 32-deep k-steps as in
//    versions 7 and 11 (64-deep k-tiles ascending, k-step (i ^ j) & 1 of each
//    first; bitwise equal where they run whole tiles).  Epilogue, edges and split hand-off are version 11's.
namespace pp128n {

using pp128w::kARow;
using pp128w::kABytes;
using pp128w::kBRow;
using pp128w::kSlot;
using pp128w::kSlots;
using pp128w::swz_a8;
constexpr int kBK = 64;
constexpr int kLdsBytes = kSlots * kSlot;  // 160 KB

template <typename OutT, bool kEdge, bool kSplit>
__global__ __launch_bounds__(kThreads) void f16_pp128n_kernel(const half_t* __restrict__ A,
                                                              const half_t* __restrict__ B,
                                                              OutT* __restrict__ C, int M, int N, int K, int units,
                                                              int pieces, int chunks, float* __restrict__ part,
                                                              unsigned* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;  // rows 64 grp .. 64 grp + 63 of the tile
  const int gw = wave & 3;    // columns 32 gw .. 32 gw + 31
  constexpr int kR = kEdge ? 1 : 0;
  const int tiles_m = (M + kR * (kBM - 1)) / kBM, tiles_n = (N + kR * (kBN - 1)) / kBN;
  const int nk_all = (K + kR * (kBK - 1)) / kBK;
  int tm, tn, kb = 0, nk = nk_all;
  SkWork w{};
  if constexpr (kSplit) {
    w = sk_work(blockIdx.x, tiles_m * tiles_n, (nk_all + 1) / 2, SkPlan{0, units, pieces, chunks}, kFillLastExtra);
    raster_tile(w.cid, tiles_m, tiles_n, tm, tn);
    kb = 2 * w.kb;
    nk = min(2 * w.ke, nk_all) - kb;
  } else {
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  }
  const int m0 = tm * kBM, n0 = tn * kBN;
  const uint32_t lds_base = lds_addr32(lds);

  // ---- loads: 4 per wave per k-tile ----
  // A load i (0, 1): rows 16 wave + 8 i + l / 8, lane l at chunk position
  //   l % 8, holding chunk (l % 8) ^ swz_a8(row).
  // B load i (0, 1): k-rows 8 wave + 4 i + l / 16, position l % 16, holding
  //   chunk (l % 16) ^ swz_b(krow).
  uint32_t voa[2], vob[2], akin = 0;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int row = wave * 16 + 8 * i + (lane >> 3);
    const int ca = (lane & 7) ^ swz_a8(row);
    voa[i] = (uint32_t)(((size_t)row * K + ca * 8) * 2);
    akin |= (uint32_t)(ca * 8) << (8 * i);  // kEdge: the chunk's first k within the k-tile
    const int krow = wave * 8 + 4 * i + (lane >> 4);
    const int cb = (lane & 15) ^ swz_b(krow);
    vob[i] = (uint32_t)(((size_t)krow * N + cb * 8) * 2);
  }
  const char* ga0 = reinterpret_cast<const char*>(A) + ((size_t)m0 * K + (size_t)kb * kBK) * 2;
  const char* gb0 = reinterpret_cast<const char*>(B) + ((size_t)kb * kBK * N + n0) * 2;
  const uint32_t a_size = kEdge ? (uint32_t)((size_t)M * K * 2) : 0u;
  const uint32_t b_size = kEdge ? (uint32_t)((size_t)K * N * 2) : 0u;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(A), 0, (int)a_size, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(B), 0, (int)b_size, kBufferWord3);
  const uint32_t sa0 = (uint32_t)(ga0 - reinterpret_cast<const char*>(A));  // kEdge: below 2^31
  const uint32_t sb0 = (uint32_t)(gb0 - reinterpret_cast<const char*>(B));
  const uint32_t la0 = lds_base + (uint32_t)(wave * 16 * kARow);
  const uint32_t lb0 = lds_base + (uint32_t)(kABytes + wave * 8 * kBRow);

  struct Ops {
    const char* ga;
    const char* gb;
    uint32_t sa, sb, kleft, la, lb;
  };
  auto ops_of = [&](int kt, int slot) {
    Ops o;
    o.ga = ga0 + (size_t)kt * kBK * 2;
    o.gb = gb0 + (size_t)kt * kBK * N * 2;
    o.sa = sa0 + (uint32_t)kt * (uint32_t)(kBK * 2);
    o.sb = sb0 + (uint32_t)kt * (uint32_t)(kBK * N * 2);
    o.kleft = kEdge ? (uint32_t)(K - (kb + kt) * kBK) : (uint32_t)kBK;
    o.la = la0 + (uint32_t)(slot * kSlot);
    o.lb = lb0 + (uint32_t)(slot * kSlot);
    return o;
  };
  auto pin = [&](const Ops& o) {
    if constexpr (kEdge)
      asm volatile("" ::"s"(o.sa), "s"(o.sb), "s"(o.kleft));
    else
      asm volatile("" ::"s"(o.ga), "s"(o.gb));
    asm volatile("" ::"s"(o.la), "s"(o.lb));
  };
  // load d: A for d < 2, B for d >= 2
  auto dma_with = [&](int d, const Ops& o) {
    const int i = d & 1;
    if (d < 2) {
      if constexpr (kEdge) {
        const uint32_t off = ((akin >> (8 * i)) & 255u) < o.kleft ? voa[i] : a_size;  // a_size: zeros
        dma16_buf(ra, off, o.sa, o.la + i * 1024);
      } else {
        dma16(o.ga, voa[i], o.la + i * 1024);
      }
    } else {
      if constexpr (kEdge)
        dma16_buf(rb, vob[i], o.sb, o.lb + i * 1024);
      else
        dma16(o.gb, vob[i], o.lb + i * 1024);
    }
  };
  auto dma_all = [&](int kt, int slot) {
    const Ops o = ops_of(kt, slot);
#pragma unroll
    for (int d = 0; d < 4; d++) dma_with(d, o);
  };

  // ---- fragment addresses (version 12's A rows, version 11's B columns) ----
  const int arow = lane & 15;
  uint32_t aoff[2];
#pragma unroll
  for (int s = 0; s < 2; s++)
    aoff[s] = (uint32_t)((grp * 64 + arow) * kARow + 16 * ((4 * s + (lane >> 4)) ^ swz_a8(arow)));
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  const int krow0 = 8 * g + jj;
  uint32_t boff[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int c = gw * 4 + 2 * j + (q >> 1);
    boff[j] = (uint32_t)(kABytes + krow0 * kBRow + 16 * (c ^ swz_b(krow0)) + 8 * (q & 1));
  }

  float4v acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  // Fragments of one k-tile: A blocks i, B blocks j, k-steps s.
  struct Frags {
    half8 a[2][4], b[2][2];
  };
  // Read number r (0..15) of a k-tile's fragments: r < 8 the A read (s, i) =
  // (r / 4, r % 4), then the B half-reads (s, j, h).
  auto read_one = [&](Frags& f, uint32_t sl, auto rc) {
    constexpr int r = decltype(rc)::value;
    if constexpr (r < 8) {
      constexpr int s = r / 4, i = r % 4;
      f.a[s][i] = lds_read_h8_off<i * 16 * kARow>(sl + aoff[s]);
    } else {
      constexpr int s = (r - 8) / 4, j = ((r - 8) / 2) % 2, h = (r - 8) % 2;
      const half4 v = lds_read_tr16_off<s * 32 * kBRow + h * 4 * kBRow>(sl + boff[j]);
      if constexpr (h == 0) {
        f.b[s][j][0] = v[0]; f.b[s][j][1] = v[1]; f.b[s][j][2] = v[2]; f.b[s][j][3] = v[3];
      } else {
        f.b[s][j][4] = v[0]; f.b[s][j][5] = v[1]; f.b[s][j][6] = v[2]; f.b[s][j][7] = v[3];
      }
    }
  };
  auto read_all = [&](Frags& f, int slot) {
    const uint32_t sl = lds_base + (uint32_t)(slot * kSlot);
    static_for<16>([&](auto rc) { read_one(f, sl, rc); });
  };
  // One step: the 16 MFMAs of `cur` (each accumulator's 2 k-steps back to
  // back, k-step (i ^ j) & 1 first as in versions 7 and 11), after each one
  // a read of `nxt` (when there is a next k-tile), and the 4 loads of `o`
  // after every 4 MFMAs.
  auto step = [&](const Frags& cur, Frags& nxt, int nslot, bool has_next, const Ops& o) {
    const uint32_t sl = lds_base + (uint32_t)(nslot * kSlot);
    static_for<8>([&](auto xc) {
      constexpr int x = decltype(xc)::value;
      constexpr int i = x >> 1, j = x & 1;
      constexpr int k0 = (i ^ j) & 1;
      acc[i][j] = mfma16x16x32(cur.b[k0][j], cur.a[k0][i], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
      if (has_next) read_one(nxt, sl, std::integral_constant<int, 2 * x>{});
      __builtin_amdgcn_sched_barrier(0);
      acc[i][j] = mfma16x16x32(cur.b[k0 ^ 1][j], cur.a[k0 ^ 1][i], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
      if (has_next) read_one(nxt, sl, std::integral_constant<int, 2 * x + 1>{});
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (x & 1) {
        dma_with(x >> 1, o);
        __builtin_amdgcn_sched_barrier(0);
      }
    });
  };

  // ---- prologue: k-tiles 0..3 (a k-tile past the last one is the last one again) ----
#pragma unroll
  for (int j = 0; j < 4; j++) dma_all(min(j, nk - 1), j);
  Frags f0, f1;
  wait_vmcnt<12>();  // k-tile 0
  lds_barrier();
  read_all(f0, 0);
  wait_vmcnt<8>();  // k-tile 1
  lds_barrier();
  // Steps in pairs, so the two fragment sets keep their registers.
  int t = 0;
  for (; t + 1 < nk; t += 2) {
    {
      const Ops o = ops_of(min(t + 4, nk - 1), (t + 4) % kSlots);
      pin(o);
      __builtin_amdgcn_sched_barrier(0);
      step(f0, f1, (t + 1) % kSlots, true, o);
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<8>();  // this wave's loads of k-tile t + 2
      lds_barrier();
    }
    {
      const Ops o = ops_of(min(t + 5, nk - 1), (t + 5) % kSlots);
      pin(o);
      __builtin_amdgcn_sched_barrier(0);
      step(f1, f0, (t + 2) % kSlots, t + 2 < nk, o);
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<8>();  // this wave's loads of k-tile t + 3
      lds_barrier();
    }
  }
  if (t < nk) {  // an odd last k-tile
    const Ops o = ops_of(nk - 1, (t + 4) % kSlots);
    pin(o);
    __builtin_amdgcn_sched_barrier(0);
    step(f0, f1, 0, false, o);
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vmcnt<0>();
  lds_barrier();

  const int row0 = m0 + grp * 64, col0 = n0 + gw * 32;
  unsigned* cnt = nullptr;
  if constexpr (kSplit) {
    const __amdgpu_buffer_rsrc_t prsrc =
        __builtin_amdgcn_make_buffer_rsrc(part, 0, (int)((size_t)units * kSlotBytes), kBufferWord3);
    const SkPlan plan{0, units, pieces, chunks};
    auto part_off = [&](int qq) {
      return (uint32_t)((size_t)sk_unit_of(plan, tiles_m * tiles_n, w.tile, qq) * kSlotBytes) +
             (uint32_t)wave * kWaveSlotBytes;
    };
    cnt = counters + (size_t)w.tile * kSkWaves + wave;
    if (!split_arrive(acc, w.np, w.p, lane, prsrc, part_off, cnt)) return;
    split_sum(acc, w.np, w.p, lane, prsrc, part_off);
  }

  const uint32_t wstage = lds_base + wave * Epi<OutT>::kRegion;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) Epi<OutT>::stage(wstage, lane, i, j, acc[i][j]);
  wait_lgkmcnt0();  // a wave reads back only its own region
  if constexpr (kEdge)
    Epi<OutT>::store_edge(wstage, C, M, N, row0, col0, lane);
  else
    Epi<OutT>::store(wstage, C + (size_t)row0 * N + col0, N, lane);
  if constexpr (kSplit) {
    if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <typename OutT, bool kEdge, bool kSplit>
hipError_t launch_t(const GemmArgs& a, const SkPlan& p) {
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_pp128n_kernel<OutT, kEdge, kSplit>;
  hipError_t e = ensure_lds_attr(kfn, kLdsBytes, a.device, attr_done);
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
  hipLaunchKernelGGL(kfn, dim3((unsigned)(kSplit ? p.units : p.dp)), dim3(kThreads), kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B), static_cast<OutT*>(a.C),
                     (int)a.m, (int)a.n, (int)a.k, p.units, p.pieces, p.chunks, part, counters);
  return hipGetLastError();
}

template <typename OutT>
hipError_t launch_out(const GemmArgs& a) {
  const SkPlan p = plan_of(a.m, a.n, a.k, a.num_cus);
  const bool grid = a.m % kBM == 0 && a.n % kBN == 0 && a.k % kBK == 0;
  if (p.units > 0) return grid ? launch_t<OutT, false, true>(a, p) : launch_t<OutT, true, true>(a, p);
  return grid ? launch_t<OutT, false, false>(a, p) : launch_t<OutT, true, false>(a, p);
}

hipError_t launch(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_out<half_t>(a) : launch_out<float>(a);
}

}  // namespace pp128n
}  // namespace pp128
}  // namespace

void register_f16_pp128() {
  KernelEntry e{};
  e.version = 11;
  e.in_dtype = VK_DTYPE_F16;
  e.name = "f16_v11_pp128_bk128";
  e.caps = make_caps(11, VK_DTYPE_F16, kOutF16 | kOutF32, 1, 8, 8, 16, pp128::kBM,
                     pp128::kBN, pp128::kBK, pp128::kThreads, pp128::kLdsBytes, 0, 0);
  e.caps.uses_workspace = 1;
  e.launch = pp128::launch;
  e.workspace = pp128::workspace;
  e.shape_ok = pp128::shape_ok;
  register_kernel(e);

  KernelEntry e12 = e;
  e12.version = 12;
  e12.name = "f16_v12_pp128_k64alt";
  e12.caps = make_caps(12, VK_DTYPE_F16, kOutF16 | kOutF32, 1, 8, 8, 16, pp128::kBM, pp128::kBN,
                       pp128::pp128w::kBK, pp128::kThreads, pp128::pp128w::kLdsBytes, 0, 0);
  e12.caps.uses_workspace = 1;
  e12.launch = pp128::pp128w::launch;
  register_kernel(e12);

  KernelEntry e13 = e12;
  e13.version = 13;
  e13.name = "f16_v13_pp128_both";
  e13.caps = make_caps(13, VK_DTYPE_F16, kOutF16 | kOutF32, 1, 8, 8, 16, pp128::kBM, pp128::kBN,
                       pp128::pp128n::kBK, pp128::kThreads, pp128::pp128n::kLdsBytes, 0, 0);
  e13.caps.uses_workspace = 1;
  e13.launch = pp128::pp128n::launch;
  register_kernel(e13);
}

}  // namespace vk
