// f16_dma.hip -- the fast fp16 GEMM family for gfx950 (versions 2..).
//
// Same job as the reference's champion lineage (results/ralph_loop_fable/src/
// matmul_f16/matmul_f16_v42_shfl2.cu:104-490: a 256x128x64 tile, a 3-stage
// cp.async ring, 8 warps of 64x64 mma.sync, an XOR-swizzled shared layout and
// a GW=8 panel raster), designed for CDNA4 instead of translated:
//
//  * Macro tile 256x256, 256 threads = 4 waves, each wave a 128x128 quadrant
//    computed as 4x4 v_mfma_f32_32x32x16_f16 blocks whose 256 fp32
//    accumulators per lane live in AGPRs (1 wave per SIMD).  At 4096^3 that is
//    256 tiles: exactly one per CU, no tail wave.
//  * Global -> LDS with global_load_lds_dwordx4 (16 B per lane, no VGPR
//    staging).  The hardware writes each wave's 1 KB contiguously, so the bank
//    swizzle is applied by choosing WHICH global 16-byte chunk each lane
//    fetches.
//  * A is kept [m][k] in LDS and read with ds_read_b128; B is kept [k][n] as it
//    sits in memory and read with ds_read_b64_tr_b16, the CDNA4 transpose
//    read, which hands each lane 4 consecutive k of one column -- the B operand
//    layout of the MFMA -- without any register shuffles.
//  * NSTAGE-deep LDS ring, prefetch distance NSTAGE-1, one barrier per k-tile.
//  * blockIdx -> tile mapping that keeps the 32 tiles of each XCD (workgroups
//    are dealt round-robin over the 8 XCDs) in a compact block of the tile grid
//    so they share A and B panels in that XCD's L2.
#include "vk_device.hpp"
#include "vk_internal.hpp"
#include "vk_tile.hpp"

#include <atomic>
#include <type_traits>

namespace vk {
namespace {

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kThreads = 256;
constexpr int kWaves = 4;

template <int BK, int NSTAGE>
struct Cfg {
  static constexpr int kAChunksPerRow = BK / 8;
  static constexpr int kABytes = kBM * BK * 2;
  static constexpr int kBBytes = BK * kBN * 2;
  static constexpr int kStageBytes = kABytes + kBBytes;
  static constexpr int kLdsBytes = kStageBytes * NSTAGE;
  static constexpr int kARowsPerInstr = 1024 / (BK * 2);            // rows per wave DMA
  static constexpr int kADma = kABytes / 1024 / kWaves;              // DMA instrs per wave (A)
  static constexpr int kBDma = kBBytes / 1024 / kWaves;              // DMA instrs per wave (B)
  static constexpr int kDmaPerStage = kADma + kBDma;
  static constexpr int kKSteps = BK / 16;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
  static_assert(kLdsBytes >= 4 * 128 * 128 * 2, "epilogue staging needs 128 KB");
};

// LDS bytes each wave uses to stage its 128x128 output block (fp16: the whole
// block; fp32: half of it per pass).
constexpr int kEpiWaveBytes = 128 * 128 * 2;

// fp16 output: the wave's 128x128 block, row pitch 256 B = 32 units of 8 B
// (4 halves), physical unit = unit ^ (row % 16).  A ds_write_b64 pass (16
// lanes: 16 consecutive rows of one unit) then covers the 16 unit positions
// of the 128-byte period in which LDS writes see the banks repeat (units
// chunk ^ (row % 16) at 16-byte granularity cost 4 conflict cycles per
// write).  A read takes units 2ch, 2ch+1 (16 B) from the 16-byte slot
// ch ^ (row % 16) / 2, its two halves swapped for odd rows; 4 rows per
// instruction.
template <typename OutT>
__device__ __forceinline__ typename std::enable_if<std::is_same<OutT, half_t>::value>::type
epilogue_store(float16v (&acc)[4][4], char*, uint32_t wbase, OutT* Cw, int N, int lane) {
  const int r0 = lane & 31, hsel = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const int row = i * 32 + r0;
        const int chunk = 4 * j + g4;
        half4 h = {(half_t)acc[i][j][4 * g4 + 0], (half_t)acc[i][j][4 * g4 + 1],
                   (half_t)acc[i][j][4 * g4 + 2], (half_t)acc[i][j][4 * g4 + 3]};
        lds_write8(wbase + row * 256 + 8 * ((2 * chunk + hsel) ^ (row & 15)), h);
      }
  const int rsub = lane >> 4, ch = lane & 15;
#pragma unroll
  for (int q = 0; q < 32; q++) {
    const int row = 4 * q + rsub;
    const uint4v u = lds_read16(wbase + row * 256 + 16 * (ch ^ ((row & 15) >> 1)));
    const bool odd = row & 1;
    const uint4v v = {odd ? u[2] : u[0], odd ? u[3] : u[1], odd ? u[0] : u[2], odd ? u[1] : u[3]};
    *reinterpret_cast<uint4v*>(Cw + (size_t)row * N + ch * 8) = v;
  }
}

// fp32 output: two passes of 64 rows (32 KB per wave each), row pitch 512 B =
// 32 chunks, physical chunk = chunk ^ (row % 32); 2 rows per read.
template <typename OutT>
__device__ __forceinline__ typename std::enable_if<std::is_same<OutT, float>::value>::type
epilogue_store(float16v (&acc)[4][4], char*, uint32_t wbase, OutT* Cw, int N, int lane) {
  const int r0 = lane & 31, hsel = lane >> 5;
#pragma unroll
  for (int pass = 0; pass < 2; pass++) {
#pragma unroll
    for (int ii = 0; ii < 2; ii++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          const int i = 2 * pass + ii;
          const int row = ii * 32 + r0;  // row within this pass
          const int chunk = 8 * j + 2 * g4 + hsel;
          float4v f = {acc[i][j][4 * g4 + 0], acc[i][j][4 * g4 + 1], acc[i][j][4 * g4 + 2],
                       acc[i][j][4 * g4 + 3]};
          lds_write16(wbase + row * 512 + 16 * (chunk ^ (row & 31)), f);
        }
    const int rsub = lane >> 5, ch = lane & 31;
#pragma unroll
    for (int q = 0; q < 32; q++) {
      const int row = 2 * q + rsub;
      const uint4v v = lds_read16(wbase + row * 512 + 16 * (ch ^ (row & 31)));
      *reinterpret_cast<uint4v*>(Cw + (size_t)(pass * 64 + row) * N + ch * 4) = v;
    }
    if (pass == 0) wait_lgkmcnt0();  // region reused next pass
  }
}

template <int BK, int NSTAGE, typename OutT>
__global__ __launch_bounds__(kThreads, 1) void f16_dma_kernel(const half_t* __restrict__ A,
                                                              const half_t* __restrict__ B,
                                                              OutT* __restrict__ C, int M, int N,
                                                              int K) {
  using G = Cfg<BK, NSTAGE>;
  extern __shared__ __attribute__((aligned(1024))) char lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  int tm, tn;
  tile_of(blockIdx.x, M / kBM, N / kBN, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;

  // ---- per-lane DMA source offsets (bytes, relative to the k-tile origin) ----
  uint32_t offA[G::kADma], offB[G::kBDma];
#pragma unroll
  for (int i = 0; i < G::kADma; i++) {
    const int row = wave * (kBM / kWaves) + i * G::kARowsPerInstr + lane / G::kAChunksPerRow;
    const int c = (lane % G::kAChunksPerRow) ^ swz_a<BK>(row);
    offA[i] = (uint32_t)(((size_t)row * K + c * 8) * 2);
  }
#pragma unroll
  for (int i = 0; i < G::kBDma; i++) {
    const int krow = wave * (BK / kWaves) + i * 2 + (lane >> 5);
    const int c = (lane & 31) ^ swz_b(krow);
    offB[i] = (uint32_t)(((size_t)krow * N + c * 8) * 2);
  }
  const char* gA = reinterpret_cast<const char*>(A) + (size_t)m0 * K * 2;
  const char* gB = reinterpret_cast<const char*>(B) + (size_t)n0 * 2;
  const size_t strideBk = (size_t)BK * N * 2;  // bytes per k-tile of B

  const uint32_t lds_base = lds_addr32(lds);
  // ---- per-lane LDS fragment offsets ----
  // A block i, k-step ks: row = wm*128 + i*32 + lane%32, chunk 2*ks + lane/32.
  const int arow = wm * 128 + (lane & 31);
  uint32_t aoff[G::kKSteps];
#pragma unroll
  for (int ks = 0; ks < G::kKSteps; ks++)
    aoff[ks] = arow * (BK * 2) + 16 * ((2 * ks + (lane >> 5)) ^ swz_a<BK>(arow));
  // B block j, k-step ks, half h: lane 16g + 4jj + q names row
  // ks*16 + 8*(g/2) + 4h + jj and columns wn*128 + j*32 + 16*(g%2) + 4q .. +3.
  const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
  uint32_t boff[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int krow0 = 8 * (g >> 1) + jj;  // plus ks*16 + 4h (multiples of 4)
    const int c = wn * 16 + j * 4 + 2 * (g & 1) + (q >> 1);
    boff[j] = krow0 * (kBN * 2) + 16 * (c ^ swz_b(krow0)) + 8 * (q & 1);
  }

  float16v acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  const int nk = K / BK;

  // One 16-deep k-step = 16 MFMAs over the current fragments.  Interleaved
  // with them, in a fixed order (sched_barrier after each slot): the 12 LDS
  // reads of the next k-step's fragments, ordered by when the next step's
  // MFMAs need them (A0, B0..B3, A1..A3), and optionally the direct-to-LDS
  // loads that refill a freed stage.  Each MFMA occupies the matrix pipe for
  // 8 passes, so one LDS or DMA issue between two MFMAs costs nothing.
  half8 fa[2][4], fb[2][4];
  half4 tlo[4], thi[4];

  auto read_slot = [&](int t, uint32_t stage_off, int ks, half8(&a)[4], half8(&b)[4]) {
    // t: 0 -> A0, 1..8 -> B0lo,B0hi,..,B3hi, 9..11 -> A1..A3
    const char* sA = lds + stage_off;
    const char* sB = sA + G::kABytes;
    if (t == 0 || t >= 9) {
      const int i = t == 0 ? 0 : t - 8;
      a[i] = *reinterpret_cast<const half8*>(sA + aoff[ks] + i * 32 * BK * 2);
    } else {
      const int j = (t - 1) >> 1, h = (t - 1) & 1;
      const half_t* p = reinterpret_cast<const half_t*>(sB + boff[j] + ks * 16 * kBN * 2) + h * 4 * kBN;
      if (h == 0) {
        tlo[j] = lds_read_tr16(p);
      } else {
        thi[j] = lds_read_tr16(p);
        b[j] = half8{tlo[j][0], tlo[j][1], tlo[j][2], tlo[j][3],
                     thi[j][0], thi[j][1], thi[j][2], thi[j][3]};
      }
    }
  };
  auto read_all = [&](uint32_t stage_off, int ks, half8(&a)[4], half8(&b)[4]) {
#pragma unroll
    for (int t = 0; t < 12; t++) read_slot(t, stage_off, ks, a, b);
  };

  // DMA slot d of a refill: A instructions first, then B.
  auto dma_slot = [&](int d, int stage, int kt) {
    const uint32_t sbase = lds_base + stage * G::kStageBytes;
    if (d < G::kADma) {
      dma16(gA + (size_t)kt * BK * 2, offA[d], sbase + (wave * G::kADma + d) * 1024);
    } else {
      const int i = d - G::kADma;
      dma16(gB + (size_t)kt * strideBk, offB[i], sbase + G::kABytes + (wave * G::kBDma + i) * 1024);
    }
  };

  // kReads: read the next k-step's fragments; kDma: refill `dstage` with
  // k-tile `dkt` (clamped to the last tile: past the end it rewrites a
  // buffer that is never read again, which keeps the vmcnt bookkeeping
  // constant and the loop free of branches around MFMAs).
  auto step = [&](auto kReads, auto kDma, int cur, uint32_t next_off, int next_ks, int dstage,
                  int dkt) {
    const int nxt = cur ^ 1;
#pragma unroll
    for (int t = 0; t < 16; t++) {
      const int i = t >> 2, j = t & 3;
      acc[i][j] = mfma32x32x16(fb[cur][j], fa[cur][i], acc[i][j]);  // C^T block, see epilogue
      if constexpr (decltype(kReads)::value) {
        if (t < 12) read_slot(t, next_off, next_ks, fa[nxt], fb[nxt]);
      }
      if constexpr (decltype(kDma)::value) {
        if (t < G::kDmaPerStage) dma_slot(t, dstage, dkt);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using True = std::true_type;
  using False = std::false_type;

  // Prologue: k-tiles 0..NSTAGE-2 in flight; once tile 0 has landed, tile
  // NSTAGE-1 goes into the last free stage.
#pragma unroll
  for (int s = 0; s < NSTAGE - 1; s++) {
    const int t = min(s, nk - 1);
#pragma unroll
    for (int d = 0; d < G::kDmaPerStage; d++) dma_slot(d, s, t);
  }
  wait_vmcnt<(NSTAGE - 2) * G::kDmaPerStage>();
  lds_barrier();
#pragma unroll
  for (int d = 0; d < G::kDmaPerStage; d++) dma_slot(d, NSTAGE - 1, min(NSTAGE - 1, nk - 1));
  read_all(0, 0, fa[0], fb[0]);

  // Every k-tile runs the same code (no peeled tail, which would make the
  // register allocator shuffle the 256 accumulators).  Its final k-step first
  // hands its stage back (tile kt+1 landed + barrier), then refills it with
  // tile kt+NSTAGE while its MFMAs overlap the reads of tile kt+1's first
  // fragments.  In the last tile those reads see a stale stage and are never
  // used.
  for (int kt = 0; kt < nk; kt++) {
    const int stage = kt % NSTAGE;
    const uint32_t soff = stage * G::kStageBytes;
#pragma unroll
    for (int ks = 0; ks + 1 < G::kKSteps; ks++) step(True{}, False{}, ks & 1, soff, ks + 1, 0, 0);
    wait_vmcnt<(NSTAGE - 2) * G::kDmaPerStage>();
    lds_barrier();
    step(True{}, True{}, (G::kKSteps - 1) & 1, ((kt + 1) % NSTAGE) * G::kStageBytes, 0, stage,
         min(kt + NSTAGE, nk - 1));
  }
  // Redundant tail refills may still be landing: drain them before the
  // workgroup can exit and its LDS be handed to another workgroup.
  wait_vmcnt<0>();

  // ---- epilogue: C tile staged through LDS, written as full 128-byte lines ----
  // The MFMAs computed C^T blocks (B fragment as the A operand): lane l,
  // register r of block (i, j) holds C[i*32 + l%32][j*32 + 8*(r/4) + 4*(l/32)
  // + r%4], i.e. 4 consecutive columns of one row per register group.  Each
  // wave writes those 4-value pieces into its own LDS region (the k-loop
  // stages are free once every wave has passed the barrier below), then reads
  // the region back row-contiguously so every global store instruction covers
  // whole 128-byte lines.  The 16-byte chunk index is XORed with the row
  // (mod 16 / mod 32) to spread the column-wise writes over the banks.
  lds_barrier();
  epilogue_store<OutT>(acc, lds + wave * kEpiWaveBytes, lds_addr32(lds) + wave * kEpiWaveBytes,
                       C + (size_t)(m0 + wm * 128) * N + n0 + wn * 128, N, lane);
}

template <int BK, int NSTAGE, typename OutT>
hipError_t launch_dma_t(const GemmArgs& a) {
  using G = Cfg<BK, NSTAGE>;
  static std::atomic<uint64_t> attr_done{0};
  auto kfn = f16_dma_kernel<BK, NSTAGE, OutT>;
  hipError_t e = ensure_lds_attr(kfn, G::kLdsBytes, a.device, attr_done);
  if (e != hipSuccess) return e;
  const int tiles = (int)((a.m / kBM) * (a.n / kBN));
  hipLaunchKernelGGL(kfn, dim3(tiles), dim3(kThreads), G::kLdsBytes, a.stream,
                     static_cast<const half_t*>(a.A), static_cast<const half_t*>(a.B),
                     static_cast<OutT*>(a.C), (int)a.m, (int)a.n, (int)a.k);
  return hipGetLastError();
}

template <int BK, int NSTAGE>
hipError_t launch_dma(const GemmArgs& a) {
  return a.out_dtype == VK_DTYPE_F16 ? launch_dma_t<BK, NSTAGE, half_t>(a)
                                     : launch_dma_t<BK, NSTAGE, float>(a);
}

// 32-bit byte offsets inside one 256-row panel of A and one BK-row slab of B
// must not overflow; the grid is 1-D.
bool dma_shape_ok(size_t m, size_t n, size_t k) {
  return (size_t)kBM * k * 2 < (1ull << 31) && (size_t)64 * n * 2 < (1ull << 31) &&
         (m / kBM) * (n / kBN) < (1ull << 31);
}

template <int BK, int NSTAGE>
void reg(int version, const char* name) {
  using G = Cfg<BK, NSTAGE>;
  KernelEntry e{};
  e.version = version;
  e.in_dtype = VK_DTYPE_F16;
  e.name = name;
  e.caps = make_caps(version, VK_DTYPE_F16, kOutF16 | kOutF32, kBM, kBN, BK, 16, kBM, kBN, BK,
                     kThreads, G::kLdsBytes, 0, 0);
  e.launch = launch_dma<BK, NSTAGE>;
  e.workspace = nullptr;
  e.shape_ok = dma_shape_ok;
  register_kernel(e);
}

}  // namespace

void register_f16_dma() {
  reg<64, 2>(2, "f16_v2_dma256_bk64x2");
  reg<32, 4>(3, "f16_v3_dma256_bk32x4");
}

}  // namespace vk
