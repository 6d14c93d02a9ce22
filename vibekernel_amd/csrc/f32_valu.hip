// f32_valu.hip -- fp32 SGEMM on the vector ALUs (version 1 for fp32).
//
// The reference has the fp32 harness path (results/naive_cycle4/include/
// playground/system.hpp:35-41, results/naive_fable_cycle2/src/CMakeLists.txt:5-11)
// and its v0 ground truth (matmul_f32_v0_cblas.cpp:8-12) but no hand-written
// fp32 kernel; its only GPU fp32 version called cublasSgemm.  Two
// register-blocked VALU kernels share one tile and thread mapping:
//   * 128x256 workgroup tile, BK = 16, 256 threads, 8x16 outputs per thread
//     held as 4x4 register blocks (rows ty*4 and 64+ty*4, columns
//     64*g + tx*4 for g = 0..3) so the LDS operand reads are 16-byte and
//     conflict-free; one barrier per k-tile over two LDS buffers;
//   * tile-divisible shapes: the k-loop as one asm block with hand-chosen
//     registers, k-tiles staged by direct-to-LDS loads (f32_valu_asm_kernel);
//   * any other shape: a C++ kernel with bounds checks, the next k-tile
//     prefetched into registers and stored into LDS (A transposed, k-major);
//     on grids of few 128x256 tiles the same kernel on 64x64 tiles (4x4
//     outputs per thread) fills more CUs.
// Roofline: the VOP2 FMA (`v_fmac_f32_e32`) runs at the full 157.3 TFLOP/s
// rate on MI355X (measured 146.7 on independent chains; the VOP3 form runs
// at half), unless its three VGPR operands share a register bank, which
// halves it.  The asm kernel's register layout rules that out: 106.0 TFLOP/s
// at 4096^3 against 92.3 for the C++ kernel, where the compiler had put a
// quarter of the FMAs' operands in one bank.  Both are power-limited (the
// board at its ~1.4 kW cap, SCLK 1.9 GHz for the asm kernel).
#include "vk_device.hpp"
#include "vk_internal.hpp"

namespace vk {
namespace {

constexpr int kTM = 128;             // tile rows
constexpr int kCG = 4;               // 64-column groups per tile
constexpr int kTN = 64 * kCG;        // tile columns
constexpr int kBK = 16;
constexpr int kApitch = kTM + 4;     // As_t[k][m] row pitch (floats)
constexpr int kLdA = kTM * kBK / 4 / 256;  // float4 loads of A per thread per k-tile
constexpr int kLdB = kBK * kTN / 4 / 256;  // float4 loads of B per thread per k-tile
static_assert(kLdA == 2 && kLdB == 4, "tile load mapping");

// kRB row blocks of 64 and kNG column groups of 64 per tile, kKT-deep
// k-tiles: 128x256x16 (the asm kernel's tile) or, for grids of few such
// tiles, 64x64x32 (4x4 outputs per thread, 4 k-steps per unrolled loop body),
// with the same per-element order.
template <bool kCheck, int kRB = 2, int kNG = kCG, int kKT = vk::kBK>
__global__ __launch_bounds__(256) void f32_valu_kernel(const float* __restrict__ A,
                                                       const float* __restrict__ B,
                                                       float* __restrict__ C, int64_t M, int64_t N,
                                                       int64_t K) {
  constexpr int kBK = kKT;  // k-tile depth
  constexpr int kUnroll = kRB * kNG == 1 ? 4 : 2;  // k-steps per unrolled loop body
  constexpr int kTM = 64 * kRB, kTN = 64 * kNG, kApitch = kTM + 4;
  constexpr int kLdA = kTM * kBK / 4 / 256, kLdB = kBK * kTN / 4 / 256;
  static_assert(kLdA * 1024 == kTM * kBK && kLdB * 1024 == kBK * kTN, "whole float4 loads per thread");
  __shared__ __attribute__((aligned(16))) float As[2][kBK * kApitch];
  __shared__ __attribute__((aligned(16))) float Bs[2][kBK * kTN];

  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * kTM;
  const int64_t n0 = (int64_t)blockIdx.x * kTN;

  // Global load mapping: A: TM rows x BK/4 float4 per row; B: BK rows x TN/4 float4.
  constexpr int kC4A = kBK / 4;   // float4 per A row
  constexpr int kC4B = kTN / 4;   // float4 per B row
  float4v ra[kLdA], rb[kLdB];
  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int e = 0; e < kLdA; e++) {
      const int idx = tid + 256 * e;
      const int row = idx / kC4A, c4 = idx % kC4A;
      const int64_t gr = m0 + row, gc = k0 + c4 * 4;
      if (!kCheck) {
        ra[e] = *reinterpret_cast<const float4v*>(&A[gr * K + gc]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++)
          ra[e][q] = (gr < M && gc + q < K) ? A[gr * K + gc + q] : 0.0f;
      }
    }
#pragma unroll
    for (int e = 0; e < kLdB; e++) {
      const int idx = tid + 256 * e;
      const int krow = idx / kC4B, c4 = idx % kC4B;
      const int64_t gr = k0 + krow, gc = n0 + c4 * 4;
      if (!kCheck) {
        rb[e] = *reinterpret_cast<const float4v*>(&B[gr * N + gc]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++)
          rb[e][q] = (gr < K && gc + q < N) ? B[gr * N + gc + q] : 0.0f;
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int e = 0; e < kLdA; e++) {
      const int idx = tid + 256 * e;
      const int row = idx / kC4A, c4 = idx % kC4A;
#pragma unroll
      for (int q = 0; q < 4; q++) As[buf][(c4 * 4 + q) * kApitch + row] = ra[e][q];
    }
#pragma unroll
    for (int e = 0; e < kLdB; e++) {
      const int idx = tid + 256 * e;
      const int krow = idx / kC4B, c4 = idx % kC4B;
      *reinterpret_cast<float4v*>(&Bs[buf][krow * kTN + c4 * 4]) = rb[e];
    }
  };

  float acc[4 * kRB][4 * kNG];
#pragma unroll
  for (int i = 0; i < 4 * kRB; i++)
#pragma unroll
    for (int j = 0; j < 4 * kNG; j++) acc[i][j] = 0.0f;

  const int64_t nk = (K + kBK - 1) / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; kt++) {
    const int cur = (int)(kt & 1);
    if (kt + 1 < nk) load_tile((kt + 1) * kBK);
#pragma unroll kUnroll
    for (int kk = 0; kk < kBK; kk++) {
      float a[4 * kRB];
#pragma unroll
      for (int r = 0; r < kRB; r++) {
        const float4v ar = *reinterpret_cast<const float4v*>(&As[cur][kk * kApitch + 64 * r + ty * 4]);
#pragma unroll
        for (int q = 0; q < 4; q++) a[4 * r + q] = ar[q];
      }
      float b[4 * kNG];
#pragma unroll
      for (int g = 0; g < kNG; g++) {
        const float4v bg = *reinterpret_cast<const float4v*>(&Bs[cur][kk * kTN + 64 * g + tx * 4]);
#pragma unroll
        for (int q = 0; q < 4; q++) b[4 * g + q] = bg[q];
      }
#pragma unroll
      for (int i = 0; i < 4 * kRB; i++)
#pragma unroll
        for (int j = 0; j < 4 * kNG; j++) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    if (kt + 1 < nk) {
      store_tile(cur ^ 1);
      __syncthreads();
    }
  }

#pragma unroll
  for (int i = 0; i < 4 * kRB; i++) {
    const int64_t row = m0 + 64 * (i / 4) + ty * 4 + i % 4;
#pragma unroll
    for (int g = 0; g < kNG; g++) {
      const int64_t col = n0 + g * 64 + tx * 4;
      if (!kCheck) {
        float4v v = {acc[i][g * 4 + 0], acc[i][g * 4 + 1], acc[i][g * 4 + 2], acc[i][g * 4 + 3]};
        *reinterpret_cast<float4v*>(&C[row * N + col]) = v;
      } else if (row < M) {
#pragma unroll
        for (int q = 0; q < 4; q++)
          if (col + q < N) C[row * N + col + q] = acc[i][g * 4 + q];
      }
    }
  }
}

// Every VGPR from v32 up: the registers the asm kernel below uses itself.
#define VK_CLOBBER_V32_V255 \
  "v32", "v33", "v34", "v35", "v36", "v37", "v38", "v39", "v40", "v41", "v42", "v43", "v44", "v45", "v46", \
  "v47", "v48", "v49", "v50", "v51", "v52", "v53", "v54", "v55", "v56", "v57", "v58", "v59", "v60", "v61", \
  "v62", "v63", "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", \
  "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", "v91", \
  "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", "v105", \
  "v106", "v107", "v108", "v109", "v110", "v111", "v112", "v113", "v114", "v115", "v116", "v117", "v118", \
  "v119", "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127", "v128", "v129", "v130", "v131", \
  "v132", "v133", "v134", "v135", "v136", "v137", "v138", "v139", "v140", "v141", "v142", "v143", "v144", \
  "v145", "v146", "v147", "v148", "v149", "v150", "v151", "v152", "v153", "v154", "v155", "v156", "v157", \
  "v158", "v159", "v160", "v161", "v162", "v163", "v164", "v165", "v166", "v167", "v168", "v169", "v170", \
  "v171", "v172", "v173", "v174", "v175", "v176", "v177", "v178", "v179", "v180", "v181", "v182", "v183", \
  "v184", "v185", "v186", "v187", "v188", "v189", "v190", "v191", "v192", "v193", "v194", "v195", "v196", \
  "v197", "v198", "v199", "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", \
  "v210", "v211", "v212", "v213", "v214", "v215", "v216", "v217", "v218", "v219", "v220", "v221", "v222", \
  "v223", "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", \
  "v236", "v237", "v238", "v239", "v240", "v241", "v242", "v243", "v244", "v245", "v246", "v247", "v248", \
  "v249", "v250", "v251", "v252", "v253", "v254", "v255"

// Tile order of the asm kernel (a 1-D grid): workgroups are dealt round-robin
// over the 8 XCDs (workgroup b runs on XCD b % 8), so XCD x gets raster
// positions [x T / 8, (x + 1) T / 8) when 8 divides the tile count T; the
// raster walks 8 row panels at a time, column strip by column strip, so an
// XCD's share is a block of 8 row panels x T / 64 column strips (at 4096^3:
// 8 x 8 tiles, 16 MB of A panels and 32 MB of B strips per XCD, where the
// row-major 2-D grid gave each XCD all 32 A panels and 2 B strips).
__host__ __device__ __forceinline__ void f32_tile_of(uint32_t bid, uint32_t tiles_m, uint32_t tiles_n, uint32_t& tm,
                                                     uint32_t& tn) {
  constexpr uint32_t GM = 8;
  const uint32_t total = tiles_m * tiles_n;
  const uint32_t cid = (total & 7) == 0 ? (bid & 7) * (total >> 3) + (bid >> 3) : bid;
  const uint32_t group = GM * tiles_n;
  const uint32_t g = cid / group;
  const uint32_t first_m = g * GM;
  const uint32_t gm = tiles_m - first_m < GM ? tiles_m - first_m : GM;
  const uint32_t r = cid - g * group;
  tm = first_m + r % gm;
  tn = r / gm;
}

// The asm kernel's 32-bit byte offsets: A's 128-row panel, B's 256-column
// strip over all of K, and C's 128-row panel.
bool asm_offsets_fit(size_t m, size_t n, size_t k) {
  (void)m;
  const uint64_t lim = 1ull << 32;
  return 128ull * k * 4 < lim && (uint64_t)k * n * 4 < lim && 128ull * n * 4 < lim && n < (1ull << 31) &&
         k < (1ull << 31);
}

// ---------------------------------------------------------------------------
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Full tiles (M % 128, N % 256, K % 16 == 0, 16-byte aligned operands): the
// same tile, thread mapping and summation order as the kernel above, with
// the k-loop written as one asm block so that the registers are chosen here
// rather than by the compiler, and the k-tiles staged by direct-to-LDS loads.
//
// Registers.  A v_fmac_f32 whose three operands (accumulator, a, b) sit in
// the same VGPR bank (register number mod 4) issues at half rate; with two in
// one bank there is no measurable loss (microbenchmarks on MI355X: 63-70
// against 124-139 TFLOP/s).  For the C++ kernel the compiler put every
// accumulator in its b operand's bank, and a quarter of the 256 FMAs of a
// k-step pair also had a in that bank.  Here:
//   acc[i][j]  v[128 + 16 i + ((j + 1) % 16)]   bank (j + 1) % 4
//   b[j]       v[64 + j] / v[80 + j]            bank j % 4  (2 buffers, one k-step)
//   a          v[32:63] / v[96:127]             (2 buffers, 4 k-steps)
// so an accumulator never shares b's bank and no FMA has three operands in
// one bank.  The inputs the compiler supplies live below v32 (every register
// from v32 up is declared clobbered).
//
// Staging.  Each wave issues 6 direct-to-LDS loads per k-tile (2 x 16 rows
// of A, 4 k-rows of B) into the other of two LDS buffers right after the
// barrier that freed it, and waits for its own loads (vmcnt) before the next
// barrier: no staging VGPRs and no LDS stores.  A is kept row-major in LDS
// (row pitch 64 B = 4 chunks of 16 B = 4 k), chunk ^ ((row / 4) % 4), so
// the rows ty*4 + i of the four ty of a wave fall in four distinct chunks;
// B as loaded (k-row pitch 1 KB).  One ds_read_b128 of A gives a thread four
// consecutive k of one row, so A is read per group of 4 k-steps (8 reads:
// rows ty*4 + i and 64 + ty*4 + i) into a[i][kk] = v[AQ + 4 i + kk % 4]; each
// k-step issues the next k-step's four B reads (and, before a group's last
// k-step, the next group's 8 A reads) into the other buffers ahead of its
// 128 FMAs.  Measured on MI355X at 4096^3 (interleaved, 3 pairs, one box):
// 1296.5 us against 1310.4 us for the same k-loop staged through registers
// with A transposed by 4-byte LDS stores (106.0 against 104.9 TFLOP/s).
// Each output is one v_fmac_f32 per k in ascending order from 0: the same
// sums, bit for bit, as the C++ kernel and the oracle.  C is stored with sc1
// (written through the XCD's L2, not left dirty for the end-of-kernel
// write-back): 1302.5 against 1314.6 us per launch at 4096^3 (3 interleaved
// rounds on one box).
__global__ __launch_bounds__(256) void f32_valu_asm_kernel(const float* __restrict__ A,
                                                           const float* __restrict__ B, float* __restrict__ C,
                                                           int M, int N, int K) {
  __shared__ __attribute__((aligned(1024))) float As[2][kTM * kBK];
  __shared__ __attribute__((aligned(1024))) float Bs[2][kBK * kTN];
  const uint32_t tid = threadIdx.x;
  const uint32_t tx = tid & 15, ty = tid >> 4, lane = tid & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint32_t tm, tn;
  f32_tile_of(blockIdx.x, (uint32_t)M / kTM, (uint32_t)N / kTN, tm, tn);
  const size_t m0 = (size_t)tm * kTM, n0 = (size_t)tn * kTN;
  const char* abase = reinterpret_cast<const char*>(A + m0 * (size_t)K);
  const char* bbase = reinterpret_cast<const char*>(B + n0);
  char* cbase = reinterpret_cast<char*>(C + m0 * (size_t)N + n0);
  // Loads: A instruction e covers rows 32w + 16e + lane/4, the lane's 16 B
  // landing at chunk position lane % 4, which holds k-chunk
  // (lane % 4) ^ ((row / 4) % 4); B instruction e covers k-row w + 4e.
  const uint32_t arow0 = 32 * w + (lane >> 2), arow1 = arow0 + 16;
  uint32_t ga0 = (arow0 * (uint32_t)K + 4 * ((lane & 3) ^ ((arow0 >> 2) & 3))) * 4;
  uint32_t ga1 = (arow1 * (uint32_t)K + 4 * ((lane & 3) ^ ((arow1 >> 2) & 3))) * 4;
  uint32_t gb0 = (w * (uint32_t)N + lane * 4) * 4;
  uint32_t gb1 = gb0 + 4u * (uint32_t)N * 4, gb2 = gb1 + 4u * (uint32_t)N * 4, gb3 = gb2 + 4u * (uint32_t)N * 4;
  const uint32_t astep = kBK * 4, bstep = (uint32_t)kBK * (uint32_t)N * 4;
  const uint32_t as0 = lds_addr32(As[0]), as1 = lds_addr32(As[1]);
  const uint32_t bs0 = lds_addr32(Bs[0]), bs1 = lds_addr32(Bs[1]);
  // LDS destinations of this wave's loads (wave-uniform) and their sums over
  // the two buffers, so that dst = sum - dst switches buffers.
  uint32_t a_dst = as0 + w * 2048, b_dst = bs0 + w * 1024;
  const uint32_t sa_dst = as0 + as1 + 2 * w * 2048, sb_dst = bs0 + bs1 + 2 * w * 1024;
  // Reads: A at rd_a ^ 16 c for k-chunk c (rd_a's bits 4-5 hold (ty % 4) * 16
  // over a 256-aligned row-block base), rows by immediate offsets.
  uint32_t rd_a = as0 + ty * 256 + 16 * (ty & 3), rd_b = bs0 + tx * 16;
  const uint32_t sum_a = as0 + as1 + 2 * (ty * 256 + 16 * (ty & 3)), sum_b = bs0 + bs1 + 2 * (tx * 16);
  uint32_t c_lo = ((ty * 4) * (uint32_t)N + tx * 4) * 4;
  uint32_t c_hi = c_lo + 64u * (uint32_t)N * 4;
  const uint32_t crow = (uint32_t)N * 4;
  uint32_t nk = (uint32_t)K / kBK;
  uint32_t tmp;

  asm volatile(
      // k-tile loads at the current global offsets into the LDS buffer at a_dst / b_dst
      ".macro VK_DMA\n"
      "  s_mov_b32 m0, %[a_dst]\n"
      "  s_nop 0\n"
      "  global_load_lds_dwordx4 %[ga0], %[abase]\n"
      "  s_add_u32 m0, %[a_dst], 1024\n"
      "  s_nop 0\n"
      "  global_load_lds_dwordx4 %[ga1], %[abase]\n"
      "  s_mov_b32 m0, %[b_dst]\n"
      "  s_nop 0\n"
      "  global_load_lds_dwordx4 %[gb0], %[bbase]\n"
      "  s_add_u32 m0, %[b_dst], 4096\n"
      "  s_nop 0\n"
      "  global_load_lds_dwordx4 %[gb1], %[bbase]\n"
      "  s_add_u32 m0, %[b_dst], 8192\n"
      "  s_nop 0\n"
      "  global_load_lds_dwordx4 %[gb2], %[bbase]\n"
      "  s_add_u32 m0, %[b_dst], 12288\n"
      "  s_nop 0\n"
      "  global_load_lds_dwordx4 %[gb3], %[bbase]\n"
      ".endm\n"
      ".macro VK_ADV\n"
      "  v_add_u32 %[ga0], %[astep], %[ga0]\n"
      "  v_add_u32 %[ga1], %[astep], %[ga1]\n"
      "  v_add_u32 %[gb0], %[bstep], %[gb0]\n"
      "  v_add_u32 %[gb1], %[bstep], %[gb1]\n"
      "  v_add_u32 %[gb2], %[bstep], %[gb2]\n"
      "  v_add_u32 %[gb3], %[bstep], %[gb3]\n"
      ".endm\n"
      // A rows of k-chunk at address ADDR into a-buffer AQ (8 x 16 B)
      ".macro VK_RDA AQ, ADDR\n"
      "  .irp i, 0,1,2,3\n"
      "  ds_read_b128 v[\\AQ+4*\\i:\\AQ+4*\\i+3], \\ADDR offset:(\\i*64)\n"
      "  ds_read_b128 v[\\AQ+16+4*\\i:\\AQ+16+4*\\i+3], \\ADDR offset:(4096+\\i*64)\n"
      "  .endr\n"
      ".endm\n"
      ".macro VK_RDB KK, BB\n"
      "  .irp g, 0,1,2,3\n"
      "  ds_read_b128 v[\\BB+4*\\g:\\BB+4*\\g+3], %[rd_b] offset:(\\KK*1024+\\g*256)\n"
      "  .endr\n"
      ".endm\n"
      // 128 FMAs of k-step KK (a-buffer AQ, b-buffer BB); a[i] of row i in
      // v[AQ + 4 i + KK % 4] for i < 4 and v[AQ + 16 + 4 (i - 4) + KK % 4]
      ".macro VK_FMA AQ, KK, BB\n"
      "  .irp i, 0,1,2,3,4,5,6,7\n"
      "  .irp j, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15\n"
      "  v_fmac_f32 v[128+16*\\i+((\\j+1)&15)], v[\\AQ+4*\\i+(\\KK&3)], v[\\BB+\\j]\n"
      "  .endr\n"
      "  .endr\n"
      ".endm\n"
      "  .irp r, 0,16,32,48,64,80,96,112\n"
      "  .irp c, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15\n"
      "  v_mov_b32 v[128+\\r+\\c], 0\n"
      "  .endr\n"
      "  .endr\n"
      // prologue: k-tile 0 into buffer 0
      "  VK_DMA\n"
      "  VK_ADV\n"
      "  s_waitcnt vmcnt(0)\n"
      "  s_barrier\n"
      "L_vkd_tile_%=:\n"
      // the next k-tile into the other buffer (freed by the barrier just passed)
      "  s_sub_u32 %[a_dst], %[sa_dst], %[a_dst]\n"
      "  s_sub_u32 %[b_dst], %[sb_dst], %[b_dst]\n"
      "  s_cmp_gt_u32 %[nk], 1\n"
      "  s_cbranch_scc0 L_vkd_noload_%=\n"
      "  VK_DMA\n"
      "  VK_ADV\n"
      "L_vkd_noload_%=:\n"
      "  VK_RDA 32, %[rd_a]\n"
      "  VK_RDB 0, 64\n"
      "  s_waitcnt lgkmcnt(0)\n"
      // k-steps 0..14: the reads of k-step kk + 1 (and of the next A group)
      // go out ahead of k-step kk's FMAs
      "  .irp kk, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14\n"
      "  VK_RDB (\\kk+1), (64+16*((\\kk+1)&1))\n"
      "  .if ((\\kk+1)&3) == 0\n"
      "  v_xor_b32 %[tmp], 16*((\\kk+1)>>2), %[rd_a]\n"
      "  VK_RDA (32+64*(((\\kk+1)>>2)&1)), %[tmp]\n"
      "  .endif\n"
      "  VK_FMA (32+64*((\\kk>>2)&1)), \\kk, (64+16*(\\kk&1))\n"
      "  s_waitcnt lgkmcnt(0)\n"
      "  .endr\n"
      "  VK_FMA 96, 15, 80\n"
      "  s_cmp_gt_u32 %[nk], 1\n"
      "  s_cbranch_scc0 L_vkd_done_%=\n"
      // this wave's loads of the next k-tile have landed; after the barrier
      // every wave's have, and every wave is done reading this buffer
      "  s_waitcnt vmcnt(0)\n"
      "  s_barrier\n"
      "  v_sub_u32 %[rd_a], %[sum_a], %[rd_a]\n"
      "  v_sub_u32 %[rd_b], %[sum_b], %[rd_b]\n"
      "  s_sub_u32 %[nk], %[nk], 1\n"
      "  s_branch L_vkd_tile_%=\n"
      "L_vkd_done_%=:\n"
      "  .irp half, 0,1\n"
      "  .irp i, 0,1,2,3\n"
      "  .irp j, 0,1,2,3,4,5,6,7,8,9,10,11,12,13,14,15\n"
      "  v_mov_b32 v[48+16*\\i+\\j], v[128+16*(4*\\half+\\i)+((\\j+1)&15)]\n"
      "  .endr\n"
      "  .endr\n"
      "  s_nop 4\n"
      "  .irp i, 0,1,2,3\n"
      "  .irp g, 0,1,2,3\n"
      "  .if \\half == 0\n"
      "  global_store_dwordx4 %[c_lo], v[48+16*\\i+4*\\g:51+16*\\i+4*\\g], %[cbase] offset:(\\g*256) sc1\n"
      "  .else\n"
      "  global_store_dwordx4 %[c_hi], v[48+16*\\i+4*\\g:51+16*\\i+4*\\g], %[cbase] offset:(\\g*256) sc1\n"
      "  .endif\n"
      "  .endr\n"
      "  .if \\half == 0\n"
      "  v_add_u32 %[c_lo], %[crow], %[c_lo]\n"
      "  .else\n"
      "  v_add_u32 %[c_hi], %[crow], %[c_hi]\n"
      "  .endif\n"
      "  s_nop 1\n"
      "  .endr\n"
      "  s_waitcnt vmcnt(0)\n"
      "  .endr\n"
      ".purgem VK_DMA\n"
      ".purgem VK_ADV\n"
      ".purgem VK_RDA\n"
      ".purgem VK_RDB\n"
      ".purgem VK_FMA\n"
      : [ga0] "+v"(ga0), [ga1] "+v"(ga1), [gb0] "+v"(gb0), [gb1] "+v"(gb1), [gb2] "+v"(gb2), [gb3] "+v"(gb3),
        [rd_a] "+v"(rd_a), [rd_b] "+v"(rd_b), [c_lo] "+v"(c_lo), [c_hi] "+v"(c_hi), [tmp] "=&v"(tmp),
        [nk] "+s"(nk), [a_dst] "+s"(a_dst), [b_dst] "+s"(b_dst)
      : [abase] "s"(abase), [bbase] "s"(bbase), [cbase] "s"(cbase), [astep] "s"(astep), [bstep] "s"(bstep),
        [crow] "s"(crow), [sum_a] "v"(sum_a), [sum_b] "v"(sum_b), [sa_dst] "s"(sa_dst), [sb_dst] "s"(sb_dst)
      : "memory", "m0", VK_CLOBBER_V32_V255);
}
#pragma clang diagnostic pop

// 64x64 tiles where the 128x256 ones, eight times the work each, need more
// rounds of the CUs for the same work (512^3: 8 tiles on 256 CUs).  Measured
// (us per launch, 2 rounds, one box, against the 128x256 kernels): 512^3
// 43.2 against 131.3, 1024^3 83.5 / 260.0, 1536^3 203.6 / 386.8, 2048^3
// 376.2 / 514.7, 4096 x 1024 x 4096 737.4 / 1024.9; a 128x128 tile (8x8
// outputs per thread) was slower than 64x64 on each of them (2048^3 420.5).
// With one wave per SIMD the small tile waits on its loads and LDS reads:
// 32-deep k-tiles and 4 k-steps per loop body took it further (512^3 35.5,
// 1024^3 69.7, 2048^3 281.8; 48-deep 42.9 / 84.1 / 359.7, 32-deep with 2
// k-steps per body 39.8 / 78.0 / 278.5, fully unrolled 37.5 / 78.8 /
// 605.5).
bool f32_valu_small(size_t m, size_t n, int num_cus) {
  const int64_t c = num_cus > 0 ? num_cus : 1;
  const int64_t big = (int64_t)((m + kTM - 1) / kTM) * (int64_t)((n + kTN - 1) / kTN);
  const int64_t small = (int64_t)((m + 63) / 64) * (int64_t)((n + 63) / 64);
  return 8 * ((big + c - 1) / c) > (small + c - 1) / c && (m + 63) / 64 <= 65535;
}

hipError_t launch_f32(const GemmArgs& a) {
  const float* A = static_cast<const float*>(a.A);
  const float* B = static_cast<const float*>(a.B);
  float* C = static_cast<float*>(a.C);
  if (f32_valu_small(a.m, a.n, a.num_cus)) {
    hipLaunchKernelGGL((f32_valu_kernel<true, 1, 1, 32>), dim3((unsigned)((a.n + 63) / 64), (unsigned)((a.m + 63) / 64)),
                       dim3(256), 0, a.stream, A, B, C, (int64_t)a.m, (int64_t)a.n, (int64_t)a.k);
    return hipGetLastError();
  }
  dim3 grid((unsigned)((a.n + kTN - 1) / kTN), (unsigned)((a.m + kTM - 1) / kTM));
  const bool full = a.m % kTM == 0 && a.n % kTN == 0 && a.k % kBK == 0 &&
                    ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 &&
                    ((uintptr_t)C & 15) == 0 && asm_offsets_fit(a.m, a.n, a.k);
  if (full)
    hipLaunchKernelGGL(f32_valu_asm_kernel, dim3(grid.x * grid.y), dim3(256), 0, a.stream, A, B, C, (int)a.m,
                       (int)a.n, (int)a.k);
  else
    hipLaunchKernelGGL(f32_valu_kernel<true>, grid, dim3(256), 0, a.stream, A, B, C, (int64_t)a.m,
                       (int64_t)a.n, (int64_t)a.k);
  return hipGetLastError();
}

bool f32_shape_ok(size_t m, size_t n, size_t k) {
  (void)n;
  (void)k;
  return (m + kTM - 1) / kTM <= 65535;
}

}  // namespace

void register_f32_valu() {
  KernelEntry e{};
  e.version = 1;
  e.in_dtype = VK_DTYPE_F32;
  e.name = "f32_v1_valu";
  e.caps = make_caps(1, VK_DTYPE_F32, kOutF32, 1, 1, 1, 4, kTM, kTN, kBK, 256,
                     2 * kBK * (kApitch + kTN) * 4, 0, 0);
  e.launch = launch_f32;
  e.workspace = nullptr;
  e.shape_ok = f32_shape_ok;
  register_kernel(e);
}

}  // namespace vk
