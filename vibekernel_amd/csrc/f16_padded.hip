// f16_padded.hip -- fp16 GEMM, version 15: any M, N and K at version 10's
// speed, for shapes whose rows are not multiples of 8 halves.
//
// Versions 7-11 load 16-byte chunks of A and B rows straight into LDS and
// store 16-byte chunks of C, so every row must start on a 16-byte boundary:
// N and K multiples of 8.  Other shapes (a vocabulary of 50,257 columns, K =
// 4095) otherwise fall back to version 1 at a twentieth of the speed.  Here
// the operands go through row-padded copies in the workspace, and version 10
// (any M; N and K multiples of 8) runs on the padded problem:
//  * A (M x K) is copied with row pitch K8 = K rounded up to 8 when K % 8 !=
//    0, the pad columns zero;
//  * B (K x N) is copied with pitch N8 and K8 rows when N % 8 or K % 8 != 0,
//    the pad columns and rows zero (A's pad columns meet B's pad rows: zero
//    times zero, so the padded product equals the product);
//  * C is computed into an M x N8 buffer when N % 8 != 0 and copied back to
//    the caller's M x N rows.
// Each element's sum runs over the same k as version 10's on the padded
// operands (the pad adds exact zeros), so the results are version 10's on
// explicitly padded inputs, bit for bit.  The copies stream each operand
// once more (at 4096 x 50257 x 4096: ~1.6 GB of copy traffic against ~1.7
// TFLOP).  Measured (us per launch, one box): 4096 x 50257 x 4096 1830
// (version 1: 33654), 4096 x 4096 x 4095 132.5 (version 10 at 4096^3:
// 102.9), 1000 x 1001 x 1000 31.6 (version 1: 122.8); element-by-element
// copies took 2393, 160.0 and 32.5.
// Workspace: version 10's own (its split tails and counters, first), then
// A', B' and C' at 256-byte boundaries.
#include "vk_device.hpp"
#include "vk_internal.hpp"

namespace vk {
namespace {

constexpr size_t kWsAlign = 256;
constexpr int kInnerVersion = 10;

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct PadLayout {
  size_t k8, n8;
  bool pad_a, pad_b, pad_c;
  size_t inner;                 // version 10's workspace bytes (at offset 0)
  size_t a_off, b_off, c_off;   // byte offsets of A', B', C' (when used)
  size_t total;
};

PadLayout layout_of(size_t m, size_t n, size_t k, int num_cus, size_t out_bytes) {
  PadLayout L{};
  L.k8 = round_up(k, 8);
  L.n8 = round_up(n, 8);
  L.pad_a = L.k8 != k;
  L.pad_b = L.k8 != k || L.n8 != n;
  L.pad_c = L.n8 != n;
  const KernelEntry* inner = find_registered(kInnerVersion, VK_DTYPE_F16);
  L.inner = inner && inner->workspace ? inner->workspace(m, L.n8, L.k8, num_cus) : 0;
  size_t off = round_up(L.inner, kWsAlign);
  L.a_off = off;
  if (L.pad_a) off = round_up(off + m * L.k8 * 2, kWsAlign);
  L.b_off = off;
  if (L.pad_b) off = round_up(off + L.k8 * L.n8 * 2, kWsAlign);
  L.c_off = off;
  if (L.pad_c) off = round_up(off + m * L.n8 * out_bytes, kWsAlign);
  L.total = off;
  return L;
}

// dst (drows x dpitch elements) <- src (rows x width, row pitch spitch), the
// elements past width or rows zero.  Each thread writes 8 consecutive
// elements of one destination row; adjacent threads take adjacent chunks,
// so every wave instruction touches contiguous bytes.  A chunk that lies
// whole inside its row moves as one 16-byte access on a side whose pitch is
// a multiple of 8 elements of 2 bytes (4 of 4 bytes: two accesses), and
// element by element on the other side (its rows need not be aligned).
template <typename T>
__global__ __launch_bounds__(256) void repitch_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                      int64_t rows, int64_t width, int64_t spitch,
                                                      int64_t drows, int64_t dwidth, int64_t dpitch) {
  constexpr int kPerVec = 16 / sizeof(T);  // elements per 16-byte access
  const bool s_vec = spitch % kPerVec == 0, d_vec = dpitch % kPerVec == 0;
  const int64_t chunks_per_row = (dwidth + 7) / 8;
  const int64_t total = drows * chunks_per_row;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    const int64_t r = c / chunks_per_row, col0 = (c - r * chunks_per_row) * 8;
    T v[8];
    if (r < rows && col0 + 8 <= width && s_vec) {
#pragma unroll
      for (int h = 0; h < 8 / kPerVec; h++) {
        const uint4v x = *reinterpret_cast<const uint4v*>(src + r * spitch + col0 + h * kPerVec);
        __builtin_memcpy(v + h * kPerVec, &x, 16);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = (r < rows && col0 + e < width) ? src[r * spitch + col0 + e] : T(0);
    }
    if (col0 + 8 <= dwidth && d_vec) {
#pragma unroll
      for (int h = 0; h < 8 / kPerVec; h++) {
        uint4v x;
        __builtin_memcpy(&x, v + h * kPerVec, 16);
        *reinterpret_cast<uint4v*>(dst + r * dpitch + col0 + h * kPerVec) = x;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++)
        if (col0 + e < dwidth) dst[r * dpitch + col0 + e] = v[e];
    }
  }
}

template <typename T>
hipError_t repitch(const void* src, void* dst, size_t rows, size_t width, size_t spitch, size_t drows, size_t dwidth,
                   size_t dpitch, hipStream_t s) {
  const int64_t total = (int64_t)drows * (int64_t)((dwidth + 7) / 8);
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 8192 ? blocks : 8192);  // grid-stride beyond 2M chunks
  hipLaunchKernelGGL(repitch_kernel<T>, dim3(grid), dim3(256), 0, s, static_cast<const T*>(src), static_cast<T*>(dst),
                     (int64_t)rows, (int64_t)width, (int64_t)spitch, (int64_t)drows, (int64_t)dwidth, (int64_t)dpitch);
  return hipGetLastError();
}

size_t out_bytes_of(vk_dtype d) { return d == VK_DTYPE_F16 ? 2 : 4; }

hipError_t launch_padded(const GemmArgs& a) {
  const KernelEntry* inner = find_registered(kInnerVersion, VK_DTYPE_F16);
  if (!inner) return hipErrorInvalidValue;
  const PadLayout L = layout_of(a.m, a.n, a.k, a.num_cus, out_bytes_of(a.out_dtype));
  char* ws = static_cast<char*>(a.workspace);
  GemmArgs b = a;
  b.n = L.n8;
  b.k = L.k8;
  hipError_t e = hipSuccess;
  if (L.pad_a) {
    b.A = ws + L.a_off;
    e = repitch<uint16_t>(a.A, ws + L.a_off, a.m, a.k, a.k, a.m, L.k8, L.k8, a.stream);
    if (e != hipSuccess) return e;
  }
  if (L.pad_b) {
    b.B = ws + L.b_off;
    e = repitch<uint16_t>(a.B, ws + L.b_off, a.k, a.n, a.n, L.k8, L.n8, L.n8, a.stream);
    if (e != hipSuccess) return e;
  }
  if (L.pad_c) b.C = ws + L.c_off;
  b.workspace = L.inner ? ws : nullptr;
  b.workspace_bytes = L.inner;
  // The region where version 10 keeps its counters may have held A', B' or
  // C' in an earlier call of this version (whose padded problem needed no
  // counters), so they are always cleared first.
  b.workspace_clean = false;
  e = inner->launch(b);
  if (e != hipSuccess || !L.pad_c) return e;
  return a.out_dtype == VK_DTYPE_F16
             ? repitch<uint16_t>(ws + L.c_off, a.C, a.m, a.n, L.n8, a.m, a.n, a.n, a.stream)
             : repitch<uint32_t>(ws + L.c_off, a.C, a.m, a.n, L.n8, a.m, a.n, a.n, a.stream);
}

// The workspace for an fp16 output; an fp32 output needs the larger C', so
// the entry reports the fp32 size (both fit).
size_t workspace_padded(size_t m, size_t n, size_t k, int num_cus) { return layout_of(m, n, k, num_cus, 4).total; }

// Version 10's limits on the padded problem.
bool shape_ok_padded(size_t m, size_t n, size_t k) {
  const KernelEntry* inner = find_registered(kInnerVersion, VK_DTYPE_F16);
  const size_t n8 = round_up(n, 8), k8 = round_up(k, 8);
  return inner && m >= 1 && n >= 1 && k >= 1 && (!inner->shape_ok || inner->shape_ok(m, n8, k8));
}

}  // namespace

void register_f16_padded() {
  KernelEntry e{};
  e.version = 15;
  e.in_dtype = VK_DTYPE_F16;
  e.name = "f16_v15_padded_v10";
  // 16-byte aligned operands, as version 10's: an operand whose rows need no
  // padding goes to version 10 as it is
  e.caps = make_caps(15, VK_DTYPE_F16, kOutF16 | kOutF32, 1, 1, 1, 16, 256, 256, 64, 512, 160 * 1024, 0, 1);
  e.launch = launch_padded;
  e.workspace = workspace_padded;
  e.shape_ok = shape_ok_padded;
  register_kernel(e);
}

}  // namespace vk
