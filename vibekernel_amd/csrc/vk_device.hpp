// vk_device.hpp -- gfx950 device helpers shared by the GEMM kernels.
//
// Operand layouts of the CDNA4 MFMAs used here (lane l of a 64-wide wave;
// measured on MI355X with an in-bounds probe before any kernel used them):
//
//   v_mfma_f32_32x32x16_f16  D(32x32) += A(32x16) . B(16x32)
//     A: lane l holds A[l % 32][8 * (l / 32) + e], e = 0..7 (8 halves)
//     B: lane l holds B[8 * (l / 32) + e][l % 32]
//     D: lane l, register r holds D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32]
//
//   v_mfma_f32_16x16x32_f16  D(16x16) += A(16x32) . B(32x16)
//     A: lane l holds A[l % 16][8 * (l / 16) + e]
//     B: lane l holds B[8 * (l / 16) + e][l % 16]
//     D: lane l, register r holds D[4 * (l / 16) + r][l % 16]
//
//   ds_read_b64_tr_b16 (LDS transpose read): each lane names 8 bytes (4
//   halves); inside every group of 16 lanes, lane i receives half (i % 4) of
//   the 8 bytes named by lane 4 * j + i / 4, for j = 0..3.  Read as a matrix:
//   the 16 lanes' 64 halves form 4 rows of 16 (row j = lanes 4j..4j+3) and
//   lane i receives column i.
//
//   global_load_lds_dwordx4 (direct-to-LDS): lane l's 16 bytes land at
//   LDS base + 16 * l; the base comes from M0 and is uniform per wave.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>
#include <utility>

namespace vk {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t uint4v __attribute__((ext_vector_type(4)));

// Word 3 of a raw (unstrided, byte-addressed) buffer resource on gfx9-family
// GPUs: data format 32-bit, everything else zero.
constexpr int kBufferWord3 = 0x00020000;

#define VK_LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

__device__ __forceinline__ float16v mfma32x32x16(const half8& a, const half8& b, const float16v& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4v mfma16x16x32(const half8& a, const half8& b, const float4v& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 4 halves, transposed across each 16-lane group (see header comment).
__device__ __forceinline__ half4 lds_read_tr16(const half_t* lds_addr) {
  short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(VK_LDS_PTR(short4v, lds_addr));
  return __builtin_bit_cast(half4, r);
}

// Same, from a 32-bit LDS byte address (no generic-pointer round trip).
__device__ __forceinline__ half4 lds_read_tr16_at(uint32_t lds_byte_addr) {
  short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4v*)(uintptr_t)lds_byte_addr);
  return __builtin_bit_cast(half4, r);
}

// 16 bytes from global straight into LDS at lds_wave_base + 16 * lane.
__device__ __forceinline__ void global_load_lds16(const void* gptr, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(gptr, VK_LDS_PTR(void, lds_wave_base), 16, 0, 0);
}

// 32-bit LDS address of a pointer into workgroup memory.
__device__ __forceinline__ uint32_t lds_addr32(const void* p) {
  return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const char*)p);
}

__device__ __forceinline__ void lds_write8(uint32_t addr, half4 v) {
  *reinterpret_cast<__attribute__((address_space(3))) half4*>(addr) = v;
}
__device__ __forceinline__ void lds_write16(uint32_t addr, float4v v) {
  *reinterpret_cast<__attribute__((address_space(3))) float4v*>(addr) = v;
}
__device__ __forceinline__ uint4v lds_read16(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) uint4v*>(addr);
}
__device__ __forceinline__ half8 lds_read_h8(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) half8*>(addr);
}

// LDS reads at base + OFF with OFF in the instruction's 16-bit offset field
// (inline asm: the compiler otherwise materialises base + OFF with a VALU add
// per read).  The "memory" clobber-free asm is ordered by its data use only;
// callers wait with lgkmcnt (or a barrier) before the results are used.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int OFF>
__device__ __forceinline__ half8 lds_read_h8_off(uint32_t base) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  half8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(base), "n"(OFF));
  return v;
}
template <int OFF>
__device__ __forceinline__ half4 lds_read_tr16_off(uint32_t base) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  half4 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(base), "n"(OFF));
  return v;
}
#pragma clang diagnostic pop

// Calls f(std::integral_constant<int, I>) for I = 0 .. N-1 (compile-time loop
// indices for template arguments such as immediate offsets).
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// s_waitcnt with only a vmcnt limit (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// vmcnt(0) that is also a compiler barrier for memory accesses: stores
// before it stay before it, and a counter update after it stays after it.
// (The s_waitcnt builtin is modelled as touching no memory.)  For hand-offs
// through global memory: the data stores must be complete before the flag.
__device__ __forceinline__ void wait_vmcnt0_ordered() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Cross-workgroup partial sums are read and written through a raw buffer
// resource with the sc1 cache policy (the encoding of agent-scope atomic loads
// and stores): such stores do not stay dirty in the writing XCD's L2, and such
// loads are not served stale from the reading XCD's L2.  16 bytes per lane, so
// one wave instruction moves a coalesced 1 KB row.
constexpr int kCpolAgent = 16;  // sc1
__device__ __forceinline__ void store_partial(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float4v v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uint4v, v), r, voff, soff, kCpolAgent);
}
__device__ __forceinline__ float4v load_partial(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kCpolAgent));
}

// Output stores of the 256x256-tile kernels: 16 bytes per lane through a raw
// buffer resource at the wave's block (offsets below 2^32), with sc1 (agent
// scope), so the lines are written through the XCD's L2 as they are stored
// instead of staying dirty there until the end-of-kernel write-back.
// Measured on MI355X (3 interleaved rounds per box, us per launch): version
// 7 at 4096^3 92.36 against 93.38 with plain global stores (another box:
// 94.9 against 96.3; the same buffer store with the default policy 96.3, nt
// 95.2, sc0 sc1 95.0); no change at 4096 x 11008 x 4096, 4096 x 4096 x
// 11008, 8192^3 or with fp32 output; version 11 -0.5 to -1.3 % on its whole
// tiles (2048 x 2048 x 4096, 1024 / 512 x 4096 x 4096, 256 x 8192 x 8192).
// The edge paths keep plain stores: at 1000^3 the sc1 form was 4 % slower.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rsrc(void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, -1, kBufferWord3);
}
__device__ __forceinline__ void store_out16(__amdgpu_buffer_rsrc_t r, uint32_t voff, const uint4v& v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, kCpolAgent);
}

// Workgroup barrier for LDS producer/consumer hand-off only: waits for this
// wave's LDS reads (lgkmcnt) but, unlike __syncthreads(), not for its
// in-flight global->LDS prefetches (vmcnt), which are waited for explicitly.
// The "memory" clobbers keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Direct-to-LDS load: lane l's 16 bytes at gbase + voff land at LDS address
// lds_dst + 16 * l (lds_dst and gbase are wave-uniform).  Issued as inline
// asm so the compiler does not track it: it would otherwise treat every later
// LDS read as aliasing the pending load and wait for all of them (vmcnt(0)),
// which would drain a prefetch ring.  Completion is awaited explicitly with
// wait_vmcnt().  Nothing else in these kernels uses M0.  An SALU write of M0
// followed by an LDS-DMA load needs one wait state on the GFX9 family (the
// s_nop 0); the compiler inserts it for its own code, not inside inline asm.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* gbase, uint32_t voff, uint32_t lds_dst) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds_dst), "v"(voff), "s"(gbase)
               : "m0");
}
// The same through a buffer resource, lane l's 16 bytes at soff + voff of
// it: a lane whose bytes are not below the resource's size reads zeros and
// touches no memory (the wave-uniform soff counts in that test: measured on
// MI355X), which is how a lane outside a matrix is masked.
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff,
                                          uint32_t lds_dst) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_dst), "v"(voff), "s"(rsrc), "s"(soff)
               : "m0");
}
#pragma clang diagnostic pop

// An inline-asm operand in an AGPR marks the kernel as using AGPRs, and the
// compiler then selects the AGPR form of the MFMAs: accumulators live in the
// AccVGPR file while LDS fragment loads land in the ordinary VGPRs.  Without it
// the compiler keeps both in VGPRs (when they fit in 256).
__device__ __forceinline__ void prefer_agpr_accumulators() {
  float z = 0.0f;
  asm volatile("; accumulators in AGPRs %0" ::"a"(z));
}

template <typename OutT>
__device__ __forceinline__ OutT convert_out(float v);
template <>
__device__ __forceinline__ half_t convert_out<half_t>(float v) {
  return (half_t)v;  // v_cvt_f16_f32: round to nearest even (default mode)
}
template <>
__device__ __forceinline__ float convert_out<float>(float v) {
  return v;
}

}  // namespace vk
