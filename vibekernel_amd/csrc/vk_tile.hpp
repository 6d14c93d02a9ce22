// vk_tile.hpp -- pieces shared by the 256x256-tile fp16 GEMM kernels: the LDS
// bank swizzles of the A and B k-tiles, the workgroup -> tile order and the
// one-time dynamic-LDS attribute.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

namespace vk {

// A rows are BK halves = BK/8 chunks of 16 B.  Swizzle of the chunk index as a
// function of the row, chosen so the 16-byte A-fragment reads of consecutive
// rows hit distinct banks.  Depends on row bits 0..3 only.
template <int BK>
__host__ __device__ constexpr int swz_a(int row) {
  if constexpr (BK == 64) {
    return (row & 7) ^ ((row >> 3) & 1);
  } else {  // BK == 32: 4 chunks per row
    return ((row >> 1) & 3) ^ ((row >> 2) & 3);
  }
}

// B rows are 256 halves = 32 chunks.  The transpose reads touch 4 consecutive
// k rows x 2 or 4 neighbouring chunks per 16 or 32 lanes; XOR by v[k % 4]
// spreads them over distinct banks.
__host__ __device__ constexpr int swz_b(int krow) {
  return (krow & 3) == 0 ? 0 : (krow & 3) == 1 ? 6 : (krow & 3) == 2 ? 12 : 10;
}

// Tile order: XCD-aware remap plus a grouped raster of GM tile-rows.
// Workgroups are dealt round-robin over the 8 XCDs, so workgroup `bid` runs on
// XCD bid % 8; the remap gives each XCD a contiguous range of the raster, and
// the raster walks GM tile-rows at a time so neighbouring tiles share panels
// of A and B in that XCD's L2.
// raster_tile: position `cid` of the grouped raster -> tile (tm, tn).
__host__ __device__ __forceinline__ void raster_tile(int cid, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int GM = 4;
  const int group = GM * tiles_n;
  const int g = cid / group;
  const int first_m = g * GM;
  const int gm = tiles_m - first_m < GM ? tiles_m - first_m : GM;
  const int r = cid - g * group;
  tm = first_m + r % gm;
  tn = r / gm;
}

// Raster position of workgroup `bid` of `total`: XCD x (= bid % 8) gets the
// contiguous positions [x q + min(x, r), (x + 1) q + min(x + 1, r)) in launch
// order, q = total / 8 and r = total % 8 (the workgroups with bid % 8 == x
// number q + (x < r)).  With total % 8 != 0 the identity (each XCD a
// scattered eighth of the raster) measured on MI355X (v11, 172 tiles of
// 128 x 128 at 136 x 11008 x 4096) 36.4 us per launch against 31.0 for the
// split-K skinny kernel: neighbouring tiles on different XCDs read their
// shared panels of B once per XCD.
__host__ __device__ __forceinline__ int xcd_remap(int bid, int total) {
  const int q = total >> 3, r = total & 7, x = bid & 7;
  return x * q + (x < r ? x : r) + (bid >> 3);
}

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  raster_tile(xcd_remap(bid, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
}

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) once per kernel instance
// and device (a bit per device id).
template <typename KFn>
hipError_t ensure_lds_attr(KFn kfn, int bytes, int device, std::atomic<uint64_t>& done) {
  const uint64_t bit = device < 64 ? (1ull << device) : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kfn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

}  // namespace vk
