// vk_internal.hpp -- host-side registry shared by the kernel translation units
// of libvk_gemm.so.  Each kernel file registers its versions; vk_gemm.hip owns
// validation, workspaces and dispatch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "vk_gemm.h"

namespace vk {

// Everything a launcher needs.  Shapes are already validated against caps.
struct GemmArgs {
  size_t m, n, k;
  const void* A;
  const void* B;
  void* C;
  vk_dtype out_dtype;
  void* workspace;
  size_t workspace_bytes;
  // True when the workspace is library-managed and was left by the previous
  // call of this same version (counters it keeps are already reset); false
  // for a caller workspace or after (re)allocation or use by another version.
  bool workspace_clean;
  hipStream_t stream;
  int device;
  int num_cus;
};

using LaunchFn = hipError_t (*)(const GemmArgs&);
// Workspace bytes for one call; num_cus is the device's compute-unit count.
using WorkspaceFn = size_t (*)(size_t m, size_t n, size_t k, int num_cus);
// Optional extra shape rule beyond the divisibility in caps (nullptr = none).
using ShapeFn = bool (*)(size_t m, size_t n, size_t k);

struct KernelEntry {
  int version;
  vk_dtype in_dtype;
  const char* name;
  vk_caps caps;
  LaunchFn launch;
  WorkspaceFn workspace;  // nullptr: no workspace
  ShapeFn shape_ok;       // nullptr: caps only
};

void register_kernel(const KernelEntry& e);

// The registered entry of a version (nullptr if none); for launchers that
// run another version on a transformed problem.
const KernelEntry* find_registered(int version, vk_dtype in);

// Fill `words` 32-bit words with zero on `stream` (a kernel, not
// hipMemsetAsync, so it may be captured into a graph).
hipError_t zero_words(void* p, size_t words, hipStream_t stream);

// Per-translation-unit registration hooks (called once from vk_gemm.hip).
void register_f16_simple();
void register_f16_dma();
void register_f16_skinny();
void register_f16_pingpong();
void register_f16_pp128();
void register_f16_skinny_sk();
void register_f16_skinny_wk();
void register_f16_padded();
void register_f32_valu();
void register_f32_mfma();

inline vk_caps make_caps(int version, vk_dtype in, int out_mask, uint32_t dm, uint32_t dn,
                         uint32_t dk, uint32_t align, uint32_t tm, uint32_t tn, uint32_t tk,
                         uint32_t threads, uint32_t lds, int tier, int uses_ws,
                         uint64_t max_m = ~0ull) {
  vk_caps c{};
  c.version = version;
  c.in_dtype = in;
  c.out_dtype_mask = out_mask;
  c.div_m = dm;
  c.div_n = dn;
  c.div_k = dk;
  c.max_m = max_m;
  c.align_bytes = align;
  c.tile_m = tm;
  c.tile_n = tn;
  c.tile_k = tk;
  c.threads = threads;
  c.lds_bytes = lds;
  c.tolerance_tier = tier;
  c.uses_workspace = uses_ws;
  return c;
}

constexpr int kOutF16 = 1 << VK_DTYPE_F16;
constexpr int kOutF32 = 1 << VK_DTYPE_F32;

}  // namespace vk
