// vk_gemm.hip -- the C ABI of libvk_gemm.so: version registry, argument
// validation, library-managed workspaces and dispatch.
//
// Stands in for the compile-time dispatch of the reference
// (results/naive_cycle4/include/playground/matmul.hpp:11-23, one template
// specialisation per (dtype, version), picked by -DMATMUL_VERSION in
// results/naive_fable_cycle2/src/CMakeLists.txt:29-50 and :66-70).  Here all
// versions live in one library and are picked at run time by id; an unknown
// id is an error code instead of a configure-time FATAL_ERROR
// (CMakeLists.txt:35-40).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <algorithm>
#include <cstring>
#include <mutex>

#include "vk_device.hpp"
#include "vk_gemm.h"
#include "vk_internal.hpp"

// Workspace of vk_gemm_noalloc: split-K / split-tail partials and their
// arrival counters.  Each device that loads this library holds its own copy
// until the process ends.  In host code this name is only a stand-in for the
// symbol: the device address of a device's copy comes from
// hipGetSymbolAddress (scratch_of below), and only that address is handed to
// kernels.
static __device__ __align__(256) unsigned char scratch[VK_GEMM_SCRATCH_BYTES];

namespace vk {
namespace {

// The registered versions, in a fixed array: a lookup never allocates.
constexpr int kMaxEntries = 48;
struct Registry {
  KernelEntry e[kMaxEntries];
  int n = 0;
  const KernelEntry* begin() const { return e; }
  const KernelEntry* end() const { return e + n; }
};
Registry& registry() {
  static Registry r;
  return r;
}

std::once_flag g_init_once;

void init_registry() {
  std::call_once(g_init_once, [] {
    register_f16_simple();
    register_f16_dma();
    register_f16_skinny();
    register_f16_pingpong();
    register_f16_pp128();
    register_f16_skinny_sk();
    register_f16_skinny_wk();
    register_f16_padded();
    register_f32_valu();
    register_f32_mfma();
  });
}

const KernelEntry* find(int version, vk_dtype in) {
  init_registry();
  for (const auto& e : registry())
    if (e.version == version && e.in_dtype == in) return &e;
  return nullptr;
}

size_t dtype_size(vk_dtype d) { return d == VK_DTYPE_F16 ? 2 : 4; }

}  // namespace

const KernelEntry* find_registered(int version, vk_dtype in) { return find(version, in); }

namespace {

struct DeviceState {
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int ws_version = 0;  // version whose launch used the library workspace last (0: none)
  int num_cus = 0;
  void* scratch = nullptr;  // this device's copy of `scratch` (vk_gemm_noalloc)
};
// One entry per device id, fixed in size: looking a device up never
// allocates (host or device memory).
constexpr int kMaxDevices = 64;
std::mutex g_dev_mutex;
DeviceState g_dev[kMaxDevices];

hipError_t device_state(int dev, DeviceState** out) {
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_dev_mutex);
  DeviceState& s = g_dev[dev];
  if (s.num_cus == 0) {
    int cus = 0;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    s.num_cus = cus;
  }
  *out = &s;
  return hipSuccess;
}

// Device address of this device's copy of `scratch`, looked up once per
// device with that device current.
hipError_t scratch_of(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_dev_mutex);
  DeviceState& s = g_dev[dev];
  if (!s.scratch) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    s.scratch = p;
  }
  *out = s.scratch;
  return hipSuccess;
}

// C := 0 for k == 0 (beta = 0 and an empty sum).  A kernel, not
// hipMemsetAsync, so the call stays safe inside stream capture.
__global__ void zero_fill_kernel(uint32_t* __restrict__ p, size_t words) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < words; i += stride) p[i] = 0u;
}
__global__ void zero_fill_u16_kernel(uint16_t* __restrict__ p, size_t count) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < count; i += stride) p[i] = 0u;
}

hipError_t zero_output(void* C, size_t count, vk_dtype out, hipStream_t s) {
  const unsigned blocks = 1024;
  if (out == VK_DTYPE_F32 || (count % 2 == 0 && ((uintptr_t)C & 3u) == 0)) {
    const size_t words = out == VK_DTYPE_F32 ? count : count / 2;
    hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, s, (uint32_t*)C, words);
  } else {
    hipLaunchKernelGGL(zero_fill_u16_kernel, dim3(blocks), dim3(256), 0, s, (uint16_t*)C, count);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t zero_words(void* p, size_t words, hipStream_t s) {
  const unsigned blocks = (unsigned)std::min<size_t>(1024, (words + 255) / 256);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks ? blocks : 1), dim3(256), 0, s, (uint32_t*)p, words);
  return hipGetLastError();
}

namespace {

int validate(const KernelEntry* e, vk_dtype out, size_t m, size_t n, size_t k, const void* A,
             const void* B, const void* C) {
  if (!e) return VK_ERR_VERSION;
  if (out != VK_DTYPE_F16 && out != VK_DTYPE_F32) return VK_ERR_DTYPE;
  if (!(e->caps.out_dtype_mask & (1 << out))) return VK_ERR_DTYPE;
  const size_t lim = 0x7fffffffu;
  if (m > lim || n > lim || k > lim) return VK_ERR_RANGE;
  if (m == 0 || n == 0) return VK_OK;  // nothing to write
  if (!C) return VK_ERR_NULL;
  if (k == 0) return VK_OK;            // C := 0, A and B unused
  if (!A || !B) return VK_ERR_NULL;
  const vk_caps& c = e->caps;
  if (m % c.div_m || n % c.div_n || k % c.div_k) return VK_ERR_SHAPE;
  if (m > c.max_m) return VK_ERR_SHAPE;
  if (e->shape_ok && !e->shape_ok(m, n, k)) return VK_ERR_SHAPE;
  const uintptr_t al = c.align_bytes ? c.align_bytes : 1;
  if (((uintptr_t)A % al) || ((uintptr_t)B % al) || ((uintptr_t)C % al)) return VK_ERR_ALIGN;
  return VK_OK;
}

int run(int version, vk_dtype in, vk_dtype out, size_t m, size_t n, size_t k, const void* A,
        const void* B, void* C, void* ws, size_t ws_bytes, bool library_ws, void* stream) {
  const KernelEntry* e = find(version, in);
  int st = validate(e, out, m, n, k, A, B, C);
  if (st != VK_OK) return st;
  if (m == 0 || n == 0) return VK_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (k == 0) return zero_output(C, m * n, out, s) == hipSuccess ? VK_OK : VK_ERR_HIP;

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return VK_ERR_HIP;
  DeviceState* ds = nullptr;
  if (device_state(dev, &ds) != hipSuccess) return VK_ERR_HIP;

  const size_t need = e->workspace ? e->workspace(m, n, k, ds->num_cus) : 0;
  bool ws_clean = false;
  bool owns_ws = false;  // this call uses the library workspace
  if (need > 0) {
    if (library_ws) {
      // A graph captured now would keep this workspace's address, which a
      // later call may free and reallocate, and would replay the counter
      // state decided here: under capture the library workspace is refused,
      // and vk_gemm_ws (caller workspace) is the capture-safe form.
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(s, &cs) != hipSuccess) return VK_ERR_HIP;
      if (cs != hipStreamCaptureStatusNone) return VK_ERR_WORKSPACE;
      std::lock_guard<std::mutex> lk(g_dev_mutex);
      if (ds->ws_bytes < need) {
        if (ds->ws) {
          if (hipFree(ds->ws) != hipSuccess) return VK_ERR_HIP;  // synchronises the device
          ds->ws = nullptr;
          ds->ws_bytes = 0;
        }
        ds->ws_version = 0;
        if (hipMalloc(&ds->ws, need) != hipSuccess) return VK_ERR_HIP;
        ds->ws_bytes = need;
      }
      ws = ds->ws;
      ws_bytes = ds->ws_bytes;
      ws_clean = ds->ws_version == version;
      // Until this launch is known to have been enqueued, the counters count
      // as unknown: a failed launch must not leave the next call skipping the
      // clear.
      ds->ws_version = 0;
      owns_ws = true;
    } else if (!ws || ws_bytes < need) {
      return VK_ERR_WORKSPACE;
    }
  }

  GemmArgs a;
  a.m = m;
  a.n = n;
  a.k = k;
  a.A = A;
  a.B = B;
  a.C = C;
  a.out_dtype = out;
  a.workspace = ws;
  a.workspace_bytes = ws_bytes;
  a.workspace_clean = ws_clean;
  a.stream = s;
  a.device = dev;
  a.num_cus = ds->num_cus;
  if (e->launch(a) != hipSuccess) return VK_ERR_HIP;
  if (owns_ws) {
    // The kernels of a version leave the counters they use at zero, so the
    // next call of the same version may skip clearing them.
    std::lock_guard<std::mutex> lk(g_dev_mutex);
    if (ds->ws == ws) ds->ws_version = version;
  }
  return VK_OK;
}

}  // namespace

void register_kernel(const KernelEntry& e) {
  Registry& r = registry();
  if (r.n < kMaxEntries) r.e[r.n++] = e;
}

}  // namespace vk

extern "C" {

int vk_gemm(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n, size_t k,
            const void* A, const void* B, void* C, void* stream) {
  return vk::run(version, in_dtype, out_dtype, m, n, k, A, B, C, nullptr, 0, true, stream);
}

int vk_gemm_ws(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n, size_t k,
               const void* A, const void* B, void* C, void* workspace, size_t workspace_bytes,
               void* stream) {
  return vk::run(version, in_dtype, out_dtype, m, n, k, A, B, C, workspace, workspace_bytes, false,
                 stream);
}

int vk_gemm_noalloc(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n, size_t k,
                    const void* A, const void* B, void* C, void* stream) {
  const int st = vk::validate(vk::find(version, in_dtype), out_dtype, m, n, k, A, B, C);
  if (st != VK_OK || m == 0 || n == 0 || k == 0)
    return st != VK_OK ? st : vk::run(version, in_dtype, out_dtype, m, n, k, A, B, C, nullptr, 0, false, stream);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return VK_ERR_HIP;
  void* sp = nullptr;
  if (vk::scratch_of(dev, &sp) != hipSuccess) return VK_ERR_HIP;
  // A caller workspace of VK_GEMM_SCRATCH_BYTES: a plan that needs more is
  // refused with VK_ERR_WORKSPACE, and the counters are cleared by a kernel
  // in every call (the scratch keeps whatever the last call left).
  return vk::run(version, in_dtype, out_dtype, m, n, k, A, B, C, sp, VK_GEMM_SCRATCH_BYTES, false, stream);
}

size_t vk_gemm_workspace_bytes(int version, vk_dtype in_dtype, size_t m, size_t n, size_t k) {
  const vk::KernelEntry* e = vk::find(version, in_dtype);
  if (!e || !e->workspace) return 0;
  // The split-tail schedule depends on the current device's compute-unit count;
  // with no device to ask, an MI355X (256 CUs) is assumed.
  int cus = 256, dev = 0;
  vk::DeviceState* ds = nullptr;
  if (hipGetDevice(&dev) == hipSuccess && vk::device_state(dev, &ds) == hipSuccess) cus = ds->num_cus;
  return e->workspace(m, n, k, cus);
}

const char* vk_gemm_name(int version, vk_dtype in_dtype) {
  const vk::KernelEntry* e = vk::find(version, in_dtype);
  return e ? e->name : nullptr;
}

int vk_gemm_query(int version, vk_dtype in_dtype, vk_caps* caps) {
  const vk::KernelEntry* e = vk::find(version, in_dtype);
  if (!e) return VK_ERR_VERSION;
  if (caps) *caps = e->caps;
  return VK_OK;
}

int vk_gemm_list(vk_dtype in_dtype, int* out, int max_count) {
  vk::init_registry();
  int n = 0;
  for (const auto& e : vk::registry()) {
    if (e.in_dtype != in_dtype) continue;
    if (out && n < max_count) out[n] = e.version;
    n++;
  }
  return n;
}

int vk_gemm_check(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n, size_t k,
                  const void* A, const void* B, const void* C) {
  return vk::validate(vk::find(version, in_dtype), out_dtype, m, n, k, A, B, C);
}

int vk_gemm_release(void) {
  std::lock_guard<std::mutex> lk(vk::g_dev_mutex);
  int st = VK_OK;
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return VK_ERR_HIP;
  for (int d = 0; d < vk::kMaxDevices; d++) {
    if (!vk::g_dev[d].ws) continue;
    if (hipSetDevice(d) != hipSuccess || hipFree(vk::g_dev[d].ws) != hipSuccess) st = VK_ERR_HIP;
    vk::g_dev[d].ws = nullptr;
    vk::g_dev[d].ws_bytes = 0;
    vk::g_dev[d].ws_version = 0;
  }
  if (hipSetDevice(cur) != hipSuccess) st = VK_ERR_HIP;
  return st;
}

const char* vk_status_string(int status) {
  switch (status) {
    case VK_OK: return "ok";
    case VK_ERR_VERSION: return "unknown version for this input dtype";
    case VK_ERR_DTYPE: return "unsupported input/output dtype pair";
    case VK_ERR_SHAPE: return "shape not supported by this version";
    case VK_ERR_ALIGN: return "operand pointer misaligned for this version";
    case VK_ERR_NULL: return "null operand with a non-empty shape";
    case VK_ERR_WORKSPACE: return "workspace too small";
    case VK_ERR_HIP: return "HIP runtime error";
    case VK_ERR_RANGE: return "dimension out of range";
    default: return "unknown status";
  }
}

int vk_gemm_abi_version(void) { return VK_GEMM_ABI_VERSION; }

}  // extern "C"
