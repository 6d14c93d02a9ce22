// The host side of libvk_gemm.so's C ABI under AddressSanitizer and
// UndefinedBehaviorSanitizer (tests/native/Makefile, target san; the HIP
// sources are compiled for the host only, so nothing here can launch a
// kernel): the registry, vk_gemm_query / vk_gemm_name / vk_gemm_list,
// vk_gemm_check over ragged, empty, huge and misaligned calls for every
// version, vk_gemm_workspace_bytes (the split-K and split-tail plans) over a
// sweep of shapes, and the launching entry points with calls that validation
// rejects before any device work.  Prints "ok <cases>".
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "vk_gemm.h"

static int fails = 0;
static void expect(bool ok, const char* what, int v, size_t m, size_t n, size_t k) {
  if (!ok) {
    std::printf("FAIL %s v%d %zux%zux%zu\n", what, v, m, n, k);
    fails++;
  }
}

int main() {
  int cases = 0;
  const vk_dtype dts[2] = {VK_DTYPE_F16, VK_DTYPE_F32};
  const size_t dims[] = {0, 1, 7, 8, 15, 16, 17, 63, 64, 65, 255, 256, 257, 1000, 4096, 4097, 11008};
  alignas(4096) static char buf[4096];
  for (vk_dtype in : dts) {
    int ids[64];
    const int nv = vk_gemm_list(in, ids, 64);
    expect(nv > 0 && nv <= 64, "list", 0, 0, 0, 0);
    for (int iv = 0; iv < nv; iv++) {
      const int v = ids[iv];
      vk_caps c;
      expect(vk_gemm_query(v, in, &c) == VK_OK && c.version == v, "query", v, 0, 0, 0);
      expect(vk_gemm_name(v, in) != nullptr && std::strlen(vk_gemm_name(v, in)) > 0, "name", v, 0, 0, 0);
      for (size_t m : dims)
        for (size_t n : dims)
          for (size_t k : dims) {
            for (vk_dtype out : dts) {
              const int st = vk_gemm_check(v, in, out, m, n, k, buf, buf, buf);
              expect(st <= 0 && st >= -8, "check range", v, m, n, k);
              if (st == VK_OK && m && n && k) {
                // a pointer off the version's alignment is refused when it needs one
                if (c.align_bytes > 1)
                  expect(vk_gemm_check(v, in, out, m, n, k, buf + 1, buf, buf) == VK_ERR_ALIGN, "align", v, m, n,
                         k);
                expect(vk_gemm_check(v, in, out, m, n, k, nullptr, buf, buf) == VK_ERR_NULL, "null A", v, m, n, k);
              }
              cases++;
            }
            // every plan of an accepted call fits the no-allocation scratch,
            // but fp16 version 15's, whose workspace holds row-padded copies
            // of the operands (vk_gemm_noalloc refuses those beyond it)
            const size_t ws = vk_gemm_workspace_bytes(v, in, m, n, k);
            if (k > 0 && !(in == VK_DTYPE_F16 && v == 15) && vk_gemm_check(v, in, in, m, n, k, buf, buf, buf) == VK_OK)
              expect(ws <= VK_GEMM_SCRATCH_BYTES, "workspace within the scratch", v, m, n, k);
          }
      // dimensions past 2^31 - 1 and an unknown output dtype
      expect(vk_gemm_check(v, in, in, (size_t)1 << 31, 256, 256, buf, buf, buf) == VK_ERR_RANGE, "range", v, 0, 0, 0);
      expect(vk_gemm_check(v, in, (vk_dtype)7, 256, 256, 64, buf, buf, buf) == VK_ERR_DTYPE, "dtype", v, 0, 0, 0);
      // the launching entry points refuse invalid calls before touching a device
      expect(vk_gemm(v, in, in, (size_t)1 << 31, 256, 256, buf, buf, buf, nullptr) == VK_ERR_RANGE, "gemm", v, 0, 0,
             0);
      expect(vk_gemm_noalloc(v, in, in, (size_t)1 << 31, 256, 256, buf, buf, buf, nullptr) == VK_ERR_RANGE,
             "noalloc", v, 0, 0, 0);
      expect(vk_gemm_ws(v, in, in, 256, 256, 64, nullptr, buf, buf, nullptr, 0, nullptr) == VK_ERR_NULL, "ws", v, 0,
             0, 0);
      cases += 5;
    }
    expect(vk_gemm_query(12345, in, nullptr) == VK_ERR_VERSION, "unknown version", 12345, 0, 0, 0);
  }
  for (int s = 1; s >= -9; s--) expect(vk_status_string(s) != nullptr, "status string", s, 0, 0, 0);
  expect(vk_gemm_abi_version() == VK_GEMM_ABI_VERSION, "abi version", 0, 0, 0, 0);
  if (fails) return 1;
  std::printf("ok %d\n", cases);
  return 0;
}
