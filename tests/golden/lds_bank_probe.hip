// lds_bank_probe.hip -- measures how gfx950 serves LDS accesses, for the
// bank model of tests/test_lds_banks.py (fixture lds_bank_probe_gfx950.json).
//
// One dispatch per line of a pattern file (make_lds_bank_fixture.py writes
// it): one wave, a per-lane LDS byte offset table, an active-lane mask and
// an op (0 ds_read_b128, 1 ds_read_b64, 2 ds_read_b64_tr_b16, 3
// ds_write_b128, 4 ds_write_b64); each dispatch issues 16 instances of the
// op, so SQ_LDS_BANK_CONFLICT / 16 is the conflict cycles per instruction.
// Every offset is checked to be below 65536 - 16 on the host and masked to
// 16 (or 8) bytes on the device; reads of uninitialised LDS are harmless.
//
//   hipcc --offload-arch=gfx950 -O3 lds_bank_probe.hip -o lds_bank_probe
//   python3 make_lds_bank_fixture.py patterns
//   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS --output-format csv \
//       -d <dir> -o p -- ./lds_bank_probe lds_bank_patterns.txt
//   python3 make_lds_bank_fixture.py fixture <dir>/p_counter_collection.csv
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstdint>
#include <vector>
#include <string>

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(64) void probe(const uint32_t* __restrict__ offs, unsigned long long mask, int op,
                                            uint32_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x;
  const uint32_t base = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)lds);
  const uint32_t a = base + (offs[lane] & 0xfff0u) + (op == 1 || op == 2 || op == 4 ? (offs[lane] & 8u) : 0u);
  uint32_t acc = 0;
  if ((mask >> lane) & 1ull) {
    if (op == 0) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        u4 v;
        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a));
        acc += v.x;
      }
    } else if (op == 1) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        u2 v;
        asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a));
        acc += v.x;
      }
    } else if (op == 2) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        u2 v;
        asm volatile("ds_read_b64_tr_b16 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a));
        acc += v.x;
      }
    } else if (op == 3) {
      u4 v = {1u, 2u, 3u, 4u};
#pragma unroll
      for (int i = 0; i < 16; i++) asm volatile("ds_write_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(a), "v"(v));
    } else {
      u2 v = {1u, 2u};
#pragma unroll
      for (int i = 0; i < 16; i++) asm volatile("ds_write_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(a), "v"(v));
    }
  }
  out[lane] = acc;
}

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { std::printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); std::exit(1); } } while (0)

int main(int argc, char** argv) {
  // manifest lines: op mask_hex off0 .. off63
  const char* path = argc > 1 ? argv[1] : "lds_bank_patterns.txt";
  FILE* f = std::fopen(path, "r");
  if (!f) { std::printf("no %s\n", path); return 1; }
  std::vector<std::vector<uint32_t>> offs;
  std::vector<unsigned long long> masks;
  std::vector<int> ops;
  int op;
  unsigned long long mask;
  while (std::fscanf(f, "%d %llx", &op, &mask) == 2) {
    std::vector<uint32_t> o(64);
    for (int i = 0; i < 64; i++) {
      if (std::fscanf(f, "%u", &o[i]) != 1) { std::printf("bad manifest\n"); return 1; }
      if (o[i] > 65536 - 16) { std::printf("offset out of range\n"); return 1; }
    }
    offs.push_back(o); masks.push_back(mask); ops.push_back(op);
  }
  std::fclose(f);
  uint32_t *d_off, *d_out;
  CK(hipMalloc(&d_off, 64 * 4 * offs.size()));
  CK(hipMalloc(&d_out, 64 * 4));
  for (size_t i = 0; i < offs.size(); i++) CK(hipMemcpy(d_off + 64 * i, offs[i].data(), 256, hipMemcpyHostToDevice));
  CK(hipFuncSetAttribute((const void*)probe, hipFuncAttributeMaxDynamicSharedMemorySize, 65536));
  for (size_t i = 0; i < offs.size(); i++) {
    hipLaunchKernelGGL(probe, dim3(1), dim3(64), 65536, 0, d_off + 64 * i, masks[i], ops[i], d_out);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
  }
  std::printf("ran %zu configs\n", offs.size());
  CK(hipFree(d_off));
  CK(hipFree(d_out));
  return 0;
}
