// matmul_gpu.cpp -- the specialisation for the binary's GPU version.
// Reference pattern: a src/matmul_f16/matmul_f16_vN_*.cu file defining
// PLAYGROUND_MATMUL_DEC(float16_t, N, ...) with a host wrapper that launches
// the kernel on the default stream (e.g. results/ralph_loop_fable/src/
// matmul_f16/matmul_f16_v42_shfl2.cu:494-529).  Here every version lives in
// libvk_gemm.so and this wrapper forwards to its C ABI on the null stream.
// The reference has no error channel; an error code here is printed and
// ends the run.
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "playground/matmul.hpp"
#include "playground/system.hpp"
#include "vk_gemm.h"

namespace playground {

#if MATMUL_VERSION != 0
PLAYGROUND_MATMUL_DEC(params::DataType, params::MatmulVersion, m, n, k, A, B, C) {
    constexpr vk_dtype dt = std::is_same_v<params::DataType, float16_t> ? VK_DTYPE_F16 : VK_DTYPE_F32;
    const int st = vk_gemm(MATMUL_VERSION, dt, dt, m, n, k, A, B, C, nullptr);
    if (st != VK_OK) {
        std::fprintf(stderr, "[Playground] vk_gemm(version=%d, m=%zu, n=%zu, k=%zu) failed: %s\n",
                     MATMUL_VERSION, m, n, k, vk_status_string(st));
        std::exit(EXIT_FAILURE);
    }
}
#endif

}  // namespace playground
