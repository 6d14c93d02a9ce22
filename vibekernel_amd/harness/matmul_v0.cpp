// matmul_v0.cpp -- version 0 specialisations: the CPU ground truth.
// Reference: results/ralph_loop_fable/src/matmul_f16/matmul_f16_v0_cblas.cpp:11-26
// and results/ralph_loop_fable/src/matmul_f32/matmul_f32_v0_cblas.cpp:8-12;
// both forward to libvk_v0.so (include/vk_v0.h) instead of OpenBLAS.
#include "playground/matmul.hpp"
#include "playground/system.hpp"
#include "vk_v0.h"

namespace playground {

PLAYGROUND_MATMUL_DEC(float16_t, 0, m, n, k, A, B, C) {
    vk_v0_hgemm(m, n, k, reinterpret_cast<const uint16_t*>(A), reinterpret_cast<const uint16_t*>(B),
                reinterpret_cast<uint16_t*>(C));
}

PLAYGROUND_MATMUL_DEC(float32_t, 0, m, n, k, A, B, C) { vk_v0_sgemm(m, n, k, A, B, C); }

}  // namespace playground
