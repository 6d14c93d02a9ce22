// playground/matmul.hpp -- the operator surface.
// Reference: results/naive_cycle4/include/playground/matmul.hpp:11-39.
// Same primary template, the same two macros (including the reference's
// PLAYGOUND spelling) and the same v0 declarations.  A specialisation for a
// GPU version forwards to the C ABI of libvk_gemm.so (include/vk_gemm.h).
#pragma once

#include <type_traits>

#include "playground/system.hpp"

namespace playground {

template <typename DType, uint8_t Version>
void matmul(size_t m, size_t n, size_t k, const DType* A, const DType* B, DType* C) = delete;

// Playground Matmul Declaration
#define PLAYGROUND_MATMUL_DEC(DType, Version, m, n, k, A, B, C)               \
    template <>                                                               \
    void matmul<DType, Version>(size_t m, size_t n, size_t k, const DType* A, \
                                const DType* B, DType* C)

#define PLAYGOUND_MATMUL_CALL(Version, m, n, k, A, B, C)                      \
    ::playground::matmul<::std::remove_cv_t<::std::remove_reference_t<decltype(*A)>>, Version>( \
        m, n, k, A, B, C)

// ============================================================================
// Version 0: the CPU ground truth (host pointers).
// ----------------------------------------------------------------------------
constexpr auto PG_MATMUL_FP16_CBLAS = 0;
constexpr auto PG_MATMUL_FP32_CBLAS = 0;

/** Matrix multiplication, fp16-v0: widen, CPU SGEMM, narrow (RNE). */
PLAYGROUND_MATMUL_DEC(float16_t, PG_MATMUL_FP16_CBLAS, m, n, k, A, B, C);

/** Matrix multiplication, fp32-v0: CPU SGEMM. */
PLAYGROUND_MATMUL_DEC(float32_t, PG_MATMUL_FP32_CBLAS, m, n, k, A, B, C);

}  // namespace playground
