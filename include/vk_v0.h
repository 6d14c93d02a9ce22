/*
 * vk_v0.h -- C ABI of the CPU ground truth (version 0 of the playground
 * harness), libvk_v0.so.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   results/ralph_loop_fable/src/matmul_f32/matmul_f32_v0_cblas.cpp:8-12
 *     matmul<float32_t, 0>: cblas_sgemm(RowMajor, NoTrans, NoTrans, m, n, k,
 *                                       1, A, k, B, n, 0, C, n)
 *   results/ralph_loop_fable/src/matmul_f16/matmul_f16_v0_cblas.cpp:11-26
 *     matmul<float16_t, 0>: widen A and B to fp32, the same sgemm, narrow C
 *                           to fp16 (round to nearest even)
 * The reference links OpenBLAS for these; this library is its own packed,
 * OpenMP-parallel AVX2/FMA SGEMM with the same semantics (host pointers,
 * row-major, alpha = 1, beta = 0, C fully overwritten).  Per output element
 * it accumulates with one fused multiply-add per k in ascending k from +0,
 * so its result does not depend on the blocking or the thread count.
 */
#ifndef VK_V0_H
#define VK_V0_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void vk_v0_sgemm(size_t m, size_t n, size_t k, const float* A, const float* B, float* C);
/* fp16 operands and result as IEEE binary16 bit patterns. */
void vk_v0_hgemm(size_t m, size_t n, size_t k, const uint16_t* A, const uint16_t* B, uint16_t* C);
/* number of threads the GEMMs use */
int vk_v0_threads(void);

#ifdef __cplusplus
}
#endif
#endif
