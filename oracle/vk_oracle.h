/*
 * vk_oracle.h -- CPU oracle for the row-major GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * task1 harness, the Python package) may include, link or call this code.
 * Only tests/ and __graft_entry__.smoke() use it, and only as the checker
 * (bench.py's cpu_baseline times the harness's version 0, libvk_v0.so).
 *
 * What it restates (paths relative to the reference repository root):
 *   - v0 fp32:  results/ralph_loop_fable/src/matmul_f32/matmul_f32_v0_cblas.cpp:8-12
 *               cblas_sgemm(RowMajor, NoTrans, NoTrans, m, n, k, 1, A, k, B, n, 0, C, n)
 *   - v0 fp16:  results/ralph_loop_fable/src/matmul_f16/matmul_f16_v0_cblas.cpp:11-26
 *               widen A, B to fp32 (exact), the same sgemm, narrow C to fp16 (RNE)
 *   - metric:   results/naive_cycle4/include/playground/test_data.hpp:145-162
 *               mean(|GT - C| / |GT|) accumulated sequentially in fp32, abort on
 *               inf/nan; plus the later skip-GT==0 rule
 *               (.claude/memory/playground-base-clean-fork-topology.md:14)
 *
 * The reference's sgemm lives in OpenBLAS 0.3.33 (a vcpkg download, absent
 * here).  Its summation order is implementation-defined; this oracle fixes one
 * order (per output element, k ascending, one fused multiply-add per term,
 * accumulator starting at +0.0f), which is a valid cblas_sgemm result.  Parity
 * against OpenBLAS is therefore statistical, never bitwise.
 *
 * Pinning (tests/test_oracle.py): fp16<->fp32 conversion is checked on all
 * 65,536 half values and on every rounding midpoint against numpy; the GEMMs
 * against integer known-answer tests that are exact under any order, against an
 * fp64 brute force, and statistically against the OpenBLAS bundled with numpy;
 * the metric against hand-computed cases and an fp64 restatement.
 */
#ifndef VK_ORACLE_H
#define VK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE-754 binary16 <-> binary32 (round to nearest even) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t count);
void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t count);

/* ---- GEMMs, row-major, C = A(m x k) . B(k x n), alpha = 1, beta = 0 ---- */
/* cblas_sgemm semantics; OpenMP over row blocks; result independent of the
 * thread count (the per-element order is fixed). */
void orc_sgemm(size_t m, size_t n, size_t k, const float* A, const float* B, float* C);
/* [v0h]: fp16 in, widen, sgemm, fp16 out (RNE). */
void orc_hgemm(size_t m, size_t n, size_t k, const uint16_t* A, const uint16_t* B, uint16_t* C);
/* fp16 in, widen, sgemm, fp32 out (the fp32-output extension; no fp16 rounding). */
void orc_hgemm_f32out(size_t m, size_t n, size_t k, const uint16_t* A, const uint16_t* B, float* C);
/* fp64 brute force (i, j, k triple loop, sequential k), inputs fp16 or fp32. */
void orc_dgemm_h(size_t m, size_t n, size_t k, const uint16_t* A, const uint16_t* B, double* C);
void orc_dgemm_f(size_t m, size_t n, size_t k, const float* A, const float* B, double* C);

/* ---- error statistics ---- */
enum {
  ORC_ERR_SKIP_ZERO = 0,   /* skip GT == 0 terms, divide by the valid count */
  ORC_ERR_LEGACY = 1       /* every term counts; GT == 0 makes the sum inf -> abort */
};
enum {
  ORC_STATUS_OK = 0,
  ORC_STATUS_INF = 1,      /* the running fp32 sum became inf (reference aborts) */
  ORC_STATUS_NAN = 2,      /* the running fp32 sum became nan (reference aborts) */
  ORC_STATUS_EMPTY = 3     /* no valid term */
};
/* test_data.hpp:145-162, GT and C given as fp16 bit patterns. */
float orc_mean_rel_err_h(const uint16_t* GT, const uint16_t* C, size_t count, int mode, int* status);
/* Same statistic on fp32 values (fp32-output extension). */
float orc_mean_rel_err_f(const float* GT, const float* C, size_t count, int mode, int* status);
/* fp64 restatement of the same statistic (cross-check only; skip-zero rule). */
double orc_mean_rel_err_f64(const double* GT, const double* C, size_t count);
/* max |GT - C| over all elements, in fp64. */
double orc_max_abs_err_f(const float* GT, const float* C, size_t count);

/* number of OpenMP threads the GEMMs use (1 without OpenMP) */
int orc_num_threads(void);
/* set it (n <= 0 keeps the current value) */
void orc_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
