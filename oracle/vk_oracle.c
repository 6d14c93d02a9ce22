/*
 * vk_oracle.c -- CPU oracle for the row-major GEMM hot path (TEST
 * INFRASTRUCTURE ONLY; see vk_oracle.h for what it restates and how each
 * function is pinned).
 *
 * Build: oracle/Makefile (gcc -O3 -mavx2 -mfma -fopenmp -ffp-contract=off).
 * -ffp-contract=off keeps every rounding step explicit: the GEMM uses fmaf()
 * on purpose and nothing else may be fused.
 */
#include "vk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* IEEE-754 binary16 <-> binary32, written from the format definition:       */
/* binary16 = 1 sign bit, 5 exponent bits (bias 15), 10 fraction bits.       */
/* The reference narrows with the half(float) constructor, which rounds to   */
/* nearest, ties to even (results/.../matmul_f16_v0_cblas.cpp:25).           */
/* ------------------------------------------------------------------------ */

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  if (e == 0) {
    /* zero or subnormal: value = mant * 2^-24, exact in binary32 */
    float v = (float)mant * 0x1p-24f;
    return sign ? -v : v;
  }
  if (e == 31) {
    /* inf (mant == 0) or NaN (payload kept in the top fraction bits) */
    return bits_f32(sign | 0x7f800000u | (mant << 13));
  }
  return bits_f32(sign | ((e - 15u + 127u) << 23) | (mant << 13));
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t x = f32_bits(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    if (ax == 0x7f800000u) return sign | 0x7c00u;               /* inf */
    uint32_t payload = (ax & 0x7fffffu) >> 13;
    return sign | 0x7c00u | 0x200u | (uint16_t)payload;         /* quiet NaN */
  }
  /* 65520 = midpoint of 65504 (largest finite half, odd significand) and
   * 2^16; ties-to-even and everything above round to inf. */
  if (ax >= 0x477ff000u) return sign | 0x7c00u;
  if (ax < 0x38800000u) {
    /* below 2^-14: the result is a subnormal half (or zero).
     * 2^-25 is the midpoint of 0 and the smallest subnormal: ties to 0. */
    if (ax <= 0x33000000u) return sign;
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;               /* value / 2^-24 = m >> shift */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return sign | (uint16_t)q;               /* q == 0x400 is the min normal */
  }
  uint32_t e = ax >> 23;
  uint32_t mant = ax & 0x7fffffu;
  uint32_t q = ((e - 112u) << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;   /* carry may bump the exponent */
  return sign | (uint16_t)q;
}

void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t count) {
  for (size_t i = 0; i < count; i++) out[i] = orc_f16_to_f32(in[i]);
}

void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t count) {
  for (size_t i = 0; i < count; i++) out[i] = orc_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* SGEMM with cblas_sgemm(RowMajor, NoTrans, NoTrans, m, n, k, 1, A, k, B, n, */
/* 0, C, n) semantics (matmul_f32_v0_cblas.cpp:10-11).                       */
/*                                                                           */
/* Fixed per-element order: acc = +0; for p = 0..k-1: acc = fmaf(A[i][p],    */
/* B[p][j], acc); C[i][j] = acc.  Blocking over rows, columns and k keeps    */
/* that order (k blocks are visited in ascending order and the partial sum   */
/* is carried through C), so the result does not depend on the blocking or  */
/* on the number of threads.                                                  */
/* ------------------------------------------------------------------------ */

#define ORC_MR 4     /* rows per register block */
#define ORC_NR 32    /* columns per register block */
#define ORC_KC 256   /* k per cache block */
#define ORC_MB 64    /* rows per thread task */

static void sgemm_block_generic(size_t i0, size_t mr, size_t j0, size_t nr, size_t k0, size_t kc,
                                size_t n, size_t k, const float* A, const float* B, float* C) {
  for (size_t r = 0; r < mr; r++) {
    for (size_t c = 0; c < nr; c++) {
      float acc = (k0 == 0) ? 0.0f : C[(i0 + r) * n + j0 + c];
      for (size_t p = k0; p < k0 + kc; p++)
        acc = fmaf(A[(i0 + r) * k + p], B[p * n + j0 + c], acc);
      C[(i0 + r) * n + j0 + c] = acc;
    }
  }
}

static void sgemm_block_full(size_t i0, size_t j0, size_t k0, size_t kc, size_t n, size_t k,
                             const float* A, const float* B, float* C) {
  float acc[ORC_MR][ORC_NR];
  for (int r = 0; r < ORC_MR; r++)
    for (int c = 0; c < ORC_NR; c++)
      acc[r][c] = (k0 == 0) ? 0.0f : C[(i0 + r) * n + j0 + c];
  const float* a0 = A + (i0 + 0) * k;
  const float* a1 = A + (i0 + 1) * k;
  const float* a2 = A + (i0 + 2) * k;
  const float* a3 = A + (i0 + 3) * k;
  for (size_t p = k0; p < k0 + kc; p++) {
    const float* b = B + p * n + j0;
    const float x0 = a0[p], x1 = a1[p], x2 = a2[p], x3 = a3[p];
    for (int c = 0; c < ORC_NR; c++) {
      const float bv = b[c];
      acc[0][c] = fmaf(x0, bv, acc[0][c]);
      acc[1][c] = fmaf(x1, bv, acc[1][c]);
      acc[2][c] = fmaf(x2, bv, acc[2][c]);
      acc[3][c] = fmaf(x3, bv, acc[3][c]);
    }
  }
  for (int r = 0; r < ORC_MR; r++)
    for (int c = 0; c < ORC_NR; c++)
      C[(i0 + r) * n + j0 + c] = acc[r][c];
}

void orc_sgemm(size_t m, size_t n, size_t k, const float* A, const float* B, float* C) {
  if (m == 0 || n == 0) return;
  if (k == 0) {
    /* beta = 0: C is overwritten with zeros */
    for (size_t i = 0; i < m * n; i++) C[i] = 0.0f;
    return;
  }
  const long nblk = (long)((m + ORC_MB - 1) / ORC_MB);
#pragma omp parallel for schedule(dynamic, 1)
  for (long ib = 0; ib < nblk; ib++) {
    const size_t ibeg = (size_t)ib * ORC_MB;
    const size_t iend = (ibeg + ORC_MB < m) ? ibeg + ORC_MB : m;
    for (size_t j0 = 0; j0 < n; j0 += ORC_NR) {
      const size_t nr = (n - j0 < ORC_NR) ? n - j0 : ORC_NR;
      for (size_t k0 = 0; k0 < k; k0 += ORC_KC) {
        const size_t kc = (k - k0 < ORC_KC) ? k - k0 : ORC_KC;
        for (size_t i0 = ibeg; i0 < iend; i0 += ORC_MR) {
          const size_t mr = (iend - i0 < ORC_MR) ? iend - i0 : ORC_MR;
          if (mr == ORC_MR && nr == ORC_NR)
            sgemm_block_full(i0, j0, k0, kc, n, k, A, B, C);
          else
            sgemm_block_generic(i0, mr, j0, nr, k0, kc, n, k, A, B, C);
        }
      }
    }
  }
}

/* [v0h] matmul_f16_v0_cblas.cpp:13-25: widen (exact), sgemm, narrow (RNE). */
void orc_hgemm(size_t m, size_t n, size_t k, const uint16_t* A, const uint16_t* B, uint16_t* C) {
  float* Af = (float*)malloc(sizeof(float) * (m * k > 0 ? m * k : 1));
  float* Bf = (float*)malloc(sizeof(float) * (k * n > 0 ? k * n : 1));
  float* Cf = (float*)malloc(sizeof(float) * (m * n > 0 ? m * n : 1));
  orc_f16_to_f32_array(A, Af, m * k);
  orc_f16_to_f32_array(B, Bf, k * n);
  orc_sgemm(m, n, k, Af, Bf, Cf);
  orc_f32_to_f16_array(Cf, C, m * n);
  free(Af); free(Bf); free(Cf);
}

void orc_hgemm_f32out(size_t m, size_t n, size_t k, const uint16_t* A, const uint16_t* B, float* C) {
  float* Af = (float*)malloc(sizeof(float) * (m * k > 0 ? m * k : 1));
  float* Bf = (float*)malloc(sizeof(float) * (k * n > 0 ? k * n : 1));
  orc_f16_to_f32_array(A, Af, m * k);
  orc_f16_to_f32_array(B, Bf, k * n);
  orc_sgemm(m, n, k, Af, Bf, C);
  free(Af); free(Bf);
}

/* fp64 brute force.  fp16 x fp16 products are exact in fp64 (22 significant
 * bits), so for the test sizes this is the exact product up to ~1e-16 rel. */
void orc_dgemm_h(size_t m, size_t n, size_t k, const uint16_t* A, const uint16_t* B, double* C) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)m; i++)
    for (size_t j = 0; j < n; j++) {
      double s = 0.0;
      for (size_t p = 0; p < k; p++)
        s += (double)orc_f16_to_f32(A[(size_t)i * k + p]) * (double)orc_f16_to_f32(B[p * n + j]);
      C[(size_t)i * n + j] = s;
    }
}

void orc_dgemm_f(size_t m, size_t n, size_t k, const float* A, const float* B, double* C) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)m; i++)
    for (size_t j = 0; j < n; j++) {
      double s = 0.0;
      for (size_t p = 0; p < k; p++) s += (double)A[(size_t)i * k + p] * (double)B[p * n + j];
      C[(size_t)i * n + j] = s;
    }
}

/* ------------------------------------------------------------------------ */
/* Error statistic, test_data.hpp:145-162:                                   */
/*   gap = float(GT[i]) - float(C[i]); errSum += |gap / float(GT[i])|;        */
/*   abort if errSum is inf or nan; avgErr = errSum / float(count).           */
/* Skip-zero mode (the later base, playground-base 0a8f197): GT == 0 terms    */
/* are skipped and the divisor is the number of valid terms.  In both modes a */
/* non-finite C element is an error on its own, so a bad kernel cannot hide   */
/* behind a skipped term.                                                     */
/* ------------------------------------------------------------------------ */

static float mean_rel_core(const float* gt_or_null, const uint16_t* gth, const float* c_or_null,
                           const uint16_t* ch, size_t count, int mode, int* status) {
  float errSum = 0.0f;
  size_t valid = 0;
  int st = ORC_STATUS_OK;
  for (size_t i = 0; i < count; i++) {
    const float g = gt_or_null ? gt_or_null[i] : orc_f16_to_f32(gth[i]);
    const float c = c_or_null ? c_or_null[i] : orc_f16_to_f32(ch[i]);
    if (isnan(c)) { st = ORC_STATUS_NAN; break; }
    if (isinf(c)) { st = ORC_STATUS_INF; break; }
    if (mode == ORC_ERR_SKIP_ZERO && g == 0.0f) continue;
    const float gap = g - c;
    errSum += fabsf(gap / g);
    valid++;
    if (isinf(errSum)) { st = ORC_STATUS_INF; break; }
    if (isnan(errSum)) { st = ORC_STATUS_NAN; break; }
  }
  if (st == ORC_STATUS_OK && valid == 0) st = ORC_STATUS_EMPTY;
  if (status) *status = st;
  if (st != ORC_STATUS_OK) return NAN;
  return errSum / (float)valid;
}

float orc_mean_rel_err_h(const uint16_t* GT, const uint16_t* C, size_t count, int mode, int* status) {
  return mean_rel_core(NULL, GT, NULL, C, count, mode, status);
}

float orc_mean_rel_err_f(const float* GT, const float* C, size_t count, int mode, int* status) {
  return mean_rel_core(GT, NULL, C, NULL, count, mode, status);
}

double orc_mean_rel_err_f64(const double* GT, const double* C, size_t count) {
  double s = 0.0;
  size_t valid = 0;
  for (size_t i = 0; i < count; i++) {
    if (GT[i] == 0.0) continue;
    s += fabs((GT[i] - C[i]) / GT[i]);
    valid++;
  }
  return valid ? s / (double)valid : NAN;
}

double orc_max_abs_err_f(const float* GT, const float* C, size_t count) {
  double mx = 0.0;
  for (size_t i = 0; i < count; i++) {
    double d = fabs((double)GT[i] - (double)C[i]);
    if (isnan(d)) return NAN;
    if (d > mx) mx = d;
  }
  return mx;
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
