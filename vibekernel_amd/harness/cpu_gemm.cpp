// cpu_gemm.cpp -- version 0 of the playground harness: the CPU ground truth
// (libvk_v0.so, include/vk_v0.h).
//
// The reference's v0 calls OpenBLAS cblas_sgemm
// (results/ralph_loop_fable/src/matmul_f32/matmul_f32_v0_cblas.cpp:10-11) and,
// for fp16, widens to fp32 and narrows the result with round-to-nearest-even
// (results/ralph_loop_fable/src/matmul_f16/matmul_f16_v0_cblas.cpp:13-25).
// This is a self-contained replacement with the same semantics:
//
//  * packed-panel GEMM: B is packed per (NC x KC) block into NR = 16 column
//    panels, A per (MC x KC) block into MR = 6 row panels, and a 6x16
//    register-tile micro-kernel runs 12 AVX2 FMA accumulators;
//  * the k dimension is visited in ascending KC blocks and each micro-tile
//    starts from the partial sum stored in C (or +0 for the first block), so
//    every output element is acc = fma(a_k, b_k, acc) over ascending k --
//    independent of the blocking and of the OpenMP thread count;
//  * fp16 <-> fp32 through the F16C instructions (round to nearest even).
//
// Built with g++ -O3 -mavx2 -mfma -mf16c -fopenmp (x86-64 hosts).
#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "vk_v0.h"

namespace {

constexpr size_t MR = 6;
constexpr size_t NR = 16;
constexpr size_t KC = 256;
constexpr size_t MC = 72;    // 12 row panels
constexpr size_t NC = 2048;  // 128 column panels

// A panel: kc x MR (row index fastest), zero rows beyond mr.
void pack_a(size_t mr, size_t kc, const float* A, size_t lda, float* dst) {
  for (size_t p = 0; p < kc; p++)
    for (size_t r = 0; r < MR; r++) dst[p * MR + r] = r < mr ? A[r * lda + p] : 0.0f;
}

// B panel: kc x NR (column index fastest), zero columns beyond nr.
void pack_b(size_t nr, size_t kc, const float* B, size_t ldb, float* dst) {
  for (size_t p = 0; p < kc; p++) {
    const float* src = B + p * ldb;
    if (nr == NR) {
      std::memcpy(dst + p * NR, src, NR * sizeof(float));
    } else {
      for (size_t c = 0; c < NR; c++) dst[p * NR + c] = c < nr ? src[c] : 0.0f;
    }
  }
}

// C[6][16] (row stride ldc): acc starts from C (first_block ? +0 : C), then
// acc = fma(a[p][r], b[p][c], acc) for p = 0..kc-1.
inline void micro_6x16(size_t kc, const float* a, const float* b, float* c, size_t ldc,
                       bool first_block) {
  __m256 acc[MR][2];
  for (size_t r = 0; r < MR; r++) {
    if (first_block) {
      acc[r][0] = _mm256_setzero_ps();
      acc[r][1] = _mm256_setzero_ps();
    } else {
      acc[r][0] = _mm256_loadu_ps(c + r * ldc);
      acc[r][1] = _mm256_loadu_ps(c + r * ldc + 8);
    }
  }
  for (size_t p = 0; p < kc; p++) {
    const __m256 b0 = _mm256_loadu_ps(b + p * NR);
    const __m256 b1 = _mm256_loadu_ps(b + p * NR + 8);
    for (size_t r = 0; r < MR; r++) {
      const __m256 av = _mm256_broadcast_ss(a + p * MR + r);
      acc[r][0] = _mm256_fmadd_ps(av, b0, acc[r][0]);
      acc[r][1] = _mm256_fmadd_ps(av, b1, acc[r][1]);
    }
  }
  for (size_t r = 0; r < MR; r++) {
    _mm256_storeu_ps(c + r * ldc, acc[r][0]);
    _mm256_storeu_ps(c + r * ldc + 8, acc[r][1]);
  }
}

void sgemm(size_t m, size_t n, size_t k, const float* A, const float* B, float* C) {
  if (m == 0 || n == 0) return;
  if (k == 0) {
    std::fill(C, C + m * n, 0.0f);
    return;
  }
  const size_t ncb = std::min(NC, n);
  std::vector<float> bpack(((ncb + NR - 1) / NR) * NR * KC);
#pragma omp parallel
  {
    std::vector<float> apack(MC * KC);
    float ctile[MR * NR];
    for (size_t jc = 0; jc < n; jc += NC) {
      const size_t nc = std::min(NC, n - jc);
      const size_t npan = (nc + NR - 1) / NR;
      for (size_t pc = 0; pc < k; pc += KC) {
        const size_t kc = std::min(KC, k - pc);
        const bool first = pc == 0;
#pragma omp for schedule(static)
        for (long jp = 0; jp < (long)npan; jp++) {
          const size_t j0 = jc + (size_t)jp * NR;
          pack_b(std::min(NR, n - j0), kc, B + pc * n + j0, n, bpack.data() + (size_t)jp * NR * kc);
        }
        // (implicit barrier: the packed B block is complete)
#pragma omp for schedule(dynamic, 1)
        for (long ib = 0; ib < (long)((m + MC - 1) / MC); ib++) {
          const size_t i0 = (size_t)ib * MC;
          const size_t mc = std::min(MC, m - i0);
          const size_t mpan = (mc + MR - 1) / MR;
          for (size_t ip = 0; ip < mpan; ip++)
            pack_a(std::min(MR, mc - ip * MR), kc, A + (i0 + ip * MR) * k + pc, k,
                   apack.data() + ip * MR * kc);
          for (size_t jp = 0; jp < npan; jp++) {
            const size_t j0 = jc + jp * NR;
            const size_t nr = std::min(NR, n - j0);
            for (size_t ip = 0; ip < mpan; ip++) {
              const size_t r0 = i0 + ip * MR;
              const size_t mr = std::min(MR, m - r0);
              const float* ap = apack.data() + ip * MR * kc;
              const float* bp = bpack.data() + jp * NR * kc;
              if (mr == MR && nr == NR) {
                micro_6x16(kc, ap, bp, C + r0 * n + j0, n, first);
              } else {
                // edge tile through a scratch tile holding the valid part
                for (size_t r = 0; r < MR; r++)
                  for (size_t c = 0; c < NR; c++)
                    ctile[r * NR + c] = (!first && r < mr && c < nr) ? C[(r0 + r) * n + j0 + c] : 0.0f;
                micro_6x16(kc, ap, bp, ctile, NR, first);
                for (size_t r = 0; r < mr; r++)
                  for (size_t c = 0; c < nr; c++) C[(r0 + r) * n + j0 + c] = ctile[r * NR + c];
              }
            }
          }
        }
        // (implicit barrier before the next B block is packed)
      }
    }
  }
}

void widen(const uint16_t* in, float* out, size_t count) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)(count / 8); i++) {
    const __m128i h = _mm_loadu_si128(reinterpret_cast<const __m128i*>(in + 8 * i));
    _mm256_storeu_ps(out + 8 * i, _mm256_cvtph_ps(h));
  }
  for (size_t i = count / 8 * 8; i < count; i++) out[i] = _cvtsh_ss(in[i]);
}

void narrow(const float* in, uint16_t* out, size_t count) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)(count / 8); i++) {
    const __m128i h = _mm256_cvtps_ph(_mm256_loadu_ps(in + 8 * i), _MM_FROUND_TO_NEAREST_INT);
    _mm_storeu_si128(reinterpret_cast<__m128i*>(out + 8 * i), h);
  }
  for (size_t i = count / 8 * 8; i < count; i++) out[i] = _cvtss_sh(in[i], _MM_FROUND_TO_NEAREST_INT);
}

}  // namespace

extern "C" {

void vk_v0_sgemm(size_t m, size_t n, size_t k, const float* A, const float* B, float* C) {
  sgemm(m, n, k, A, B, C);
}

void vk_v0_hgemm(size_t m, size_t n, size_t k, const uint16_t* A, const uint16_t* B, uint16_t* C) {
  std::vector<float> af(m * k), bf(k * n), cf(m * n);
  widen(A, af.data(), m * k);
  widen(B, bf.data(), k * n);
  sgemm(m, n, k, af.data(), bf.data(), cf.data());
  narrow(cf.data(), C, m * n);
}

int vk_v0_threads(void) { return omp_get_max_threads(); }

}  // extern "C"
