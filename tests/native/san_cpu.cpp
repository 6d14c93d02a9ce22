// Host code under AddressSanitizer and UndefinedBehaviorSanitizer (built by
// tests/native/Makefile, target san): the product's version 0
// (vibekernel_amd/harness/cpu_gemm.cpp: packing, 6x16 micro-kernel, edge
// blocks, fp16 widen/narrow) and the CPU oracle (oracle/vk_oracle.c) on
// ragged shapes that reach every edge path, each result compared bit for bit
// between the two; plus the oracle's statistic on edge arrays.  Any invalid
// access or undefined operation aborts the run (-fno-sanitize-recover).
// Prints "ok <cases>".
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "vk_v0.h"
extern "C" {
#include "vk_oracle.h"
}

static int fails = 0;

static void check(bool ok, const char* what, size_t m, size_t n, size_t k) {
  if (!ok) {
    std::printf("FAIL %s %zux%zux%zu\n", what, m, n, k);
    fails++;
  }
}

int main() {
  const size_t shapes[][3] = {{1, 1, 1},     {1, 17, 3},    {6, 16, 1},   {7, 17, 300}, {5, 1, 33},
                              {13, 31, 0},   {64, 64, 64},  {130, 70, 513}, {73, 2100, 260}, {257, 3, 129},
                              {3, 259, 1027}, {97, 101, 103}};
  std::mt19937 g(7);
  std::uniform_real_distribution<float> d(-1.f, 1.f);
  int cases = 0;
  for (const auto& s : shapes) {
    const size_t m = s[0], n = s[1], k = s[2];
    // exact-size allocations, so any access past an operand is caught
    std::vector<float> A(m * k), B(k * n), C(m * n, NAN), R(m * n, NAN);
    for (auto& x : A) x = d(g);
    for (auto& x : B) x = d(g);
    vk_v0_sgemm(m, n, k, A.data(), B.data(), C.data());
    orc_sgemm(m, n, k, A.data(), B.data(), R.data());
    check(std::memcmp(C.data(), R.data(), C.size() * 4) == 0, "sgemm", m, n, k);
    std::vector<uint16_t> Ah(m * k), Bh(k * n), Ch(m * n, 0x7e00), Rh(m * n, 0x7e00);
    for (size_t i = 0; i < Ah.size(); i++) Ah[i] = orc_f32_to_f16(A[i]);
    for (size_t i = 0; i < Bh.size(); i++) Bh[i] = orc_f32_to_f16(B[i]);
    vk_v0_hgemm(m, n, k, Ah.data(), Bh.data(), Ch.data());
    orc_hgemm(m, n, k, Ah.data(), Bh.data(), Rh.data());
    check(std::memcmp(Ch.data(), Rh.data(), Ch.size() * 2) == 0, "hgemm", m, n, k);
    std::vector<float> Rf(m * n);
    orc_hgemm_f32out(m, n, k, Ah.data(), Bh.data(), Rf.data());
    std::vector<double> D(m * n);
    orc_dgemm_h(m, n, k, Ah.data(), Bh.data(), D.data());
    cases += 4;
    if (m * n) {
      int st = -1;
      const float e = orc_mean_rel_err_h(Rh.data(), Ch.data(), m * n, ORC_ERR_SKIP_ZERO, &st);
      check(k == 0 ? st == ORC_STATUS_EMPTY : (st == ORC_STATUS_OK && e == 0.0f), "stat", m, n, k);
      cases++;
    }
  }
  // statistic edge arrays: zeros, infinities, NaN, one element
  const float gt[5] = {0.f, 1.f, -2.f, 4.f, 0.f}, c_ok[5] = {3.f, 1.5f, -2.f, 4.f, 0.f};
  const float c_inf[5] = {0.f, INFINITY, 1.f, 1.f, 1.f}, c_nan[5] = {0.f, 1.f, NAN, 1.f, 1.f};
  int st = -1;
  const float e = orc_mean_rel_err_f(gt, c_ok, 5, ORC_ERR_SKIP_ZERO, &st);
  check(st == ORC_STATUS_OK && e == (0.5f + 0.f + 0.f) / 3.f, "stat skip-zero", 5, 1, 1);
  orc_mean_rel_err_f(gt, c_inf, 5, ORC_ERR_SKIP_ZERO, &st);
  check(st == ORC_STATUS_INF, "stat inf", 5, 1, 1);
  orc_mean_rel_err_f(gt, c_nan, 5, ORC_ERR_SKIP_ZERO, &st);
  check(st == ORC_STATUS_NAN, "stat nan", 5, 1, 1);
  orc_mean_rel_err_f(gt, c_ok, 5, ORC_ERR_LEGACY, &st);
  check(st != ORC_STATUS_OK, "stat legacy", 5, 1, 1);
  orc_mean_rel_err_f(gt, c_ok, 1, ORC_ERR_SKIP_ZERO, &st);
  check(st == ORC_STATUS_EMPTY, "stat empty", 1, 1, 1);
  cases += 5;
  // every fp16 pattern through both conversions
  for (uint32_t h = 0; h < 65536; h++) {
    const float f = orc_f16_to_f32((uint16_t)h);
    if (!std::isnan(f)) check(orc_f32_to_f16(f) == h, "f16 round trip", h, 0, 0);
  }
  cases++;
  if (fails) return 1;
  std::printf("ok %d\n", cases);
  return 0;
}
