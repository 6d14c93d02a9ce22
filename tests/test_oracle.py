"""Pins the CPU oracle (oracle/vk_oracle.c) before anything is checked against it.

The reference ships no golden vectors, known-answer tests or fixtures for this
path (its only evidence is run logs), and its v0 lives in OpenBLAS 0.3.33, a
network dependency absent here.  So every oracle function is pinned by checks
that a plausible mistake would fail:

* binary16 <-> binary32: all 65,536 half patterns and every rounding midpoint
  against numpy's IEEE conversion (a wrong bias, a dropped subnormal branch or
  ties-away instead of ties-even fails);
* sgemm / hgemm: integer known-answer tests that are exact under any summation
  order (a dropped term, a transposed operand or a wrong stride changes an
  integer), the identity, the fp64 brute force under the standard error bound
  |C - C64| <= k * u * (|A| |B|), thread-count independence, and a
  statistical comparison with the OpenBLAS bundled in numpy;
* the error statistic (test_data.hpp:145-162): hand-computed values, the
  GT == 0 skip / legacy-abort rules, NaN/inf in C, and an fp64 restatement.
"""
import numpy as np
import pytest

U32 = 2.0 ** -24  # unit roundoff of binary32


# ----------------------------------------------------------------------------
# fp16 <-> fp32
# ----------------------------------------------------------------------------

def test_f16_to_f32_all_patterns(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_roundtrip_all_halves(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    back = oracle.f32_to_f16(f).view(np.uint16)
    finite = ~np.isnan(f)
    assert np.array_equal(back[finite], h[finite])
    assert np.all(np.isnan(back[~finite].view(np.float16)))


def test_f32_to_f16_midpoints_and_neighbours(oracle):
    # Midpoints between consecutive finite halves (exact in fp32) are ties:
    # round-half-even decides them.  Their fp32 neighbours must round to the
    # nearer half.
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)  # +0 .. max finite
    lo = h[:-1].view(np.float16).astype(np.float64)
    hi = h[1:].view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    assert np.array_equal(mid.astype(np.float64), (lo + hi) / 2)  # exact
    pts = np.concatenate([mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(np.inf))])
    pts = np.concatenate([pts, -pts])
    got = oracle.f32_to_f16(pts).view(np.uint16)
    ref = pts.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_f16_special_values(oracle):
    vals = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 65536.0, 1e30, np.inf, -np.inf,
                     2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -14, 6.1e-5, 5.96e-8],
                    dtype=np.float32)
    got = oracle.f32_to_f16(vals).view(np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    assert np.isnan(oracle.f32_to_f16(np.array([np.nan], dtype=np.float32))[0])


def test_f32_to_f16_random(oracle):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    got = oracle.f32_to_f16(f).view(np.uint16)
    ref = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ----------------------------------------------------------------------------
# GEMMs
# ----------------------------------------------------------------------------

SHAPES = [(1, 1, 1), (3, 5, 7), (16, 16, 16), (17, 33, 65), (64, 96, 128), (130, 70, 300), (256, 256, 64)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_sgemm_integer_kat(oracle, m, n, k):
    # Small integers: every partial sum is an integer < 2^24, so every
    # summation order gives the exact integer product.
    rng = np.random.default_rng(m * 1000 + n * 10 + k)
    A = rng.integers(-8, 9, size=(m, k))
    B = rng.integers(-8, 9, size=(k, n))
    exact = A @ B
    got = oracle.sgemm(A.astype(np.float32), B.astype(np.float32))
    assert np.array_equal(got.astype(np.int64), exact)


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_hgemm_integer_kat(oracle, m, n, k):
    # |C| <= 2048 keeps the fp16 output exact as well.
    rng = np.random.default_rng(k * 1000 + m)
    A = rng.integers(-2, 3, size=(m, k))
    B = rng.integers(-2, 3, size=(k, n))
    exact = A @ B
    assert np.abs(exact).max() <= 2048
    got = oracle.hgemm(A.astype(np.float16), B.astype(np.float16))
    assert np.array_equal(got.astype(np.int64), exact)
    got32 = oracle.hgemm(A.astype(np.float16), B.astype(np.float16), out="f32")
    assert np.array_equal(got32.astype(np.int64), exact)


def test_identity_and_ones(oracle):
    rng = np.random.default_rng(3)
    B = rng.standard_normal((64, 80)).astype(np.float32)
    assert np.array_equal(oracle.sgemm(np.eye(64, dtype=np.float32), B), B)
    Bh = B.astype(np.float16)
    assert np.array_equal(oracle.hgemm(np.eye(64, dtype=np.float16), Bh).view(np.uint16), Bh.view(np.uint16))
    ones = oracle.hgemm(np.ones((8, 2048), np.float16), np.ones((2048, 8), np.float16))
    assert np.all(ones == 2048)


def test_rectangular_orientation(oracle):
    # One-hot rows/columns: C[i][j] = A[i][p] * B[p][j] for a single p, so a
    # transposed operand or a swapped stride lands a value in the wrong place.
    m, n, k = 5, 7, 3
    A = np.zeros((m, k), np.float32)
    B = np.zeros((k, n), np.float32)
    A[4, 2] = 3.0
    B[2, 6] = 5.0
    C = oracle.sgemm(A, B)
    assert C[4, 6] == 15.0 and np.count_nonzero(C) == 1


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_sgemm_fp64_error_bound(oracle, m, n, k):
    rng = np.random.default_rng(11 + k)
    A = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    B = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    C = oracle.sgemm(A, B).astype(np.float64)
    C64 = oracle.dgemm(A, B)
    # dgemm itself against numpy's float64 matmul (independent code path)
    assert np.allclose(C64, A.astype(np.float64) @ B.astype(np.float64), rtol=1e-12, atol=1e-12)
    bound = k * U32 * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)) * 1.01
    assert np.all(np.abs(C - C64) <= bound + 1e-30)


def test_hgemm_matches_rounded_fp64(oracle):
    # fp16 out: the fp32 accumulation error is far below half an fp16 ulp, so
    # the result is the RNE rounding of the exact product except when the exact
    # value sits within that error of a rounding midpoint (then 1 ulp apart).
    rng = np.random.default_rng(5)
    m, n, k = 192, 160, 512
    A = rng.standard_normal((m, k)).astype(np.float16)
    B = rng.standard_normal((k, n)).astype(np.float16)
    C = oracle.hgemm(A, B)
    C64 = oracle.dgemm(A, B)
    R = C64.astype(np.float16)  # numpy rounds fp64 -> fp16 with RNE
    bound = k * U32 * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    # half the larger gap around R (at a power of two the gap away from zero
    # is twice the gap toward it)
    up = np.abs(np.nextafter(R, np.float16(np.inf)).astype(np.float64) - R.astype(np.float64))
    dn = np.abs(R.astype(np.float64) - np.nextafter(R, np.float16(-np.inf)).astype(np.float64))
    half_ulp = np.maximum(up, dn) / 2
    # always: within the fp32 accumulation bound plus the final rounding
    assert np.all(np.abs(C.astype(np.float64) - C64) <= bound + half_ulp * 1.0001)
    # where that bound is below half an ulp, at most 1 ulp from RNE(exact)
    diff = np.abs(C.view(np.uint16).astype(np.int32) - R.view(np.uint16).astype(np.int32))
    well_conditioned = bound < half_ulp
    assert diff[well_conditioned].max() <= 1
    assert (diff > 0).mean() < 1e-2


def test_sgemm_thread_independent(oracle):
    rng = np.random.default_rng(9)
    A = rng.standard_normal((300, 513)).astype(np.float32)
    B = rng.standard_normal((513, 257)).astype(np.float32)
    n0 = oracle.num_threads()
    try:
        oracle.set_num_threads(1)
        c1 = oracle.sgemm(A, B)
        oracle.set_num_threads(max(2, n0))
        c2 = oracle.sgemm(A, B)
    finally:
        oracle.set_num_threads(n0)
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))


def test_sgemm_vs_numpy_openblas(oracle):
    # numpy bundles OpenBLAS (a different version than the reference's
    # 0.3.33): statistical agreement only, never bitwise.
    rng = np.random.default_rng(21)
    A = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    B = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    C = oracle.sgemm(A, B)
    N = A @ B
    C64 = oracle.dgemm(A, B)
    e_orc = np.abs(C - C64).max()
    e_np = np.abs(N - C64).max()
    assert e_orc < 4 * e_np + 1e-6 and e_np < 4 * e_orc + 1e-6
    assert np.abs(C - N).max() < 1e-4


def test_k_zero_writes_zeros(oracle):
    C = oracle.sgemm(np.zeros((4, 0), np.float32), np.zeros((0, 5), np.float32))
    assert C.shape == (4, 5) and np.all(C == 0)


# ----------------------------------------------------------------------------
# error statistic (test_data.hpp:145-162)
# ----------------------------------------------------------------------------

def test_mean_rel_err_hand_values(oracle):
    GT = np.array([1.0, 2.0, 4.0], np.float16)
    C = np.array([1.5, 2.0, 3.0], np.float16)
    v, st = oracle.mean_rel_err(GT, C)
    # |(-0.5)/1| + 0 + |1/4| = 0.75, / 3
    assert st == oracle.STATUS_OK and v == pytest.approx(0.25, rel=0, abs=1e-7)


def test_mean_rel_err_zero_gt_rules(oracle):
    GT = np.array([0.0, 2.0], np.float16)
    C = np.array([1.0, 1.0], np.float16)
    v, st = oracle.mean_rel_err(GT, C, oracle.ERR_SKIP_ZERO)
    assert st == oracle.STATUS_OK and v == 0.5
    v, st = oracle.mean_rel_err(GT, C, oracle.ERR_LEGACY)
    assert st == oracle.STATUS_INF
    # 0/0 in legacy mode is nan
    v, st = oracle.mean_rel_err(np.array([0.0], np.float16), np.array([0.0], np.float16), oracle.ERR_LEGACY)
    assert st == oracle.STATUS_NAN
    v, st = oracle.mean_rel_err(np.array([0.0], np.float16), np.array([0.0], np.float16))
    assert st == oracle.STATUS_EMPTY


def test_mean_rel_err_nonfinite_c(oracle):
    GT = np.array([0.0, 1.0, 1.0], np.float16)
    for bad in (np.nan, np.inf):
        C = np.array([bad, 1.0, 1.0], np.float16)  # hidden behind a GT == 0 term
        v, st = oracle.mean_rel_err(GT, C)
        assert st in (oracle.STATUS_NAN, oracle.STATUS_INF)


def test_mean_rel_err_fp32_sequential_vs_fp64(oracle):
    rng = np.random.default_rng(4)
    GT = rng.standard_normal(100_000).astype(np.float16)
    C = (GT.astype(np.float32) * (1 + rng.uniform(-1e-3, 1e-3, GT.size))).astype(np.float16)
    v, st = oracle.mean_rel_err(GT, C)
    v64 = oracle.mean_rel_err_f64(GT.astype(np.float64), C.astype(np.float64))
    assert st == oracle.STATUS_OK
    assert v == pytest.approx(v64, rel=1e-3)
    # the fp32 statistic is not the fp64 one bit for bit (its own rounding)
    assert abs(v - v64) < 1e-3 * v64


def test_max_abs_err(oracle):
    a = np.array([1.0, 2.0, -3.0], np.float32)
    b = np.array([1.5, 2.0, -2.0], np.float32)
    assert oracle.max_abs_err(a, b) == 1.0
