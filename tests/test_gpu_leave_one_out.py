"""Versions 71-77: version 7 with one ingredient of its k-loop or tile order
turned off each (A swizzle, B swizzle, direct-to-LDS loads, the third B
slot, the ping-pong, the XCD-aware tile order, the accumulator chains).

None of them changes what is summed or in which order (per element: k-tiles
ascending, k-step (i ^ j) & 1 of each first for the 16 x 16 block (i, j)
of a wave's 128 x 64 block, the MFMA's own sum over its 32 k), so
each must equal version 7 bit for bit on the same inputs; integer products
must be exact; and at the headline 4096^3 the fp32 output must lie within
the fp32 accumulation bound of the exact (fp64) product.  Small shapes cover
k-loops of 1, 2, 3 and 5 k-tiles (the prologue, the clamped refills and the
two-slot B ring's wrap)."""
import numpy as np
import pytest

from gpu_util import check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

LEAVE_ONE_OUT = list(range(71, 78))
SHAPES = [(256, 256, 64), (256, 512, 128), (512, 256, 192), (768, 512, 320), (1024, 1024, 1024)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_equal_to_version7(gpu, shape, out):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=m + 3 * n + 5 * k)
    C7 = run_gemm(7, A, B, out)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    if out == "f32":
        check_f32_out(C7, A, B, exact)
    for v in LEAVE_ONE_OUT:
        C = run_gemm(v, A, B, out)
        assert np.array_equal(C.view(np.uint16 if out == "f16" else np.uint32),
                              C7.view(np.uint16 if out == "f16" else np.uint32)), f"version {v}"


@pytest.mark.parametrize("shape", SHAPES[:3])
def test_integer_exact(gpu, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=11 * m + n + k)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    for v in LEAVE_ONE_OUT:
        assert np.array_equal(run_gemm(v, A, B, "f32").astype(np.float64), exact), f"version {v}"


@pytest.fixture(scope="module")
def headline_uniform(gpu):
    A, B = make_inputs(4096, 4096, 4096, "uniform", seed=7071)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    return A, B, exact, run_gemm(7, A, B, "f32")


@pytest.mark.slow
@pytest.mark.parametrize("version", LEAVE_ONE_OUT)
def test_headline_4096_fp32_bound_and_equal(gpu, headline_uniform, version):
    """4096^3, uniform[-1,1): within the fp32 bound of the exact product and
    bitwise equal to version 7."""
    A, B, exact, C7 = headline_uniform
    C = run_gemm(version, A, B, "f32")
    check_f32_out(C, A, B, exact)
    assert np.array_equal(C.view(np.uint32), C7.view(np.uint32))


@pytest.fixture(scope="module")
def headline_int(gpu):
    A, B = make_inputs(4096, 4096, 4096, "int", seed=7072)
    return A, B, A.astype(np.float64) @ B.astype(np.float64)


@pytest.mark.slow
@pytest.mark.parametrize("version", LEAVE_ONE_OUT)
def test_headline_4096_integer_exact(gpu, headline_int, version):
    A, B, exact = headline_int
    assert np.array_equal(run_gemm(version, A, B, "f32").astype(np.float64), exact)
