"""GPU parity of the fp32 VALU SGEMM (version 1 for fp32) against the oracle's
cblas_sgemm restatement (matmul_f32_v0_cblas.cpp:8-12), through the C ABI."""
import numpy as np
import pytest

from gpu_util import announce, make_inputs

pytestmark = pytest.mark.gpu

SHAPES = [(128, 128, 16), (256, 384, 64), (512, 512, 512), (1, 1, 1), (17, 33, 65), (130, 250, 70)]


def _run(A, B):
    import torch
    import vibekernel_amd as vk
    m, k = A.shape
    n = B.shape[1]
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    tC = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    announce(f"f32 version=1 m={m} n={n} k={k}")
    vk.matmul(m, n, k, tA, tB, tC, 1)
    torch.cuda.synchronize()
    return tC.cpu().numpy()


@pytest.mark.parametrize("shape", SHAPES)
def test_f32_integer_kat(gpu, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m * n + k, dtype=np.float32)
    C = _run(A, B)
    assert np.array_equal(C.astype(np.int64), A.astype(np.int64) @ B.astype(np.int64))


@pytest.mark.parametrize("shape", SHAPES)
def test_f32_random_vs_fp64(gpu, oracle, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=99 + k, dtype=np.float32)
    C = _run(A, B)
    C64 = oracle.dgemm(A, B)
    bound = 1.01 * k * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    assert np.all(np.abs(C - C64) <= bound + 1e-30)
    # Same per-element order as the oracle (k ascending, one fmaf per term,
    # from +0): the results are equal, not just close.
    Corc = oracle.sgemm(A, B)
    assert np.array_equal(C, Corc)


@pytest.mark.slow
def test_f32_4096(gpu, oracle):
    m = n = k = 4096
    A, B = make_inputs(m, n, k, "uniform", seed=5, dtype=np.float32)
    C = _run(A, B)
    Corc = oracle.sgemm(A, B)
    absAB = oracle.sgemm(np.abs(A), np.abs(B)).astype(np.float64)
    assert np.all(np.abs(C.astype(np.float64) - Corc) <= 2 * 1.01 * k * 2.0 ** -24 * absAB)
    assert np.array_equal(C, Corc)
