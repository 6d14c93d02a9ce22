"""GPU parity of the fp32 kernels against the oracle's cblas_sgemm restatement
(matmul_f32_v0_cblas.cpp:8-12), through the C ABI.

* version 1 (VALU, one fmaf per term in ascending k): equal to the oracle,
  bit for bit, on every shape;
* version 2 (matrix cores, v_mfma_f32_32x32x2_f32, two products per step):
  integer inputs exact; random inputs within 2 k u |A||B| of the exact
  (fp64) product; bitwise repeatable launch to launch.
"""
import numpy as np
import pytest

from gpu_util import announce, make_inputs

pytestmark = pytest.mark.gpu

SHAPES_V1 = [(128, 128, 16), (256, 384, 64), (512, 512, 512), (1, 1, 1), (17, 33, 65), (130, 250, 70)]
SHAPES_V2 = [(256, 256, 16), (512, 256, 64), (256, 512, 48), (768, 512, 256), (1024, 1024, 512)]
CASES = [(1, s) for s in SHAPES_V1] + [(2, s) for s in SHAPES_V2]


def _run(A, B, version):
    import torch
    import vibekernel_amd as vk
    m, k = A.shape
    n = B.shape[1]
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    tC = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    announce(f"f32 version={version} m={m} n={n} k={k}")
    vk.matmul(m, n, k, tA, tB, tC, version)
    torch.cuda.synchronize()
    return tC.cpu().numpy()


def _bound(A, B, factor):
    k = A.shape[1]
    return factor * k * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))


@pytest.mark.parametrize("version,shape", CASES)
def test_f32_integer_kat(gpu, version, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m * n + k, dtype=np.float32)
    C = _run(A, B, version)
    # entries in [-2, 2]: the fp64 BLAS product is exact
    assert np.array_equal(C.astype(np.int64), (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64))


@pytest.mark.parametrize("version,shape", CASES)
def test_f32_random_vs_fp64(gpu, oracle, version, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=99 + k, dtype=np.float32)
    C = _run(A, B, version)
    C64 = oracle.dgemm(A, B)
    factor = 1.01 if version == 1 else 2.0
    assert not np.isnan(C).any()
    assert np.all(np.abs(C - C64) <= _bound(A, B, factor) + 1e-30)
    if version == 1:
        # Same per-element order as the oracle (k ascending, one fmaf per term,
        # from +0): the results are equal, not just close.
        assert np.array_equal(C, oracle.sgemm(A, B))


@pytest.mark.slow
@pytest.mark.parametrize("version", [1, 2])
def test_f32_4096(gpu, oracle, version):
    m = n = k = 4096
    A, B = make_inputs(m, n, k, "uniform", seed=5, dtype=np.float32)
    C = _run(A, B, version)
    Corc = oracle.sgemm(A, B)
    absAB = oracle.sgemm(np.abs(A), np.abs(B)).astype(np.float64)
    # both within k u |A||B| (times the factor) of the exact product
    assert np.all(np.abs(C.astype(np.float64) - Corc) <= 2 * 2.0 * k * 2.0 ** -24 * absAB)
    if version == 1:
        assert np.array_equal(C, Corc)


def test_f32_mfma_repeat_deterministic(gpu):
    """20 launches of version 2 with C poisoned before each: bitwise equal."""
    import torch
    import vibekernel_amd as vk
    m, n, k = 1024, 768, 512
    g = torch.Generator(device="cuda:0").manual_seed(2)
    A = torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1
    B = torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1
    C = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    announce(f"f32 version=2 repeat x20 m={m} n={n} k={k}")
    vk.matmul(m, n, k, A, B, C, 2)
    ref = C.clone()
    for _ in range(20):
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, 2)
        assert torch.equal(C, ref)
    torch.cuda.synchronize()


def test_f32_mfma_rejects_unaligned_shape(gpu):
    import torch
    import vibekernel_amd as vk
    A = torch.zeros((500, 64), dtype=torch.float32, device="cuda:0")
    B = torch.zeros((64, 256), dtype=torch.float32, device="cuda:0")
    C = torch.zeros((500, 256), dtype=torch.float32, device="cuda:0")
    with pytest.raises(vk.VkError) as e:
        vk.matmul(500, 256, 64, A, B, C, 2)
    assert e.value.status == -3
