"""Version 11 (f16_pp128.hip: version 7's ping-pong on 128 x 128 tiles,
128-deep k-tiles), the kernel for grids that 256 x 256 tiles leave part
empty.

Bars:
* bitwise equal to version 7 wherever both accept the shape (M, N multiples
  of 256, K of 128): every output element is the same chain of 16x16x32 MFMAs
  over 32-deep k-steps in the same order (64-deep k-tiles ascending; in
  each, k-step ((row / 16) ^ (column / 16)) & 1 first), so any difference is a wrong
  fragment, swizzle, ring slot or store;
* fp32 and fp16 output against the exact product within the fp32
  accumulation bound (fp16: plus half an fp16 ulp), every element written
  (C poisoned with NaN), on shapes version 7 does not take;
* small-integer inputs bit-exact against the oracle;
* off the 128 x 128 x 128 grid (edge tiles: any M, N and K multiples of 8)
  bitwise equal to version 10 where version 10 runs whole tiles: both sum
  each element over the same 32-deep k-steps with zero padding past K (a
  128-deep boundary adds exact zeros to the 64-deep one); the
  guard, past-the-edge and past-the-allocation tests of version 10 cover
  version 11 too (tests/test_gpu_edge.py).
"""
import numpy as np
import pytest

from gpu_util import check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("out", ["f16", "f32"])
@pytest.mark.parametrize("shape", [(256, 256, 128), (512, 768, 384), (1024, 4096, 4096), (2048, 2048, 1024)])
def test_bitwise_equal_version7(gpu, shape, out):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=m * 7 + n * 3 + k)
    C11 = run_gemm(11, A, B, out)
    C7 = run_gemm(7, A, B, out)
    bits = np.uint16 if out == "f16" else np.uint32
    assert np.array_equal(C11.view(bits), C7.view(bits))


@pytest.mark.parametrize("shape", [(128, 128, 128), (384, 640, 256), (128, 2048, 1152), (1152, 384, 512)])
def test_against_exact_product(gpu, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "normal", seed=m + 11 * n + k)
    C64 = A.astype(np.float64) @ B.astype(np.float64)
    check_f32_out(run_gemm(11, A, B, "f32"), A, B, C64)
    check_f16_out(run_gemm(11, A, B, "f16"), A, B, C64)


def test_integer_exact(gpu, oracle):
    m, n, k = 640, 896, 384
    A, B = make_inputs(m, n, k, "int", seed=11)
    C = run_gemm(11, A, B, "f32")
    ref = oracle.hgemm(A, B, out="f32")
    assert np.array_equal(C.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def test_repeat_launch_deterministic(gpu):
    import torch
    import vibekernel_amd as vk
    m, n, k = 1024, 4096, 4096
    A, B = make_inputs(m, n, k, "uniform", seed=5)
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    ref = torch.empty((m, n), dtype=torch.float16, device="cuda")
    vk.matmul(m, n, k, tA, tB, ref, 11)
    C = torch.empty_like(ref)
    for _ in range(20):
        vk.matmul(m, n, k, tA, tB, C, 11)
    torch.cuda.synchronize()
    assert torch.equal(C.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("out", ["f16", "f32"])
@pytest.mark.parametrize("shape", [(1, 8, 8), (100, 264, 136), (257, 520, 200), (1000, 4096, 448), (3000, 1000, 520),
                                   (129, 136, 256)])
def test_edges_bitwise_equal_version10(gpu, shape, out):
    """K <= 448 (at most 7 k-tiles of 64): version 10's split-tail plan never
    splits (a piece needs 8), so it runs whole tiles, one chain per element."""
    import vibekernel_amd as vk
    m, n, k = shape
    assert vk._abi.workspace_bytes(10, vk._abi.DTYPE_F16, m, n, k) == 0
    A, B = make_inputs(m, n, k, "uniform", seed=m + 5 * n + 3 * k)
    C11 = run_gemm(11, A, B, out)
    C10 = run_gemm(10, A, B, out)
    bits = np.uint16 if out == "f16" else np.uint32
    assert np.array_equal(C11.view(bits), C10.view(bits))
