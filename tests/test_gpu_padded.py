"""GPU parity of version 15 -- any fp16 shape through row-padded copies of
A, B and C around version 10 -- through the C ABI.

* Its results are version 10's on explicitly zero-padded operands (N and K
  rounded up to 8), bit for bit: the pad only adds exact zeros.
* Random inputs: within the fp32 accumulation bound of the exact (fp64)
  product (plus fp16 rounding for fp16 output); integer inputs exact.
* Nothing outside C is written (NaN guards before and after it).
* Shapes include K and N off the 8-element alignment, both, a vocabulary of
  50,257 columns, and one element.
"""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

SHAPES = [(1000, 1001, 1000), (999, 1000, 1001), (17, 33, 65), (1, 1, 1), (257, 4095, 136), (64, 50257, 512),
          (300, 200, 4095), (1024, 1024, 1023)]


def _padded(A, B):
    m, k = A.shape
    n = B.shape[1]
    k8, n8 = -(-k // 8) * 8, -(-n // 8) * 8
    Ap = np.zeros((m, k8), dtype=A.dtype)
    Ap[:, :k] = A
    Bp = np.zeros((k8, n8), dtype=B.dtype)
    Bp[:k, :n] = B
    return Ap, Bp


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_random_vs_exact_and_v10_padded(gpu, oracle, shape, out):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=m + 3 * n + k)
    C = run_gemm(15, A, B, out)
    C64 = oracle.dgemm(A.astype(np.float32), B.astype(np.float32))
    (check_f16_out if out == "f16" else check_f32_out)(C, A, B, C64)
    Ap, Bp = _padded(A, B)
    C10 = run_gemm(10, Ap, Bp, out)[:, :n]
    u = np.uint16 if out == "f16" else np.uint32
    assert np.array_equal(np.ascontiguousarray(C).view(u), np.ascontiguousarray(C10).view(u))


@pytest.mark.parametrize("shape", [(300, 261, 77), (1, 9, 7), (130, 1001, 1030)])
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_integer_exact_and_writes_only_c(gpu, shape, out):
    import torch
    import vibekernel_amd as vk
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m * 5 + n + k)
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    if out == "f16" and np.abs(exact).max() > 2048:
        pytest.skip("integer result not exact in fp16")
    pad = 4096
    dt = torch.float16 if out == "f16" else torch.float32
    buf = torch.full((pad + m * n + pad,), float("nan"), dtype=dt, device="cuda:0")
    C = buf[pad:pad + m * n].view(m, n)
    announce(f"version=15 guarded m={m} n={n} k={k} out={out}")
    vk.matmul(m, n, k, torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda(), C, 15)
    torch.cuda.synchronize()
    assert torch.isnan(buf[:pad]).all() and torch.isnan(buf[pad + m * n:]).all()
    assert np.array_equal(C.cpu().numpy().astype(np.int64), exact)


def test_repeatable(gpu):
    """Two calls in a row (the second reuses the library workspace and version
    10's counters): bitwise equal."""
    A, B = make_inputs(1000, 1001, 4001, "normal", seed=11)
    C1 = run_gemm(15, A, B, "f16")
    C2 = run_gemm(15, A, B, "f16")
    assert np.array_equal(C1.view(np.uint16), C2.view(np.uint16))
