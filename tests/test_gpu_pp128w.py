"""Version 12 (f16_pp128.hip, namespace pp128w): version 11's 128 x 128
tiles with each group of 4 waves taking alternate 64-deep k-tiles of the
whole tile (64 x 64 blocks per wave), the two groups' sums added at the end,
on the 128 x 128 x 64 grid and off it (edges), whole or split over K.

Bars: the fp32 and fp16 outputs against the exact product within the fp32
accumulation bound (fp16: plus half an fp16 ulp), every element written (C
poisoned with NaN); small-integer inputs bit-exact against the oracle (any
k-tile dropped, doubled or taken by both groups changes the sum); fp16
output equal to the rounding of the same call's fp32 output; bitwise
repeatable.  k-tile counts 1, 2, 5, 6 and 7 cover the ring's prologue, the
clamped loads past the last k-tile and an odd count (P computes one more
k-tile than Q).
"""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

WHOLE = [(128, 128, 64), (128, 256, 128), (256, 384, 320), (384, 128, 384), (256, 256, 448),
         (1024, 4096, 4096), (2048, 2048, 1024)]
EDGES = [(1, 8, 8), (100, 264, 136), (257, 520, 200), (129, 136, 72), (300, 264, 72), (1000, 1000, 1000)]
SPLIT = [(512, 4096, 4096), (1000, 1000, 4000), (128, 2048, 2304), (384, 640, 8192), (200, 296, 2000)]


def _ws(m, n, k):
    from vibekernel_amd import _abi
    return _abi.workspace_bytes(12, _abi.DTYPE_F16, m, n, k)


@pytest.mark.parametrize("shape", WHOLE + EDGES + SPLIT)
def test_against_exact_product(gpu, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "normal", seed=m + 13 * n + k)
    C64 = A.astype(np.float64) @ B.astype(np.float64)
    announce(f"version=12 normal m={m} n={n} k={k}")
    C32 = run_gemm(12, A, B, "f32")
    check_f32_out(C32, A, B, C64)
    C16 = run_gemm(12, A, B, "f16")
    check_f16_out(C16, A, B, C64)
    assert np.array_equal(C16.view(np.uint16), C32.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("shape", WHOLE + EDGES + SPLIT)
def test_integer_exact(gpu, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=3 * m + n + 7 * k)
    # entries in [-2, 2], k <= 8192: every partial sum an integer below 2^24
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    announce(f"version=12 int m={m} n={n} k={k}")
    C = run_gemm(12, A, B, "f32")
    assert np.array_equal(C.view(np.uint32), exact.view(np.uint32))


def test_plans(gpu):
    """The split shapes really split (a workspace), the others do not."""
    for shape in SPLIT:
        assert _ws(*shape) > 0
    for shape in WHOLE + EDGES:
        assert _ws(*shape) == 0


def test_repeat_and_reshape(gpu):
    """60 launches cycling over a whole, an edge and a split shape with C
    poisoned before each: every result bitwise equal to that shape's first."""
    import torch
    import vibekernel_amd as vk
    g = torch.Generator(device="cuda:0").manual_seed(12)
    data = []
    for m, n, k in [(1024, 4096, 4096), (1000, 1000, 1000), (512, 4096, 4096)]:
        A = (torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1).half()
        B = (torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1).half()
        C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
        announce(f"version=12 first call m={m} n={n} k={k}")
        vk.matmul(m, n, k, A, B, C, 12)
        data.append((m, n, k, A, B, C, C.clone()))
    for it in range(60):
        m, n, k, A, B, C, ref = data[it % len(data)]
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, 12)
        assert torch.equal(C, ref), f"call {it}: m={m} n={n} k={k}"
    torch.cuda.synchronize()
