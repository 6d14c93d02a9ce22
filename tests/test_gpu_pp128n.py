"""Version 13 (f16_pp128.hip, namespace pp128n): version 11's 128 x 128 tiles
and 64 x 32 wave blocks without the ping-pong -- every wave computes its
64-deep k-tile while reading the next one's fragments.

Each element is the same chain of 16x16x32 MFMAs over 32-deep k-steps in
the same order as in version 11 (64-deep halves ascending, k-step
(i ^ j) & 1 of each first), with the same zero padding at the edges
and the same k-slices where K is split, so the bar is bitwise equality with
version 11 on every shape, whole, edge and split, fp16 and fp32 output (any
wrong fragment, slot, swizzle, wait or piece shows up as a different bit);
plus the exact-product bound on a few shapes and bitwise repeatability.
k-tile counts 1, 2, 3, 5 and 7 cover the prologue, the paired steps and an
odd last step.
"""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

WHOLE = [(128, 128, 64), (128, 256, 128), (256, 384, 192), (384, 128, 320), (256, 256, 448),
         (1024, 4096, 4096), (2048, 2048, 1024)]
EDGES = [(1, 8, 8), (100, 264, 136), (257, 520, 200), (129, 136, 72), (300, 264, 72), (1000, 1000, 1000)]
SPLIT = [(512, 4096, 4096), (1000, 1000, 4000), (128, 2048, 2304), (384, 640, 8192), (200, 296, 2000)]


@pytest.mark.parametrize("out", ["f16", "f32"])
@pytest.mark.parametrize("shape", WHOLE + EDGES + SPLIT)
def test_bitwise_equal_version11(gpu, shape, out):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=m + 17 * n + 3 * k)
    announce(f"version=13 vs 11 m={m} n={n} k={k} out={out}")
    C13 = run_gemm(13, A, B, out)
    C11 = run_gemm(11, A, B, out)
    bits = np.uint16 if out == "f16" else np.uint32
    assert np.array_equal(C13.view(bits), C11.view(bits))


@pytest.mark.parametrize("shape", [(256, 384, 192), (1000, 1000, 1000), (384, 640, 8192)])
def test_against_exact_product(gpu, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "normal", seed=m + n + 5 * k)
    C64 = A.astype(np.float64) @ B.astype(np.float64)
    check_f32_out(run_gemm(13, A, B, "f32"), A, B, C64)
    check_f16_out(run_gemm(13, A, B, "f16"), A, B, C64)


def test_repeat_and_reshape(gpu):
    """60 launches cycling over a whole, an edge and a split shape with C
    poisoned before each: every result bitwise equal to that shape's first."""
    import torch
    import vibekernel_amd as vk
    g = torch.Generator(device="cuda:0").manual_seed(13)
    data = []
    for m, n, k in [(1024, 4096, 4096), (1000, 1000, 1000), (512, 4096, 4096)]:
        A = (torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1).half()
        B = (torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1).half()
        C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
        announce(f"version=13 first call m={m} n={n} k={k}")
        vk.matmul(m, n, k, A, B, C, 13)
        data.append((m, n, k, A, B, C, C.clone()))
    for it in range(60):
        m, n, k, A, B, C, ref = data[it % len(data)]
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, 13)
        assert torch.equal(C, ref), f"call {it}: m={m} n={n} k={k}"
    torch.cuda.synchronize()
