"""End to end through the version pick: for shapes that land on each fp16
and fp32 version, pick_version's choice runs on the GPU and its result is
checked against the exact (fp64) product with the fp32 accumulation bound
(tests/gpu_util.py)."""
import numpy as np
import pytest

from gpu_util import check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

F16_CASES = [
    ((1, 256, 64), 8),           # one row: the skinny split-K kernel
    ((16, 4096, 4096), 14),      # 2048 < N <= 4096: K split over the waves of a workgroup too
    ((16, 4096, 14336), 8),      # up to 32 rows with K > 12288: version 8 again
    ((100, 3000, 2048), 14),     # a last column block of 56 columns
    ((128, 2048, 8192), 14),     # N <= 2048 from 65 rows
    ((160, 1024, 2048), 11),     # from 129 rows: 128 x 128 tiles (off the grid, K split)
    ((160, 8192, 512), 11),      # from 129 rows, 128 x 128 tiles over 2 x 64 tiles
    ((96, 4096, 8192), 14),      # 65-128 rows: K up to 8192
    ((1, 1536, 8192), 14),       # up to 8 rows at 1024 < N <= 2048
    ((200, 1024, 2048), 11),     # 128 x 128 tiles (off the grid, K split)
    ((16, 8224, 256), 8),        # n % 128 != 0: the last column block cut short
    ((4096, 4096, 256), 7),      # one full wave of 256 x 256 tiles
    ((512, 512, 512), 11),       # 16 tiles of 128 x 128 where 256 x 256 gives 4 (and no split)
    ((2048, 2048, 4096), 11),    # 256 tiles of 128 x 128: one wave
    ((1024, 1024, 8192), 11),    # 64 tiles of 128 x 128: K split 4 ways over the idle CUs
    ((2048, 2304, 4096), 9),     # 288 tiles of 128 x 128; 72 of 256 x 256, each cut in 3 k-slices
    ((300, 264, 72), 11),        # off the grid: 128 x 128 tiles with edges
    ((1000, 1000, 4000), 11),    # off the grid, 64 tiles of 128 x 128
    ((512, 512, 544), 11),       # k % 64 != 0
    ((2600, 2600, 72), 10),      # off the grid, 441 tiles of 128 x 128: 256 x 256 tiles with edges
    ((100, 300, 70), 1),         # n % 8 != 0: any shape
]
F32_CASES = [
    ((512, 512, 512), 2),
    ((500, 512, 512), 3),
    ((500, 510, 512), 1),
]


@pytest.mark.parametrize("shape,expected", F16_CASES)
def test_f16_pick_runs_and_matches(gpu, oracle, shape, expected):
    import vibekernel_amd as vk
    m, n, k = shape
    v = vk.pick_version(m, n, k)
    assert v == expected
    A, B = make_inputs(m, n, k, "uniform", seed=m + 3 * n + 7 * k)
    check_f32_out(run_gemm(v, A, B, "f32"), A, B, oracle.dgemm(A, B))


@pytest.mark.parametrize("shape,expected", F32_CASES)
def test_f32_pick_runs_and_matches(gpu, oracle, shape, expected):
    import vibekernel_amd as vk
    m, n, k = shape
    v = vk.pick_version(m, n, k, "f32")
    assert v == expected
    A, B = make_inputs(m, n, k, "uniform", seed=m + n + k, dtype=np.float32)
    C = run_gemm(v, A, B, "f32")
    C64 = oracle.dgemm(A, B)
    bound = 2.0 * k * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    assert np.all(np.abs(C - C64) <= bound + 1e-30)


def test_gemm_without_version_uses_the_pick(gpu, oracle):
    """vibekernel_amd.gemm(A, B) with no version: the picked kernel, fp16 and
    fp32 outputs, within the fp32 bound."""
    import torch
    import vibekernel_amd as vk
    for m, n, k in [(1, 4000, 512), (300, 264, 72), (512, 512, 512)]:
        A, B = make_inputs(m, n, k, "uniform", seed=m + n)
        tA, tB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
        C = vk.gemm(tA, tB, out_dtype=torch.float32)
        torch.cuda.synchronize()
        check_f32_out(C.cpu().numpy(), A, B, oracle.dgemm(A, B))
        assert vk.gemm(tA, tB).dtype == torch.float16
