"""Version 9 (version 7's tile loop with a split tail) on the GPU, through the
C ABI.  The schedule's own arithmetic is checked on the host
(test_splittail_sched.py); here the split tiles' hand-off runs for real.

Shapes and their plans on 256 CUs (vk_splittail.hpp):
  2048 x 2048 x 4096    64 tiles x 4 pieces = 256 units, dealt per XCD
  768 x 2560 x 4096     30 tiles x 4 pieces = 120 units, one chunk
  1024 x 1280 x 2752    20 tiles of 43 k-tiles x 4 pieces of 10/10/10/13
  512 x 512 x 8192      4 tiles x 6 pieces (the last arrival folds 5 partials)
  4096 x 2048 x 4096    128 tiles x 2 pieces = 256 units, dealt per XCD
  4096 x 4352 x 4096    272 tiles: 256 whole + 16 tail tiles x 4 pieces, per XCD
Bars: integer inputs bit-exact (any lost or doubled k-range changes the sum);
random inputs within the fp32 accumulation bound of the exact product (fp32
out) plus half an fp16 ulp (fp16 out); fp16 output equal to the rounding of
the same call's fp32 output; results bitwise repeatable (the pieces are summed
in k order whoever arrives last); a full wave of tiles identical to version 7.
"""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

SK_SHAPES = [(2048, 2048, 4096), (768, 2560, 4096), (1024, 1280, 2752), (512, 512, 8192),
             (4096, 2048, 4096), (4096, 4352, 4096)]


def _ws(m, n, k):
    from vibekernel_amd import _abi
    return _abi.workspace_bytes(9, _abi.DTYPE_F16, m, n, k)


@pytest.mark.parametrize("shape", SK_SHAPES)
def test_splittail_schedule_active(gpu, shape):
    """Each shape really runs split tiles on this device (a workspace is
    needed only then)."""
    assert _ws(*shape) > 0


@pytest.mark.parametrize("shape", SK_SHAPES)
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_splittail_integer_kat_bit_exact(gpu, shape, out):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m + 3 * n + 5 * k)
    # Entries in [-2, 2] and k <= 8192: every partial sum is an integer below
    # 2^15, exact in fp64 whatever the order, so the BLAS product is exact
    # (numpy's int64 matmul has no BLAS path and takes minutes at these sizes).
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    if out == "f16" and np.abs(exact).max() > 2048:
        pytest.skip("integer result not exact in fp16")
    C = run_gemm(9, A, B, out)
    assert np.array_equal(C.astype(np.int64), exact)


@pytest.mark.parametrize("shape", SK_SHAPES)
@pytest.mark.parametrize("dist", ["uniform", "normal"])
def test_splittail_random_vs_oracle(gpu, oracle, shape, dist):
    m, n, k = shape
    A, B = make_inputs(m, n, k, dist, seed=9 * m + n + k)
    C64 = oracle.dgemm(A, B)
    C32 = run_gemm(9, A, B, "f32")
    check_f32_out(C32, A, B, C64)
    C16 = run_gemm(9, A, B, "f16")
    check_f16_out(C16, A, B, C64)
    assert np.array_equal(C16.view(np.uint16), C32.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("out", ["f16", "f32"])
def test_splittail_whole_wave_equals_v7(gpu, out):
    """4096^3 is one full wave on 256 CUs: no split tiles, and the same tile
    loop as version 7, so the results are bit-identical."""
    m = n = k = 4096
    assert _ws(m, n, k) == 0
    A, B = make_inputs(m, n, k, "uniform", seed=97)
    assert np.array_equal(run_gemm(9, A, B, out).view(np.uint8), run_gemm(7, A, B, out).view(np.uint8))


def test_splittail_repeat_and_reshape(gpu):
    """90 launches cycling over three schedules (different unit counts, chunk
    dealing and counters) with C poisoned before each: every result bitwise
    equal to that shape's first.  Counters left non-zero by any call, or a
    partial read before it was complete, would show up here."""
    import torch
    import vibekernel_amd as vk
    g = torch.Generator(device="cuda:0").manual_seed(9)
    data = []
    for m, n, k in [(2048, 2048, 4096), (1024, 1280, 2752), (512, 512, 8192)]:
        A = (torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1).half()
        B = (torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1).half()
        C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
        announce(f"version=9 first call m={m} n={n} k={k}")
        vk.matmul(m, n, k, A, B, C, 9)
        data.append((m, n, k, A, B, C, C.clone()))
    for it in range(90):
        m, n, k, A, B, C, ref = data[it % len(data)]
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, 9)
        assert torch.equal(C, ref), f"call {it}: m={m} n={n} k={k}"
    torch.cuda.synchronize()


def test_splittail_caller_workspace(gpu):
    """vk_gemm_ws with a caller workspace full of garbage: the launch clears
    the counters it keeps there, so the result equals the library-workspace
    call; a workspace one word short is refused."""
    import torch
    from vibekernel_amd import _abi
    m, n, k = 768, 2560, 4096
    A, B = make_inputs(m, n, k, "uniform", seed=6)
    ref = run_gemm(9, A, B, "f32")
    need = _ws(m, n, k)
    ws = torch.full((need // 4 + 64,), -1, dtype=torch.int32, device="cuda:0")
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    tC = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    for _ in range(3):
        tC.fill_(float("nan"))
        announce(f"version=9 caller workspace m={m} n={n} k={k}")
        st = _abi.gemm_ws(9, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                          tC.data_ptr(), ws.data_ptr(), ws.numel() * 4)
        assert st == 0
        torch.cuda.synchronize()
        assert np.array_equal(tC.cpu().numpy(), ref)
    small = _abi.gemm_ws(9, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                         tC.data_ptr(), ws.data_ptr(), need - 4)
    assert small == -6  # VK_ERR_WORKSPACE
