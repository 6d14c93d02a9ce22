"""Version 11's split of under-filled grids on the GPU, through the C ABI: a
grid whose 128 x 128 tiles fill at most half of the CUs has every tile cut
into s aligned k-slices computed by s workgroups at once, and the pieces meet
through fp32 partials in the workspace (sk_plan_fill in
vibekernel_amd/csrc/vk_splittail.hpp; the schedule's arithmetic is checked on
the host by tests/native/splittail_check.cpp).

Shapes and their plans on 256 CUs:
  512 x 4096 x 4096     128 tiles x 2 pieces of 15 / 17 k-tiles, per XCD
  1000 x 1000 x 4000    64 tiles (edges) x 4 pieces, per XCD
  128 x 2048 x 2304     16 tiles x 2 pieces of 8 / 10 k-tiles, per XCD
  384 x 640 x 8192      15 tiles x 8 pieces (the last folds 7 partials)
  200 x 296 x 2000      6 tiles (edges) x 2 pieces, one chunk
Bars: integer inputs bit-exact (a lost or doubled k-range changes the sum);
random inputs within the fp32 accumulation bound of the exact product (fp32
out) plus half an fp16 ulp (fp16 out); fp16 output equal to the rounding of
the same call's fp32 output; results bitwise repeatable across calls and
shape changes (the pieces are summed in k order whoever arrives last).
"""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

SPLIT_SHAPES = [(512, 4096, 4096), (1000, 1000, 4000), (128, 2048, 2304), (384, 640, 8192), (200, 296, 2000)]


def _ws(m, n, k):
    from vibekernel_amd import _abi
    return _abi.workspace_bytes(11, _abi.DTYPE_F16, m, n, k)


@pytest.mark.parametrize("shape", SPLIT_SHAPES)
def test_split_schedule_active(gpu, shape):
    """Each shape really runs split tiles on this device (a workspace is
    needed only then), and a full wave of tiles needs none."""
    assert _ws(*shape) > 0
    assert _ws(2048, 2048, 4096) == 0


@pytest.mark.parametrize("shape", SPLIT_SHAPES)
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_split_integer_kat_bit_exact(gpu, shape, out):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m + 7 * n + 3 * k)
    # Entries in [-2, 2] and k <= 8192: every partial sum is an integer below
    # 2^15, exact in fp64 whatever the order.
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    if out == "f16" and np.abs(exact).max() > 2048:
        pytest.skip("integer result not exact in fp16")
    announce(f"version=11 split int m={m} n={n} k={k} out={out}")
    C = run_gemm(11, A, B, out)
    assert np.array_equal(C.astype(np.int64), exact)


@pytest.mark.parametrize("shape", SPLIT_SHAPES)
@pytest.mark.parametrize("dist", ["uniform", "normal"])
def test_split_random_vs_oracle(gpu, oracle, shape, dist):
    m, n, k = shape
    A, B = make_inputs(m, n, k, dist, seed=11 * m + n + k)
    C64 = oracle.dgemm(A, B)
    announce(f"version=11 split {dist} m={m} n={n} k={k}")
    C32 = run_gemm(11, A, B, "f32")
    check_f32_out(C32, A, B, C64)
    C16 = run_gemm(11, A, B, "f16")
    check_f16_out(C16, A, B, C64)
    assert np.array_equal(C16.view(np.uint16), C32.astype(np.float16).view(np.uint16))


def test_split_repeat_and_reshape(gpu):
    """90 launches cycling over three schedules (different piece counts,
    chunk dealing and edges) with C poisoned before each: every result
    bitwise equal to that shape's first.  Counters left non-zero by any call,
    or a partial read before it was complete, would show up here."""
    import torch
    import vibekernel_amd as vk
    g = torch.Generator(device="cuda:0").manual_seed(11)
    data = []
    for m, n, k in [(512, 4096, 4096), (384, 640, 8192), (200, 296, 2000)]:
        A = (torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1).half()
        B = (torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1).half()
        C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
        announce(f"version=11 split first call m={m} n={n} k={k}")
        vk.matmul(m, n, k, A, B, C, 11)
        data.append((m, n, k, A, B, C, C.clone()))
    for it in range(90):
        m, n, k, A, B, C, ref = data[it % len(data)]
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, 11)
        assert torch.equal(C, ref), f"call {it}: m={m} n={n} k={k}"
    torch.cuda.synchronize()


def test_split_caller_workspace(gpu):
    """vk_gemm_ws with a caller workspace full of garbage: the launch clears
    the counters it keeps there, so the result equals the library-workspace
    call; a workspace one word short is refused."""
    import torch
    from vibekernel_amd import _abi
    m, n, k = 1000, 1000, 4000
    A, B = make_inputs(m, n, k, "uniform", seed=12)
    ref = run_gemm(11, A, B, "f32")
    need = _ws(m, n, k)
    ws = torch.full((need // 4 + 64,), -1, dtype=torch.int32, device="cuda:0")
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    tC = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    for _ in range(3):
        tC.fill_(float("nan"))
        announce(f"version=11 caller workspace m={m} n={n} k={k}")
        st = _abi.gemm_ws(11, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                          tC.data_ptr(), ws.data_ptr(), ws.numel() * 4)
        assert st == 0
        torch.cuda.synchronize()
        assert np.array_equal(tC.cpu().numpy(), ref)
    small = _abi.gemm_ws(11, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                         tC.data_ptr(), ws.data_ptr(), need - 4)
    assert small == -6  # VK_ERR_WORKSPACE
