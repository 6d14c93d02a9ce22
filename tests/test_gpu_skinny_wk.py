"""Version 14 (f16_skinny_wk.hip): skinny A (M <= 128) with K split over the
4 waves of a workgroup (each wave every 4th 32-deep k-step, its own loads and
LDS ring) and over workgroups (ks pieces per 64-column block, handed off
through per-(column block, wave) counters).

Shapes cover 1 to 8 row blocks (the register rings change at 5), k-step
counts that leave waves with no step, with whole rings of steps and with
steps of zeros padding the last ring, column blocks that N cuts short, and
ks = 1, 2, 4 and 8, with pieces of equal and unequal step counts (the CPU test of the plan
is tests/test_abi.py).  Bars: small-integer
inputs bit-exact (every partial sum is an integer below 2^24, so any step
dropped, doubled, or taken by two waves or two pieces changes the result);
N(0,1) inputs within the fp32 accumulation bound (fp16 output: plus half an
fp16 ulp) against the float64 product, and fp16 output equal to the
rounding of the same call's fp32 output; every element written (C poisoned
with NaN) and nothing else; no byte past the operands read; bitwise
repeatable across reshapes and with a caller workspace.
"""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

VERSIONS = [14]
MAX_ROWS = {14: 128}
SHAPES = [
    (1, 64, 32),        # one k-step: waves 1-3 have none
    (16, 64, 96),       # three k-steps
    (17, 72, 160),      # N cut (8 of 64 columns in the second block)
    (33, 200, 416),     # 13 k-steps: remainders of the 6-step ring
    (64, 264, 1024),    # ks = 4, 2 steps per wave; 4 row blocks (ring of 6)
    (65, 136, 1088),    # 5 row blocks (ring of 4); 34 steps in 4 pieces of 8 or 9
    (100, 136, 2048),   # 7 row blocks
    (128, 128, 4096),   # ks = 8
    (96, 8192, 1056),   # 33 k-steps in pieces of 16 and 17
    (48, 1000, 2016),   # last column block of 40 columns; 63 k-steps in 4 pieces of 15 or 16
    (5, 8, 8192),       # one 8-column block, ks = 8
    (128, 520, 4064),   # 127 k-steps in 8 pieces of 15 or 16
    (64, 5120, 4096),   # 80 column blocks x 3 pieces of 42 or 43 steps
    (112, 2048, 4096),  # ks = 8 over 32 column blocks
    (128, 8192, 8192),  # batch-128 decode: ks = 2
]
SPLIT = {(64, 264, 1024), (128, 128, 4096), (5, 8, 8192), (112, 2048, 4096), (128, 8192, 8192), (100, 136, 2048),
         (65, 136, 1088), (96, 8192, 1056), (48, 1000, 2016), (128, 520, 4064), (64, 5120, 4096)}


def _ws(v, m, n, k):
    from vibekernel_amd import _abi
    return _abi.workspace_bytes(v, _abi.DTYPE_F16, m, n, k)


def _cases(shapes):
    return [(v, s) for v in VERSIONS for s in shapes if s[0] <= MAX_ROWS[v]]


@pytest.mark.parametrize("V,shape", _cases(SHAPES))
def test_integer_exact(gpu, V, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=5 * m + n + 3 * k)
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    announce(f"version={V} int m={m} n={n} k={k}")
    C = run_gemm(V, A, B, "f32")
    assert np.array_equal(C.view(np.uint32), exact.view(np.uint32))


@pytest.mark.parametrize("V,shape", _cases(SHAPES))
def test_against_exact_product(gpu, V, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "normal", seed=m + 11 * n + k)
    C64 = A.astype(np.float64) @ B.astype(np.float64)
    C32 = run_gemm(V, A, B, "f32")
    check_f32_out(C32, A, B, C64)
    C16 = run_gemm(V, A, B, "f16")
    check_f16_out(C16, A, B, C64)
    assert np.array_equal(C16.view(np.uint16), C32.astype(np.float16).view(np.uint16))


def test_plans(gpu):
    """Which shapes split K over workgroups (a workspace) on this device."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip("the split counts below are those of 256 CUs")
    for shape in SHAPES:
        assert (_ws(14, *shape) > 0) == (shape in SPLIT), shape


@pytest.mark.parametrize("V,shape", _cases([(17, 72, 160), (1, 8, 32), (100, 136, 2048), (128, 8192, 1024),
                                            (80, 264, 2048)]))
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_writes_only_c(gpu, V, shape, out):
    """C between two guard regions of NaN; integer inputs (exact sums)."""
    import torch
    import vibekernel_amd as vk
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m + 7 * n + k)
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    if out == "f16" and np.abs(exact).max() > 2048:
        pytest.skip("integer result not exact in fp16")
    pad = 4096
    dt = torch.float16 if out == "f16" else torch.float32
    buf = torch.full((pad + m * n + pad,), float("nan"), dtype=dt, device="cuda:0")
    C = buf[pad:pad + m * n].view(m, n)
    announce(f"version={V} guarded m={m} n={n} k={k} out={out}")
    vk.matmul(m, n, k, torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda(), C, V)
    torch.cuda.synchronize()
    assert torch.isnan(buf[:pad]).all() and torch.isnan(buf[pad + m * n:]).all()
    assert np.array_equal(C.cpu().numpy().astype(np.int64), exact)


@pytest.mark.parametrize("V,shape", _cases([(3, 8, 64), (17, 40, 224), (100, 136, 2048), (127, 264, 1056),
                                            (79, 136, 1056)]))
def test_memory_past_the_operands_is_never_read(gpu, V, shape):
    """A and B at the start of larger buffers of +inf: rows past M (a block
    of 16 rows loads row M - 1 instead) and columns past N (a cut column
    block loads its last valid chunk instead) never reach memory past the
    matrices, so every C element is finite and exact."""
    import torch
    import vibekernel_amd as vk
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m + 3 * n + 5 * k)
    pad = 1 << 16
    bufA = torch.full((m * k + pad,), float("inf"), dtype=torch.float16, device="cuda:0")
    bufB = torch.full((k * n + pad,), float("inf"), dtype=torch.float16, device="cuda:0")
    bufA[:m * k] = torch.from_numpy(A.ravel()).cuda()
    bufB[:k * n] = torch.from_numpy(B.ravel()).cuda()
    C = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    announce(f"version={V} inf past the operands m={m} n={n} k={k}")
    vk.matmul(m, n, k, bufA[:m * k].view(m, k), bufB[:k * n].view(k, n), C, V)
    torch.cuda.synchronize()
    got = C.cpu().numpy().astype(np.float64)
    assert np.all(np.isfinite(got))
    assert np.array_equal(got, A.astype(np.float64) @ B.astype(np.float64))


@pytest.mark.parametrize("V", VERSIONS)
def test_repeat_and_reshape(gpu, V):
    """80 launches cycling over split and unsplit shapes with different
    column-block and piece counts, C poisoned before each: every result
    bitwise equal to that shape's first (the last arrival sums the pieces in
    k order, and each call leaves the counters at zero)."""
    import torch
    import vibekernel_amd as vk
    g = torch.Generator(device="cuda:0").manual_seed(14)
    data = []
    shapes = [(128, 8192, 8192), (16, 8192, 1056), (64, 1024, 4096), (5, 8, 8192), (100, 264, 2048), (80, 4096, 4096)]
    for m, n, k in [s for s in shapes if s[0] <= MAX_ROWS[V]]:
        A = (torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1).half()
        B = (torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1).half()
        C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
        announce(f"version={V} first call m={m} n={n} k={k}")
        vk.matmul(m, n, k, A, B, C, V)
        data.append((m, n, k, A, B, C, C.clone()))
    for it in range(80):
        m, n, k, A, B, C, ref = data[it % len(data)]
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, V)
        assert torch.equal(C, ref), f"call {it}: m={m} n={n} k={k}"
    torch.cuda.synchronize()


@pytest.mark.parametrize("V", VERSIONS)
def test_caller_workspace(gpu, V):
    """vk_gemm_ws with a caller workspace full of garbage: the launch clears
    its counters, so the result equals the library-workspace call; a
    workspace one word short is refused."""
    import torch
    from vibekernel_amd import _abi
    m, n, k = 80, 2048, 4096
    A, B = make_inputs(m, n, k, "uniform", seed=14)
    ref = run_gemm(V, A, B, "f32")
    need = _ws(V, m, n, k)
    assert need > 0
    ws = torch.full((need // 4 + 64,), -1, dtype=torch.int32, device="cuda:0")
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    for _ in range(3):
        tC = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
        announce(f"version={V} caller workspace m={m} n={n} k={k}")
        st = _abi.gemm_ws(V, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                          tC.data_ptr(), ws.data_ptr(), ws.numel() * 4)
        assert st == 0
        torch.cuda.synchronize()
        assert np.array_equal(tC.cpu().numpy(), ref)
    small = _abi.gemm_ws(V, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                         tC.data_ptr(), ws.data_ptr(), need - 4)
    assert small == -6  # VK_ERR_WORKSPACE


@pytest.mark.parametrize("V,m", [(v, m) for v in VERSIONS for m in [1, 16, 64, 80, 128] if m <= MAX_ROWS[v]])
def test_decode_shapes_vs_oracle(gpu, oracle, V, m):
    """M x 8192 x 8192 (decode-like, HBM-bound), uniform[-1,1): fp32 and
    fp16 output against the oracle's float64 product, and the reference's
    statistic against the oracle's v0 result."""
    n, k = 8192, 8192
    A, B = make_inputs(m, n, k, "uniform", seed=1400 + m)
    C64 = oracle.dgemm(A, B)
    check_f32_out(run_gemm(V, A, B, "f32"), A, B, C64)
    C16 = run_gemm(V, A, B, "f16")
    check_f16_out(C16, A, B, C64)
    err, st = oracle.mean_rel_err(oracle.hgemm(A, B), C16)
    assert st == oracle.STATUS_OK and err < 2e-4


@pytest.mark.parametrize("V", VERSIONS)
def test_rejects_more_rows(gpu, V):
    import torch
    import vibekernel_amd as vk
    m = MAX_ROWS[V] + 1
    A = torch.zeros((m, 128), dtype=torch.float16, device="cuda:0")
    B = torch.zeros((128, 128), dtype=torch.float16, device="cuda:0")
    C = torch.zeros((m, 128), dtype=torch.float16, device="cuda:0")
    with pytest.raises(vk.VkError) as e:
        vk.matmul(m, 128, 128, A, B, C, V)
    assert e.value.status == -3
