"""GPU parity of version 10 -- version 7's kernel for shapes off its
256 x 256 x 64 grid (any M; N and K multiples of 8) -- and of versions 11
and 12's edge tiles (128 x 128 tiles off their grid, the same treatment)
through the C ABI.

* On the grid it runs version 7's arithmetic in version 7's order: bitwise
  equal results.
* Ragged shapes (the generic f16 suite adds more): integer inputs exact,
  random inputs within the fp32 bound of the exact product.
* Nothing outside C is written: guard regions before and after C keep their
  NaN poison.
* Where its split-tail plan splits (a part-empty last wave, e.g. 1000 x
  1000 x 4000 = 16 tiles), the pieces of a tile meet through the workspace
  as in version 9: same bars, bitwise repeatable, a caller workspace works.
* What lies past an edge in memory -- the next row of A after k = K, the next
  row of B after column N -- never reaches a stored element of C: an
  infinity placed there leaves the other rows and columns finite and exact.
"""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(256, 256, 64), (512, 768, 320), (1024, 512, 1024)])
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_on_grid_equals_v7(gpu, shape, out):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "normal", seed=m + n + k)
    C7 = run_gemm(7, A, B, out)
    C10 = run_gemm(10, A, B, out)
    assert np.array_equal(C7.view(np.uint16 if out == "f16" else np.uint32),
                          C10.view(np.uint16 if out == "f16" else np.uint32))


@pytest.mark.parametrize("version", [10, 11, 12, 13])
@pytest.mark.parametrize("shape", [(300, 264, 72), (1, 8, 8), (257, 1000, 512), (600, 40, 1032), (257, 520, 4096)])
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_writes_only_c(gpu, shape, out, version):
    """C sits between two 4096-element guard regions of NaN; integer inputs
    in [-2, 2] with k <= 1032 keep every sum exact in fp32 and, up to 2048,
    in fp16."""
    import torch
    import vibekernel_amd as vk
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m * 7 + n + k)
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    if out == "f16" and np.abs(exact).max() > 2048:
        pytest.skip("integer result not exact in fp16")
    pad = 4096
    dt = torch.float16 if out == "f16" else torch.float32
    buf = torch.full((pad + m * n + pad,), float("nan"), dtype=dt, device="cuda:0")
    C = buf[pad:pad + m * n].view(m, n)
    announce(f"version={version} guarded m={m} n={n} k={k} out={out}")
    vk.matmul(m, n, k, torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda(), C, version)
    torch.cuda.synchronize()
    assert torch.isnan(buf[:pad]).all() and torch.isnan(buf[pad + m * n:]).all()
    assert np.array_equal(C.cpu().numpy().astype(np.int64), exact)


@pytest.mark.parametrize("version", [10, 11, 12, 13])
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_values_past_the_edges_never_reach_c(gpu, out, version):
    """M = 3, N = 8, K = 72: row 0's last k-tile covers k = 64..127, and
    k = 72..79 of row 0 is, in memory, A[1][0..7]; columns 8..15 of B's row r
    are B[r+1][0..7].  With A[1][0] and B[5][0] infinite, row 1 and column 0
    of C are not finite, and everything else must equal the exact product."""
    m, n, k = 3, 8, 72
    A, B = make_inputs(m, n, k, "int", seed=72)
    A[1, 0] = np.inf
    B[5, 0] = np.inf
    C = run_gemm(version, A, B, out).astype(np.float64)
    with np.errstate(invalid="ignore"):
        exact = A.astype(np.float64) @ B.astype(np.float64)
    keep = np.ones((m, n), dtype=bool)
    keep[1, :] = False
    keep[:, 0] = False
    assert np.all(np.isfinite(C[keep]))
    assert np.array_equal(C[keep], exact[keep])


@pytest.mark.parametrize("version", [10, 11, 12, 13])
@pytest.mark.parametrize("shape", [(1000, 1000, 1000), (4096, 4096, 4128), (2000, 3000, 1000), (1000, 1000, 4000),
                                   (257, 520, 4096), (1496, 1496, 3000)])
def test_ragged_random_vs_oracle(gpu, oracle, shape, version):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=10 + m + k)
    C64 = oracle.dgemm(A, B)
    check_f32_out(run_gemm(version, A, B, "f32"), A, B, C64)
    C16 = run_gemm(version, A, B, "f16")
    check_f16_out(C16, A, B, C64)
    err, st = oracle.mean_rel_err(oracle.hgemm(A, B), C16)
    assert st == oracle.STATUS_OK and err < 2e-4


@pytest.mark.slow
def test_4000_cubed(gpu, oracle):
    m = n = k = 4000
    A, B = make_inputs(m, n, k, "uniform", seed=4000)
    C64 = oracle.dgemm(A, B)
    check_f16_out(run_gemm(10, A, B, "f16"), A, B, C64)


@pytest.mark.slow
def test_edge_repeat_deterministic(gpu):
    """110 launches with C poisoned before each: bitwise equal."""
    import torch
    import vibekernel_amd as vk
    m, n, k = 1000, 1000, 4000  # split tail: 16 tiles in k-slices
    g = torch.Generator(device="cuda:0").manual_seed(10)
    A = (torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1).half()
    B = (torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1).half()
    C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
    announce(f"version=10 repeat x110 {m}x{n}x{k}")
    vk.matmul(m, n, k, A, B, C, 10)
    ref = C.clone()
    for _ in range(110):
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, 10)
        assert torch.equal(C, ref)
    torch.cuda.synchronize()


def test_split_caller_workspace(gpu):
    """vk_gemm_ws with a caller workspace full of garbage on a split shape:
    the launch clears the counters it keeps there, so the result equals the
    library-workspace call, call after call."""
    import torch
    from vibekernel_amd import _abi
    m, n, k = 257, 520, 4096
    A, B = make_inputs(m, n, k, "uniform", seed=257)
    ref = run_gemm(10, A, B, "f32")
    need = _abi.workspace_bytes(10, _abi.DTYPE_F16, m, n, k)
    assert need > 0
    ws = torch.full((need // 4 + 64,), -1, dtype=torch.int32, device="cuda:0")
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    for _ in range(3):
        tC = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
        announce(f"version=10 caller workspace m={m} n={n} k={k}")
        st = _abi.gemm_ws(10, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                          tC.data_ptr(), ws.data_ptr(), ws.numel() * 4)
        assert st == 0
        torch.cuda.synchronize()
        assert np.array_equal(tC.cpu().numpy(), ref)


@pytest.mark.parametrize("version,dtype", [(10, "f16"), (11, "f16"), (12, "f16"), (13, "f16"), (3, "f32")])
@pytest.mark.parametrize("shape", [(3, 8, 72), (17, 40, 200), (300, 264, 104), (100, 136, 2056)])
def test_memory_past_the_operands_is_never_read(gpu, version, dtype, shape):
    """A and B are views at the start of larger buffers whose elements past
    the matrices are +inf: the last k-tile's B rows past K and the A rows past
    M lie beyond the allocations' matrix bytes, and the loads through buffer
    resources sized to the matrices must return zeros there (K % 64 != 0 and
    M, N off the tile grid; 100 x 136 x 2056 also splits K under version
    11).  Every C element is finite and exact."""
    import torch
    import vibekernel_amd as vk
    m, n, k = shape
    npdt = np.float16 if dtype == "f16" else np.float32
    tdt = torch.float16 if dtype == "f16" else torch.float32
    A, B = make_inputs(m, n, k, "int", seed=m + 3 * n + 5 * k, dtype=npdt)
    pad = 1 << 16
    bufA = torch.full((m * k + pad,), float("inf"), dtype=tdt, device="cuda:0")
    bufB = torch.full((k * n + pad,), float("inf"), dtype=tdt, device="cuda:0")
    bufA[:m * k] = torch.from_numpy(A.ravel()).cuda()
    bufB[:k * n] = torch.from_numpy(B.ravel()).cuda()
    tA = bufA[:m * k].view(m, k)
    tB = bufB[:k * n].view(k, n)
    C = torch.full((m, n), float("nan"), dtype=tdt, device="cuda:0")
    announce(f"version={version} {dtype} inf past the operands m={m} n={n} k={k}")
    vk.matmul(m, n, k, tA, tB, C, version)
    torch.cuda.synchronize()
    got = C.cpu().numpy().astype(np.float64)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    assert np.all(np.isfinite(got))
    assert np.array_equal(got, exact)
