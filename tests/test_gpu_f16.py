"""GPU parity of every fp16 kernel version against the CPU oracle, through the
C ABI (vibekernel_amd.matmul -> vk_gemm).

Bars (tolerances are stated in tests/gpu_util.py):
* integer known-answer inputs: bit-exact, fp16 and fp32 output;
* random inputs, fp32 output: |C - exact| <= 2 k u |A||B| for every element;
* random inputs, fp16 output: that bound plus half an fp16 ulp, and the
  reference's own statistic (mean relative error vs the oracle's v0 result,
  test_data.hpp:145-162) at the strict-tier level (< 1e-4 on N(0,1));
* every element written (C is poisoned with NaN before each launch).
"""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, check_f32_out, make_inputs, run_gemm

pytestmark = pytest.mark.gpu

TILE_SHAPES = [(256, 256, 64), (512, 256, 128), (256, 512, 192), (768, 512, 256), (1024, 1024, 512)]
ANY_SHAPES = [(1, 1, 1), (17, 33, 65), (127, 129, 31), (200, 300, 100), (256, 256, 64), (64, 8, 1000)]
EDGE_SHAPES = [(1, 8, 8), (17, 40, 72), (100, 264, 136), (255, 256, 64), (257, 520, 200), (300, 1000, 520)]
SKINNY_SHAPES = [(16, 256, 512), (32, 512, 1024), (48, 96, 128), (64, 128, 256), (16, 2048, 4096),
                 (80, 256, 512), (96, 384, 96), (112, 128, 1024), (128, 1024, 2048),
                 (1, 128, 32), (5, 256, 512), (17, 384, 1024), (144, 256, 512), (170, 512, 1024),
                 (176, 128, 96), (161, 1024, 2048), (200, 512, 1024), (250, 128, 96), (256, 1024, 2048),
                 (1, 4000, 512), (16, 1000, 256), (200, 264, 1024), (33, 8, 64),
                 (16, 2048, 4064), (100, 1024, 2016)]  # K split in unequal pieces


def _versions():
    import vibekernel_amd as vk
    return vk.versions("f16")


def _shapes_for(version):
    import vibekernel_amd as vk
    c = vk.query(version)
    shapes = [s for s in TILE_SHAPES if s[0] % c.div_m == 0 and s[1] % c.div_n == 0 and s[2] % c.div_k == 0]
    if c.div_m == 1 and c.div_n == 1 and c.div_k == 1:
        shapes = ANY_SHAPES + shapes[:2]
    elif c.div_m == 1:
        shapes = EDGE_SHAPES + shapes[:2]
    if c.max_m <= 256:
        shapes = [s for s in SKINNY_SHAPES if s[0] <= c.max_m and s[0] % c.div_m == 0
                  and s[1] % c.div_n == 0 and s[2] % c.div_k == 0]
    return shapes


def _cases():
    import vibekernel_amd as vk
    vk.load()
    out = []
    for v in _versions():
        for s in _shapes_for(v):
            out.append((v, s))
    return out


@pytest.mark.parametrize("version,shape", _cases())
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_integer_kat_bit_exact(gpu, oracle, version, shape, out):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m + 7 * n + 13 * k)
    # integer entries in [-2, 2]: the fp64 BLAS product is exact (sums < 2^53)
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    if out == "f16" and np.abs(exact).max() > 2048:
        pytest.skip("integer result not exact in fp16")
    C = run_gemm(version, A, B, out)
    assert np.array_equal(C.astype(np.int64), exact)


@pytest.mark.parametrize("version,shape", _cases())
@pytest.mark.parametrize("dist", ["uniform", "normal"])
def test_random_f32_out(gpu, oracle, version, shape, dist):
    m, n, k = shape
    A, B = make_inputs(m, n, k, dist, seed=1000 + m + n + k)
    C = run_gemm(version, A, B, "f32")
    C64 = oracle.dgemm(A, B)
    check_f32_out(C, A, B, C64)
    # same statistic as against the oracle's own fp32 result
    Corc = oracle.hgemm(A, B, out="f32")
    assert np.abs(C - Corc).max() <= 2 * np.abs(Corc.astype(np.float64) - C64).max() + 1e-6


@pytest.mark.parametrize("version,shape", _cases())
@pytest.mark.parametrize("dist", ["uniform", "normal"])
def test_random_f16_out(gpu, oracle, version, shape, dist):
    m, n, k = shape
    A, B = make_inputs(m, n, k, dist, seed=2000 + m + n + k)
    C = run_gemm(version, A, B, "f16")
    C64 = oracle.dgemm(A, B)
    check_f16_out(C, A, B, C64)
    GT = oracle.hgemm(A, B)
    err, st = oracle.mean_rel_err(GT, C)
    assert st == oracle.STATUS_OK
    assert err < 2e-4


@pytest.mark.parametrize("version", [1, 2, 3])
def test_identity(gpu, version):
    n = 256
    rng = np.random.default_rng(1)
    A = np.eye(n, dtype=np.float16)
    B = rng.standard_normal((n, n * 2)).astype(np.float16)
    C = run_gemm(version, A, B, "f16")
    assert np.array_equal(C.view(np.uint16), B.view(np.uint16))


@pytest.mark.parametrize("version", [1, 2, 3])
def test_k_zero_and_empty(gpu, version):
    import torch
    import vibekernel_amd as vk
    C = torch.full((256, 256), float("nan"), dtype=torch.float16, device="cuda:0")
    A = torch.empty((256, 0), dtype=torch.float16, device="cuda:0")
    B = torch.empty((0, 256), dtype=torch.float16, device="cuda:0")
    announce(f"version={version} k=0")
    vk.matmul(256, 256, 0, A, B, C, version)
    torch.cuda.synchronize()
    assert torch.count_nonzero(C).item() == 0
    E = torch.empty((0, 256), dtype=torch.float16, device="cuda:0")
    vk.matmul(0, 256, 0, E, B, E, version)  # m == 0: nothing to do
    torch.cuda.synchronize()


def test_rejected_shape_raises_before_launch(gpu):
    import torch
    import vibekernel_amd as vk
    A = torch.zeros((300, 64), dtype=torch.float16, device="cuda:0")
    B = torch.zeros((64, 256), dtype=torch.float16, device="cuda:0")
    C = torch.zeros((300, 256), dtype=torch.float16, device="cuda:0")
    with pytest.raises(vk.VkError) as e:
        vk.matmul(300, 256, 64, A, B, C, 2)
    assert e.value.status == -3


@pytest.mark.slow
@pytest.mark.parametrize("version", [2, 3, 5, 6, 7])
def test_headline_4096_reference_metric(gpu, oracle, version):
    """4096^3 on the reference's own input distribution (N(0,1)) and metric
    (mean relative error of the fp16 C, test_data.hpp:145-162).

    The statistic between two fp32-accumulated results is dominated by the
    few near-zero outputs, where both sides' fp32 rounding noise is large
    relative to the value, so it measures the noisier side.  The bar is
    therefore: the GPU's distance from the exactly rounded product (fp64 GEMM
    rounded to fp16) is no larger than the v0 restatement's own distance,
    and the reference-style GPU-vs-v0 figure stays within the band that
    noise explains."""
    m = n = k = 4096
    A, B = make_inputs(m, n, k, "normal", seed=20261201)
    C = run_gemm(version, A, B, "f16")
    GT = oracle.hgemm(A, B)
    exact16 = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float16)
    e_gpu, st1 = oracle.mean_rel_err(exact16, C)
    e_v0, st2 = oracle.mean_rel_err(exact16, GT)
    e_ref, st3 = oracle.mean_rel_err(GT, C)
    # The reference's own ground truth is an OpenBLAS sgemm (blocked, not one
    # sequential chain per element): numpy's bundled OpenBLAS on the widened
    # inputs, narrowed with RNE, stands in for it.  Statistical, not bitwise.
    GTb = (A.astype(np.float32) @ B.astype(np.float32)).astype(np.float16)
    e_blas, st4 = oracle.mean_rel_err(GTb, C)
    assert st1 == st2 == st3 == st4 == oracle.STATUS_OK
    print(f"v{version} 4096^3 N(0,1): mean-rel vs exact {e_gpu:.3e} (v0: {e_v0:.3e}); vs v0 {e_ref:.3e}; "
          f"vs OpenBLAS GT {e_blas:.3e} (the reference's strict tier on A100: 3.4e-5 to 4.6e-5)")
    assert e_gpu <= e_v0
    assert e_gpu < 1e-5
    assert e_ref < 3e-4
    # Against a blocked-summation ground truth like the reference's, the
    # statistic is an order of magnitude below the reference's strict tier
    # (its best fp32-accumulate kernels logged 3.4e-5, results/ralph_loop_fable/
    # result.csv:59-60).
    assert e_blas < 1e-5


@pytest.mark.slow
@pytest.mark.parametrize("version", [2, 3, 5, 6, 7])
def test_headline_4096_f32_out(gpu, oracle, version):
    m = n = k = 4096
    A, B = make_inputs(m, n, k, "uniform", seed=7)
    C = run_gemm(version, A, B, "f32")
    Corc = oracle.hgemm(A, B, out="f32")
    absAB = oracle.sgemm(np.abs(A.astype(np.float32)), np.abs(B.astype(np.float32))).astype(np.float64)
    bound = 2 * 2 * k * 2.0 ** -24 * absAB  # both results within k u |A||B| of the exact one
    diff = np.abs(C.astype(np.float64) - Corc)
    assert np.all(diff <= bound)
    print(f"v{version} 4096^3 uniform max |gpu - oracle| = {diff.max():.3e}")


@pytest.mark.slow
@pytest.mark.parametrize("version", [2, 3, 5, 6, 7])
def test_repeat_launch_deterministic(gpu, version):
    """110 launches (the reference caught its cp.async race only after >=110
    runs): C poisoned with NaN before each launch, every result bitwise equal
    to the first."""
    import torch
    import vibekernel_amd as vk
    m = n = k = 2048
    g = torch.Generator(device="cuda:0").manual_seed(3)
    A = (torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1).half()
    B = (torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1).half()
    C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
    announce(f"version={version} repeat x110 {m}^3")
    vk.matmul(m, n, k, A, B, C, version)
    ref = C.clone()
    for _ in range(110):
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, version)
        assert torch.equal(C, ref)
    torch.cuda.synchronize()


@pytest.mark.slow
def test_square8192_normal05(gpu, oracle):
    """8192^3 on N(0, 0.5) inputs (the configuration of the reference's
    fp16-accumulate tier, matmul_f16_v14_f16acc.cu; CDNA4 accumulates in fp32,
    so the strict checks apply): fp32 output within the fp32 accumulation
    bound of the oracle; fp16 output bit-identical to the RNE rounding of the
    kernel's own fp32 output; reference statistic against v0 below the
    relaxed tier's 1e-3."""
    import vibekernel_amd as vk
    version = vk.DEFAULT_F16_VERSION
    m = n = k = 8192
    A, B = make_inputs(m, n, k, "normal0.5", seed=8192)
    C32 = run_gemm(version, A, B, "f32")
    C16 = run_gemm(version, A, B, "f16")
    assert np.array_equal(C16.view(np.uint16), C32.astype(np.float16).view(np.uint16))
    Corc = oracle.hgemm(A, B, out="f32")
    absAB = oracle.sgemm(np.abs(A.astype(np.float32)), np.abs(B.astype(np.float32)))
    diff = np.abs(C32.astype(np.float64) - Corc)
    assert np.all(diff <= 2 * 2 * k * 2.0 ** -24 * absAB.astype(np.float64))
    del absAB, diff
    err, st = oracle.mean_rel_err(Corc.astype(np.float16), C16)
    print(f"v{version} 8192^3 N(0,0.5): mean-rel vs v0 {err:.3e}")
    assert st == oracle.STATUS_OK and err < 1e-3


@pytest.mark.slow
@pytest.mark.parametrize("version", [7, 9])
@pytest.mark.parametrize("shape", [(4096, 11008, 4096), (4096, 4096, 11008)])
def test_mlp_shapes(gpu, oracle, shape, version):
    """The MLP projections (up: 688 tiles of 256 x 256 = 2.69 waves on 256
    CUs, whose tail version 9 leaves whole, as version 7; down:
    one wave of 256 deep tiles): fp32 output against the oracle within the
    fp32 accumulation bound, fp16 output equal to its rounding."""
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=11008)
    C32 = run_gemm(version, A, B, "f32")
    C16 = run_gemm(version, A, B, "f16")
    assert np.array_equal(C16.view(np.uint16), C32.astype(np.float16).view(np.uint16))
    Corc = oracle.hgemm(A, B, out="f32")
    absAB = oracle.sgemm(np.abs(A.astype(np.float32)), np.abs(B.astype(np.float32)))
    assert np.all(np.abs(C32.astype(np.float64) - Corc) <= 2 * 2 * k * 2.0 ** -24 * absAB.astype(np.float64))


@pytest.mark.slow
@pytest.mark.parametrize("version,m", [(4, 16), (8, 16), (8, 128), (8, 1), (8, 200)])
def test_skinny_decode_shape(gpu, oracle, version, m):
    """M = 1, 16, 128 or 200, N = K = 8192 (the decode-like, HBM-bound
    configurations) on the skinny kernels, fp16 and fp32 output, against the
    oracle."""
    n, k = 8192, 8192
    A, B = make_inputs(m, n, k, "uniform", seed=16)
    C64 = oracle.dgemm(A, B)
    C32 = run_gemm(version, A, B, "f32")
    check_f32_out(C32, A, B, C64)
    C16 = run_gemm(version, A, B, "f16")
    check_f16_out(C16, A, B, C64)
    err, st = oracle.mean_rel_err(oracle.hgemm(A, B), C16)
    assert st == oracle.STATUS_OK and err < 2e-4


@pytest.mark.slow
def test_splitk_skinny_repeat_and_reshape(gpu):
    """Version 8 splits K over workgroups and reduces through a counter per
    column block in the library workspace, reset by the last arrival.  110
    launches must give bitwise-identical C (the last arrival sums the parts in
    k order), also when calls of other shapes -- a different split count and
    number of counters -- run in between."""
    import torch
    import vibekernel_amd as vk
    g = torch.Generator(device="cuda:0").manual_seed(8)
    shapes = [(16, 8192, 8192), (64, 1024, 2048), (32, 384, 96), (128, 2048, 4096), (80, 512, 1024)]
    data = []
    for m, n, k in shapes:
        A = (torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1).half()
        B = (torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1).half()
        C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
        announce(f"version=8 first call m={m} n={n} k={k}")
        vk.matmul(m, n, k, A, B, C, 8)
        data.append((m, n, k, A, B, C, C.clone()))
    for it in range(110):
        m, n, k, A, B, C, ref = data[it % len(data)]
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, 8)
        assert torch.equal(C, ref), f"call {it}: m={m} n={n} k={k}"
    torch.cuda.synchronize()


def test_splitk_skinny_shape_sequence(gpu, oracle):
    """Version 8 through the library workspace over shapes whose numbers of
    column blocks and k parts differ, narrow to wide and back: each call's
    partials must leave the next call's counters zero (they once overlapped
    the counters of a wider call), so every call matches the oracle."""
    shapes = [(16, 128, 4096), (128, 256, 2048), (16, 8192, 8192), (32, 28672, 1024), (16, 16384, 1024),
              (48, 384, 2048), (128, 8192, 1024), (200, 1024, 2048), (1, 8192, 1024), (256, 512, 4096), (16, 128, 4096)]
    for m, n, k in shapes:
        A, B = make_inputs(m, n, k, "uniform", seed=m + n + k)
        C = run_gemm(8, A, B, "f32")
        check_f32_out(C, A, B, oracle.dgemm(A, B))


def test_splitk_skinny_caller_workspace(gpu, oracle):
    """vk_gemm_ws with a caller workspace full of garbage: the launch clears the
    counters it keeps there, so the result equals the library-workspace call."""
    import torch
    import vibekernel_amd as vk
    from vibekernel_amd import _abi
    m, n, k = 32, 1024, 4096
    A, B = make_inputs(m, n, k, "uniform", seed=5)
    ref = run_gemm(8, A, B, "f32")
    need = _abi.workspace_bytes(8, _abi.DTYPE_F16, m, n, k)
    assert need > 0
    ws = torch.full((need // 4 + 64,), -1, dtype=torch.int32, device="cuda:0")
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    for _ in range(3):
        tC = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
        announce(f"version=8 caller workspace m={m} n={n} k={k}")
        st = _abi.gemm_ws(8, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                          tC.data_ptr(), ws.data_ptr(), ws.numel() * 4)
        assert st == 0
        torch.cuda.synchronize()
        assert np.array_equal(tC.cpu().numpy(), ref)
    small = _abi.gemm_ws(8, _abi.DTYPE_F16, _abi.DTYPE_F32, m, n, k, tA.data_ptr(), tB.data_ptr(),
                         tC.data_ptr(), ws.data_ptr(), need - 4)
    assert small == -6  # VK_ERR_WORKSPACE


@pytest.mark.parametrize("version,m", [(4, 80), (8, 272)])
def test_skinny_rejects_wide_m(gpu, version, m):
    import torch
    import vibekernel_amd as vk
    A = torch.zeros((m, 128), dtype=torch.float16, device="cuda:0")
    B = torch.zeros((128, 128), dtype=torch.float16, device="cuda:0")
    C = torch.zeros((m, 128), dtype=torch.float16, device="cuda:0")
    with pytest.raises(vk.VkError) as e:
        vk.matmul(m, 128, 128, A, B, C, version)
    assert e.value.status == -3


@pytest.mark.slow
@pytest.mark.parametrize("version", [7, 9])
def test_headline_4096_integer_exact(gpu, version):
    """Every element at the full headline size, bit for bit: integer inputs in
    [-2, 2] keep every partial sum an integer below 2^15, exact in fp32
    whatever the summation order, so the fp32-output C must equal the exact
    product (computed in fp64 by BLAS, itself exact for these values)."""
    m = n = k = 4096
    A, B = make_inputs(m, n, k, "int", seed=4096)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    C = run_gemm(version, A, B, "f32")
    assert np.array_equal(C.astype(np.float64), exact)


@pytest.mark.slow
def test_headline_4096_transpose_and_split_invariants(gpu, oracle):
    """(A.B)^T = B^T.A^T and C = A[:, :K/2].B[:K/2] + A[:, K/2:].B[K/2:] at
    4096^3 on the default kernel, random fp16 inputs, fp32 output.  The
    transposed problem forms the same products and sums them in the same k
    order (k-tiles ascending, the MFMA's own reduction over its 32 k), so it
    is bit-identical; the k-split adds two half sums, so it is held to the
    fp32 accumulation bound (2 x 2 k u |A||B|)."""
    import vibekernel_amd as vk
    version = vk.DEFAULT_F16_VERSION
    m = n = k = 4096
    A, B = make_inputs(m, n, k, "uniform", seed=77)
    C = run_gemm(version, A, B, "f32")
    absAB = oracle.sgemm(np.abs(A.astype(np.float32)), np.abs(B.astype(np.float32))).astype(np.float64)
    bound = 2 * 2 * k * 2.0 ** -24 * absAB
    Ct = run_gemm(version, np.ascontiguousarray(B.T), np.ascontiguousarray(A.T), "f32")
    diff_t = np.abs(Ct.T.astype(np.float64) - C)
    print(f"transpose: max |diff| {diff_t.max():.3e}")
    assert np.array_equal(Ct.T, C)
    h = k // 2
    C1 = run_gemm(version, np.ascontiguousarray(A[:, :h]), np.ascontiguousarray(B[:h]), "f32")
    C2 = run_gemm(version, np.ascontiguousarray(A[:, h:]), np.ascontiguousarray(B[h:]), "f32")
    diff_s = np.abs((C1.astype(np.float64) + C2) - C)
    print(f"k-split: max |diff| {diff_s.max():.3e}")
    assert np.all(diff_s <= bound)
