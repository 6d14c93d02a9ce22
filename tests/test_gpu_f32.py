"""GPU parity of the fp32 kernels against the oracle's cblas_sgemm restatement
(matmul_f32_v0_cblas.cpp:8-12), through the C ABI.

* version 1 (VALU, one fmaf per term in ascending k; 128 x 256 tiles, or
  64 x 64 where those fill the CUs in fewer rounds): equal to the oracle,
  bit for bit, on every shape;
* version 2 (matrix cores, v_mfma_f32_32x32x2_f32, two products per step;
  the four-wave kernel when K % 32 == 0 -- 256 x 256 tiles where they fill
  the CUs in as few rounds as smaller ones, else 128 x 128 tiles, or 64 x 64
  where those are fewer than the CUs, K split where the tiles fill at
  most half of them or leave a last round part empty; K % 32 == 16 on
  256 x 256 tiles: the eight-wave kernel with 16-deep k-tiles): integer
  inputs exact; random inputs within 2 k u |A||B| of the exact (fp64)
  product; bitwise repeatable launch to launch (a split shape); shapes
  include one k-tile (K = 32), more tiles than CUs, every tile size whole
  and split;
* version 3 (version 2 with masked edges: any M, N and K multiples of 4; the
  four-wave kernel when K % 32 == 0 or on 128 x 128 tiles, the last k-tile
  then masked per lane): the same bars on ragged shapes,
  bitwise equal to version 2 on its grid, nothing written outside C, and the
  values past an edge in memory never reach C.
"""
import numpy as np
import pytest

from gpu_util import announce, make_inputs

pytestmark = pytest.mark.gpu

# version 1 on 256 CUs: 64 x 64 tiles for every shape here but the last two
# (the bounds-checked 128 x 256 kernel at 4000 x 4000, the asm kernel at
# 4096 x 4096)
SHAPES_V1 = [(128, 128, 16), (256, 384, 64), (512, 512, 512), (1, 1, 1), (17, 33, 65), (130, 250, 70),
             (128, 256, 16), (256, 512, 32), (384, 768, 48), (1024, 512, 1024), (128, 256, 2000),
             (4000, 4000, 40), (4096, 4096, 32)]
# (version 2, 256 CUs) 256 x 256 tiles: (4096, 4096, 64); 128 x 128 whole:
# (2048, 2048, 128), (4352, 4096, 64) (272 tiles of 256 x 256 would take two
# rounds of the CUs); 128 x 128 with 256 whole tiles and a tail split:
# (2304, 2048, 2048) 32 tail tiles in 4 pieces, (2304, 2304, 2048) 68 in 3
# (one chunk); 64 x 64 whole: (512, 256, 64), (256, 256, 32), (1024, 1024,
# 512), (1024, 1024, 1024), (1280, 1280, 256); 64 x 64 split: (768, 512,
# 256) in 2 pieces, (512, 512, 512) in 4, (256, 256, 1024) in 8;
# 4096 x 4096 x 48: the eight-wave kernel; (256, 256, 16), (256, 512, 48):
# 64 x 64 tiles with the last k-tile masked; (1536, 1536, 1536): 576 tiles of
# 64 x 64, 64 of them in a tail split in 3
SHAPES_V2 = [(256, 256, 16), (512, 256, 64), (256, 512, 48), (768, 512, 256), (1024, 1024, 512), (256, 256, 32),
             (4352, 4096, 64), (512, 512, 512), (1024, 1024, 1024), (256, 256, 1024), (2048, 2048, 128),
             (4096, 4096, 64), (1280, 1280, 256), (4096, 4096, 48), (2304, 2048, 2048),
             (2304, 2304, 2048), (1536, 1536, 1536)]
# 64 x 64 edge tiles split: (300, 600, 2048) in 5 pieces, (129, 4, 512) in
# 8; the k mask on 64 x 64 tiles: (300, 260, 100) in 2 pieces, (1000, 1000,
# 1000) and (17, 36, 68) whole; 4096 x 4096 x 100: the eight-wave kernel with
# its mask; (2100, 2000, 2048): 128 x 128 edge tiles with a split tail
SHAPES_V3 = [(1, 4, 4), (17, 36, 68), (300, 260, 100), (257, 512, 36), (1000, 1000, 1000), (256, 256, 64),
             (300, 260, 96), (257, 516, 64), (1000, 1000, 1024), (1, 4, 32), (300, 600, 2048), (129, 4, 512),
             (4096, 4096, 100), (2100, 2000, 2048)]
CASES = [(1, s) for s in SHAPES_V1] + [(2, s) for s in SHAPES_V2] + [(3, s) for s in SHAPES_V3]


def _run(A, B, version):
    import torch
    import vibekernel_amd as vk
    m, k = A.shape
    n = B.shape[1]
    tA = torch.from_numpy(A).cuda()
    tB = torch.from_numpy(B).cuda()
    tC = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    announce(f"f32 version={version} m={m} n={n} k={k}")
    vk.matmul(m, n, k, tA, tB, tC, version)
    torch.cuda.synchronize()
    return tC.cpu().numpy()


def _bound(A, B, factor):
    k = A.shape[1]
    return factor * k * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))


@pytest.mark.parametrize("version,shape", CASES)
def test_f32_integer_kat(gpu, version, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m * n + k, dtype=np.float32)
    C = _run(A, B, version)
    # entries in [-2, 2]: the fp64 BLAS product is exact
    assert np.array_equal(C.astype(np.int64), (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64))


@pytest.mark.parametrize("version,shape", CASES)
def test_f32_random_vs_fp64(gpu, oracle, version, shape):
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=99 + k, dtype=np.float32)
    C = _run(A, B, version)
    C64 = oracle.dgemm(A, B)
    factor = 1.01 if version == 1 else 2.0
    assert not np.isnan(C).any()
    assert np.all(np.abs(C - C64) <= _bound(A, B, factor) + 1e-30)
    if version == 1:
        # Same per-element order as the oracle (k ascending, one fmaf per term,
        # from +0): the results are equal, not just close.
        assert np.array_equal(C, oracle.sgemm(A, B))


@pytest.mark.slow
@pytest.mark.parametrize("version", [1, 2])
def test_f32_4096(gpu, oracle, version):
    m = n = k = 4096
    A, B = make_inputs(m, n, k, "uniform", seed=5, dtype=np.float32)
    C = _run(A, B, version)
    Corc = oracle.sgemm(A, B)
    absAB = oracle.sgemm(np.abs(A), np.abs(B)).astype(np.float64)
    # both within k u |A||B| (times the factor) of the exact product
    assert np.all(np.abs(C.astype(np.float64) - Corc) <= 2 * 2.0 * k * 2.0 ** -24 * absAB)
    if version == 1:
        assert np.array_equal(C, Corc)


def test_f32_mfma_repeat_deterministic(gpu):
    """20 launches of version 2 with C poisoned before each: bitwise equal
    (64 tiles of 64 x 64, K split in 4: whichever piece arrives last, the
    pieces are summed in k order)."""
    import torch
    import vibekernel_amd as vk
    m, n, k = 512, 512, 1024
    g = torch.Generator(device="cuda:0").manual_seed(2)
    A = torch.rand((m, k), generator=g, device="cuda:0") * 2 - 1
    B = torch.rand((k, n), generator=g, device="cuda:0") * 2 - 1
    C = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    announce(f"f32 version=2 repeat x20 m={m} n={n} k={k}")
    vk.matmul(m, n, k, A, B, C, 2)
    ref = C.clone()
    for _ in range(20):
        C.fill_(float("nan"))
        vk.matmul(m, n, k, A, B, C, 2)
        assert torch.equal(C, ref)
    torch.cuda.synchronize()


def test_f32_mfma_rejects_unaligned_shape(gpu):
    import torch
    import vibekernel_amd as vk
    A = torch.zeros((500, 64), dtype=torch.float32, device="cuda:0")
    B = torch.zeros((64, 256), dtype=torch.float32, device="cuda:0")
    C = torch.zeros((500, 256), dtype=torch.float32, device="cuda:0")
    with pytest.raises(vk.VkError) as e:
        vk.matmul(500, 256, 64, A, B, C, 2)
    assert e.value.status == -3


def test_f32_edge_on_grid_equals_v2(gpu):
    """On version 2's grid with K % 32 == 0 both run 32-deep k-tiles in the
    same order, with the same tiles and split: bitwise equal."""
    for m, n, k in [(256, 256, 64), (512, 768, 320), (256, 512, 32), (512, 512, 512), (256, 256, 1024),
                    (2304, 2048, 2048)]:
        A, B = make_inputs(m, n, k, "normal", seed=m + k, dtype=np.float32)
        assert np.array_equal(_run(A, B, 2).view(np.uint32), _run(A, B, 3).view(np.uint32))


@pytest.mark.parametrize("shape", [(300, 260, 100), (1, 4, 4), (600, 36, 1028), (300, 260, 128), (600, 36, 1024)])
def test_f32_edge_writes_only_c(gpu, shape):
    import torch
    import vibekernel_amd as vk
    m, n, k = shape
    A, B = make_inputs(m, n, k, "int", seed=m + n, dtype=np.float32)
    pad = 4096
    buf = torch.full((pad + m * n + pad,), float("nan"), dtype=torch.float32, device="cuda:0")
    C = buf[pad:pad + m * n].view(m, n)
    announce(f"f32 version=3 guarded m={m} n={n} k={k}")
    vk.matmul(m, n, k, torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda(), C, 3)
    torch.cuda.synchronize()
    assert torch.isnan(buf[:pad]).all() and torch.isnan(buf[pad + m * n:]).all()
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    assert np.array_equal(C.cpu().numpy().astype(np.int64), exact)


def test_f32_edge_values_past_the_edges_never_reach_c(gpu):
    """M = 3, N = 4, K = 36: row 0's k = 36..39 is, in memory, A[1][0..3];
    columns 4..7 of B's row r are B[r+1][0..3].  With A[1][0] and B[5][0]
    infinite, everything outside row 1 and column 0 must be exact."""
    m, n, k = 3, 4, 36
    A, B = make_inputs(m, n, k, "int", seed=36, dtype=np.float32)
    A[1, 0] = np.inf
    B[5, 0] = np.inf
    C = _run(A, B, 3).astype(np.float64)
    with np.errstate(invalid="ignore"):
        exact = A.astype(np.float64) @ B.astype(np.float64)
    keep = np.ones((m, n), dtype=bool)
    keep[1, :] = False
    keep[:, 0] = False
    assert np.all(np.isfinite(C[keep])) and np.array_equal(C[keep], exact[keep])
