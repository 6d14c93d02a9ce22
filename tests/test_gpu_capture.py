"""Stream capture (HIP graphs) of the C ABI: a split call (1000 x 1000 x 4000
on version 10, whose tail tiles are cut into pieces that meet through a
workspace, and version 11, whose 64 tiles of 128 x 128 are each cut into 4
k-slices; 64 x 2048 x 4096 on the skinny version 8, K in 8 pieces; 128 x
4096 x 4096 on version 14, K in 4 pieces over workgroups and 4 over each
workgroup's waves) captured with a caller workspace (vk_gemm_ws) and
replayed several times, with eager work and synchronisations between the replays, each replay
bit-identical to the eager call and within the fp32 bound of the exact
product; the same call through the library workspace (vk_gemm) is refused
under capture; a version with no workspace captures through vk_gemm; and
vk_gemm_noalloc (the library's static scratch, no allocation) captures and
replays bitwise equal to vk_gemm."""
import numpy as np
import pytest

from gpu_util import announce, check_f16_out, make_inputs

pytestmark = pytest.mark.gpu


def _ptr(t):
    import ctypes
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("version,shape", [(10, (1000, 1000, 4000)), (11, (1000, 1000, 4000)),
                                           (8, (64, 2048, 4096)), (14, (128, 4096, 4096))])
def test_split_tail_capture_and_replay(gpu, oracle, version, shape):
    import torch
    import vibekernel_amd as vk
    from vibekernel_amd import _abi
    m, n, k = shape
    A, B = make_inputs(m, n, k, "uniform", seed=31)
    tA, tB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    need = _abi.workspace_bytes(version, vk.DTYPE_F16, m, n, k)
    assert need > 0  # the plan splits this shape
    ws = torch.empty(need, dtype=torch.uint8, device="cuda:0")
    C_eager = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda:0")
    announce(f"capture: eager v{version} {m}x{n}x{k} with caller workspace")
    s = torch.cuda.current_stream()
    st = _abi.gemm_ws(version, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, _ptr(tA), _ptr(tB), _ptr(C_eager),
                      _ptr(ws), need, _ptr_stream(s))
    assert st == 0
    torch.cuda.synchronize()
    ref = C_eager.cpu().numpy()
    check_f16_out(ref, A, B, A.astype(np.float64) @ B.astype(np.float64))

    C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            cs = torch.cuda.current_stream()
            # the library workspace is refused under capture
            st_lib = _abi.gemm(version, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, _ptr(tA), _ptr(tB), _ptr(C),
                               _ptr_stream(cs))
            st_ws = _abi.gemm_ws(version, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, _ptr(tA), _ptr(tB), _ptr(C),
                                 _ptr(ws), need, _ptr_stream(cs))
    torch.cuda.current_stream().wait_stream(side)
    assert st_lib == -6 and st_ws == 0
    for r in range(4):
        C.fill_(float("nan"))
        torch.matmul(tA[:64].float(), tB[:, :64].float())  # eager work between replays
        torch.cuda.synchronize()
        announce(f"capture: v{version} replay {r}")
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy().view(np.uint16), ref.view(np.uint16)), f"replay {r}"


def _ptr_stream(s):
    import ctypes
    return ctypes.c_void_p(s.cuda_stream)


def test_no_workspace_version_captures_through_vk_gemm(gpu):
    import torch
    import vibekernel_amd as vk
    from vibekernel_amd import _abi
    m = n = k = 512
    A, B = make_inputs(m, n, k, "int", seed=5)
    tA, tB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    announce("capture: v7 512^3 through vk_gemm")
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            st = _abi.gemm(7, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, _ptr(tA), _ptr(tB), _ptr(C),
                           _ptr_stream(torch.cuda.current_stream()))
    torch.cuda.current_stream().wait_stream(side)
    assert st == 0
    exact = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float16)
    for _ in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy().view(np.uint16), exact.view(np.uint16))

# vk_gemm_noalloc under capture: version 14 at 128 x 4096 x 4096 (K in 4
# pieces over workgroups and 4 over each workgroup's waves) and version 11 at
# 512 x 4096 x 4096 (64 tiles of 128 x 128, K split over the idle CUs), each
# captured on a side stream and replayed over a poisoned C with eager work
# between the replays; every replay bitwise equal to vk_gemm with the library
# workspace.  This file runs before any other test of vk_gemm_noalloc, so the
# first case is the process's first call of it (the scratch address is looked
# up while the stream captures), in a fresh process or in the whole suite.
def _p(t):
    import ctypes
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("version,shape", [(14, (128, 4096, 4096)), (11, (512, 4096, 4096))])
def test_noalloc_capture_and_replay(gpu, version, shape):
    import ctypes

    import torch
    import vibekernel_amd as vk
    from vibekernel_amd import _abi
    m, n, k = shape
    assert _abi.workspace_bytes(version, vk.DTYPE_F16, m, n, k) > 0  # the plan splits K
    A, B = make_inputs(m, n, k, "uniform", seed=41 + version)
    tA, tB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    C_ref = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda:0")
    announce(f"noalloc capture: eager vk_gemm v{version} {m}x{n}x{k}")
    s0 = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert _abi.gemm(version, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, _p(tA), _p(tB), _p(C_ref), s0) == 0
    torch.cuda.synchronize()
    ref = C_ref.cpu().numpy()
    assert not np.isnan(ref.astype(np.float32)).any()

    C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    announce(f"noalloc capture: capturing v{version}")
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            st = _abi.gemm_noalloc(version, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, _p(tA), _p(tB), _p(C), cs)
    torch.cuda.current_stream().wait_stream(side)
    assert st == 0
    for r in range(3):
        C.fill_(float("nan"))
        torch.matmul(tA[:64].float(), tB[:, :64].float())  # eager work between replays
        torch.cuda.synchronize()
        announce(f"noalloc capture: v{version} replay {r}")
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy().view(np.uint16), ref.view(np.uint16)), f"replay {r}"
