"""vk_gemm_noalloc: the entry point that allocates nothing (its workspace is
the library's static device scratch array), checked through the C ABI
against vk_gemm on the same inputs -- bit-identical, since both run the same
kernels with the same plans -- on two calls in a row, the second with a
smaller input, for each version that uses a workspace (8: split-K skinny,
9: split tail, 10: split tail with edges, 11: split of an under-filled grid,
14: K split over the waves of a workgroup and over workgroups) and one that
uses none (7)."""
import ctypes

import numpy as np
import pytest

from gpu_util import announce, make_inputs

pytestmark = pytest.mark.gpu

CASES = [
    (8, [(128, 8192, 4096), (16, 2048, 1024)]),
    (9, [(2048, 2048, 4096), (512, 512, 8192)]),
    (10, [(1000, 1000, 4000), (257, 520, 4096)]),
    (11, [(512, 4096, 4096), (200, 296, 2000)]),
    (14, [(128, 4096, 4096), (16, 2048, 8192)]),
    (7, [(1024, 768, 512), (256, 256, 64)]),
]


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("version,shapes", CASES)
def test_noalloc_matches_vk_gemm(gpu, version, shapes):
    import torch
    import vibekernel_amd as vk
    from vibekernel_amd import _abi
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, (m, n, k) in enumerate(shapes):
        A, B = make_inputs(m, n, k, "uniform", seed=100 * version + i)
        tA, tB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
        need = _abi.workspace_bytes(version, vk.DTYPE_F16, m, n, k)
        assert version == 7 or need > 0, "the case must use a workspace"
        assert need <= 64 * 1024 * 1024 + 64 * 1024
        C_ref = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda:0")
        C = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda:0")
        announce(f"noalloc v{version} {m}x{n}x{k} (call {i + 1})")
        assert _abi.gemm(version, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, _p(tA), _p(tB), _p(C_ref), s) == 0
        assert _abi.gemm_noalloc(version, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, _p(tA), _p(tB), _p(C), s) == 0
        torch.cuda.synchronize()
        ref = C_ref.cpu().numpy()
        got = C.cpu().numpy()
        assert not np.isnan(got.astype(np.float32)).any()
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), f"call {i + 1} {m}x{n}x{k}"


def test_noalloc_rejects_bad_calls(gpu):
    import torch
    import vibekernel_amd as vk
    from vibekernel_amd import _abi
    A = torch.zeros((300, 64), dtype=torch.float16, device="cuda:0")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # shape not handled by version 7: rejected before any launch
    assert _abi.gemm_noalloc(7, vk.DTYPE_F16, vk.DTYPE_F16, 300, 64, 64, _p(A), _p(A), _p(A), s) == -3
    assert _abi.gemm_noalloc(99, vk.DTYPE_F16, vk.DTYPE_F16, 256, 256, 64, _p(A), _p(A), _p(A), s) == -1
