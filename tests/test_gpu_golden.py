"""Every kernel version against the committed golden fixtures (tests/golden),
through the C ABI, on every fixture shape the version accepts.

Bars: integer fixtures exact (fp32 output; fp16 output where the values fit);
random fixtures within the fp32 accumulation bound of the exact product, plus
half an fp16 ulp for fp16 output; fp32 version 1 equal to the oracle's v0
result bit for bit (same fmaf chain)."""
import glob
import os

import numpy as np
import pytest

from gpu_util import check_f16_out, check_f32_out, run_gemm

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def _cases():
    import vibekernel_amd as vk
    from vibekernel_amd import _abi
    vk.load()
    out = []
    for path in FIXTURES:
        with np.load(path, allow_pickle=False) as z:
            (m, k), n = z["A"].shape, z["B"].shape[1]
            f16 = z["A"].dtype == np.float16
        dt = _abi.DTYPE_F16 if f16 else _abi.DTYPE_F32
        for v in _abi.versions(dt):
            outs = ["f16", "f32"] if f16 else ["f32"]
            for o in outs:
                odt = _abi.DTYPE_F16 if o == "f16" else _abi.DTYPE_F32
                if _abi.check(v, dt, odt, m, n, k, 4096, 4096, 4096) == _abi.VK_OK:
                    out.append((os.path.basename(path)[:-4], v, o))
    return out


@pytest.mark.parametrize("name,version,out", _cases())
def test_version_on_golden(gpu, name, version, out):
    with np.load(os.path.join(HERE, "golden", name + ".npz"), allow_pickle=False) as z:
        A, B, exact = z["A"], z["B"], z["exact_f64"]
        v0_f32 = z["v0_f32"]
    C = run_gemm(version, A, B, out)
    integer = "_int" in name
    if integer and (out == "f32" or np.abs(exact).max() <= 2048):
        assert np.array_equal(C.astype(np.float64), exact)
    elif out == "f32":
        check_f32_out(C, A, B, exact)
    else:
        check_f16_out(C, A, B, exact)
    if A.dtype == np.float32 and version == 1:
        assert np.array_equal(C.view(np.uint32), v0_f32.view(np.uint32))
