"""The task1 binaries for GPU versions, end to end on the GPU: reference
result line, error statistic against the binary's own v0 ground truth, and
the C++ timing loops behind bench.py (include/vk_bench.h)."""
import ctypes
import os
import re
import subprocess

import pytest

from gpu_util import announce

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "vibekernel_amd", "harness", "bin")
RESULT_RE = re.compile(r"TFLOPS: (?P<tf>[0-9.eE+-]+); *Average Error: (?P<err>[0-9.eE+-]+)")


@pytest.mark.parametrize("binary,shape,bound", [
    ("task1_float16_v1", (512, 512, 512), 2e-4),
    ("task1_float16_v2", (1024, 512, 256), 2e-4),
    ("task1_float16_v3", (1024, 1024, 1024), 2e-4),
    ("task1_float16_v4", (32, 1024, 2048), 2e-4),
    ("task1_float16_v5", (1024, 768, 512), 2e-4),
    ("task1_float16_v6", (768, 1024, 320), 2e-4),
    ("task1_float16_v7", (1024, 768, 576), 2e-4),
    ("task1_float16_v8", (48, 1024, 2048), 2e-4),
    ("task1_float16_v9", (768, 2560, 2048), 2e-4),
    ("task1_float16_v10", (1000, 1000, 1000), 2e-4),
    ("task1_float16_v11", (512, 4096, 2048), 2e-4),
    ("task1_float16_v12", (1000, 1000, 1000), 2e-4),
    ("task1_float16_v13", (768, 1024, 2048), 2e-4),
    ("task1_float16_v14", (96, 4096, 4096), 2e-4),
    ("task1_float16_v15", (1000, 1001, 999), 2e-4),
    ("task1_float32_v1", (512, 384, 256), 1e-6),
    ("task1_float32_v2", (512, 512, 256), 1e-5),
    ("task1_float32_v3", (1000, 1000, 1000), 1e-5),
])
def test_task1_gpu_binary(gpu, binary, shape, bound):
    m, n, k = shape
    announce(f"{binary} -m {m} -n {n} -k {k}")
    p = subprocess.run([os.path.join(BIN, binary), "-m", str(m), "-n", str(n), "-k", str(k), "-w", "2",
                        "-t", "5", "--json"], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    res = RESULT_RE.search(p.stdout)
    assert res, p.stdout
    assert float(res.group("tf")) > 0
    assert float(res.group("err")) < bound
    assert '"iters": 5' in p.stdout


def test_bench_loops(gpu):
    import torch
    import vibekernel_amd as vk
    import bench
    L = bench.load_bench_lib()
    m = n = k = 1024
    A = torch.rand((m, k), device="cuda:0").half()
    B = torch.rand((k, n), device="cuda:0").half()
    C = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    call = (3, vk.DTYPE_F16, vk.DTYPE_F16, m, n, k, ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(B.data_ptr()),
            ctypes.c_void_p(C.data_ptr()), s)
    per = (ctypes.c_float * 7)()
    announce("bench loops v3 1024^3")
    assert L.vkb_reference_loop(*call, 2, 7, per) == 0
    assert all(x > 0 for x in per)
    tot = ctypes.c_float(0)
    assert L.vkb_back_to_back(*call, 5, ctypes.byref(tot)) == 0 and tot.value > 0
    tot = ctypes.c_float(0)
    assert L.vkb_stream_loop(*call, 2, 5, ctypes.byref(tot)) == 0 and tot.value > 0
    assert L.vkb_stream_loop(*call, 0, 0, ctypes.byref(tot)) == -3  # no timed launches: rejected
    ref = torch.matmul(A.float(), B.float())
    # fp16 output: within half an fp16 ulp (2^-11 relative) plus fp32 noise
    assert float(((C.float() - ref).abs() / ref.abs().clamp_min(1.0)).max()) < 1e-3
    # an invalid call reports its status instead of launching
    bad = (3, vk.DTYPE_F16, vk.DTYPE_F16, 1000, n, k) + call[6:]
    assert L.vkb_reference_loop(*bad, 0, 1, per) == -3


def test_task1_printed_error_equals_oracle_statistic(gpu, oracle, tmp_path):
    """The 'Average Error' a GPU binary prints is the oracle's statistic of
    the same GT and C (--dump writes them), bit for bit, and nonzero; GT is
    the oracle's v0 result bit for bit; the --json line carries the clock
    sampled over the timed loop, the CU count and the host cores."""
    import json

    import numpy as np

    from gpu_util import check_f16_out
    from test_stat_parity import _read_dump
    dump = str(tmp_path / "v7.bin")
    announce("task1_float16_v7 -m 512 -n 768 -k 1024 --dump")
    p = subprocess.run([os.path.join(BIN, "task1_float16_v7"), "-m", "512", "-n", "768", "-k", "1024", "-w", "2",
                        "-t", "20", "--json", "--dump", dump], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    A, B, GT, C = _read_dump(dump)
    assert np.array_equal(GT.view(np.uint16), oracle.hgemm(A, B).view(np.uint16))
    exact = A.astype(np.float64) @ B.astype(np.float64)
    check_f16_out(C, A, B, exact)
    printed = np.float32(RESULT_RE.search(p.stdout).group("err"))
    v, st = oracle.mean_rel_err(GT, C)
    assert st == oracle.STATUS_OK and printed > 0
    assert printed.view(np.uint32) == np.float32(v).view(np.uint32)
    j = json.loads([ln for ln in p.stdout.splitlines() if ln.startswith("{")][0])
    assert j["cus"] > 0 and j["host_cores"] > 0 and 0 < j["pct_peak"] < 100
    clk = j["clock"]
    print("task1 clock record:", clk)
    assert clk is not None and ("error" in clk or (clk["sclk_mhz"] > 0 and 0 < clk["frac_clock"] <= 1.05))
