"""The task1 harness layer without a GPU: the product's version 0 (libvk_v0.so)
against the oracle, the per-version binaries' command line and result line,
the handwritten-kernel scanner, and the harness C ABIs' exported symbols."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "vibekernel_amd", "harness")
LIB = os.path.join(ROOT, "vibekernel_amd", "lib")
# results/parse_run.sh:58-59 of the reference
RESULT_RE = re.compile(r"TFLOPS: (?P<tf>[0-9.eE+-]+); *Average Error: (?P<err>[0-9.eE+-]+)")


@pytest.fixture(scope="module")
def v0():
    L = ctypes.CDLL(os.path.join(LIB, "libvk_v0.so"))
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    L.vk_v0_sgemm.argtypes = [sz, sz, sz, vp, vp, vp]
    L.vk_v0_hgemm.argtypes = [sz, sz, sz, vp, vp, vp]
    L.vk_v0_threads.restype = ctypes.c_int
    return L


def _v0_sgemm(L, A, B):
    m, k = A.shape
    n = B.shape[1]
    C = np.empty((m, n), np.float32)
    L.vk_v0_sgemm(m, n, k, A.ctypes.data, B.ctypes.data, C.ctypes.data)
    return C


def _v0_hgemm(L, A, B):
    m, k = A.shape
    n = B.shape[1]
    C = np.empty((m, n), np.uint16)
    L.vk_v0_hgemm(m, n, k, A.view(np.uint16).ctypes.data, B.view(np.uint16).ctypes.data, C.ctypes.data)
    return C.view(np.float16)


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (6, 16, 3), (7, 17, 300), (130, 70, 513), (256, 256, 256),
                                   (73, 2100, 260)])
def test_v0_sgemm_equals_oracle(v0, oracle, m, n, k):
    # Same per-element operation sequence (fma over ascending k from +0), so
    # the packed AVX2 kernel and the plain-C oracle agree bit for bit.
    rng = np.random.default_rng(m + n + k)
    A = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    B = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    assert np.array_equal(_v0_sgemm(v0, A, B).view(np.uint32), oracle.sgemm(A, B).view(np.uint32))


@pytest.mark.parametrize("m,n,k", [(5, 9, 33), (64, 64, 64), (129, 257, 130)])
def test_v0_hgemm_equals_oracle(v0, oracle, m, n, k):
    rng = np.random.default_rng(7 * m + k)
    A = rng.standard_normal((m, k)).astype(np.float16)
    B = rng.standard_normal((k, n)).astype(np.float16)
    assert np.array_equal(_v0_hgemm(v0, A, B).view(np.uint16), oracle.hgemm(A, B).view(np.uint16))


def test_v0_k_zero_and_integer_kat(v0):
    C = _v0_sgemm(v0, np.zeros((3, 0), np.float32), np.zeros((0, 4), np.float32))
    assert np.all(C == 0)
    rng = np.random.default_rng(2)
    A = rng.integers(-8, 9, (40, 50))
    B = rng.integers(-8, 9, (50, 30))
    assert np.array_equal(_v0_sgemm(v0, A.astype(np.float32), B.astype(np.float32)).astype(np.int64), A @ B)


def _run(binary, *args, check=True):
    p = subprocess.run([os.path.join(HARNESS, "bin", binary), *args], capture_output=True, text=True,
                       timeout=120)
    if check:
        assert p.returncode == 0, p.stderr
    return p


@pytest.mark.parametrize("binary", ["task1_float16_v0", "task1_float32_v0"])
def test_task1_v0_result_line(binary):
    p = _run(binary, "-m", "96", "-n", "80", "-k", "64", "--dist", "uniform")
    lines = p.stdout.strip().splitlines()
    dt = "float16" if "16" in binary else "float32"
    assert lines[0] == f"[Playground] Start Testing for GEMM Version 0 with DType {dt} ..."
    assert lines[1] == "[Playground] Calculating Finished"
    m = RESULT_RE.search(lines[2])
    assert m and float(m.group("tf")) > 0
    assert float(m.group("err")) == 0.0  # v0 against its own ground truth, as in the reference


def test_task1_json_and_seed_reproducible():
    a = _run("task1_float32_v0", "-m", "64", "-n", "64", "-k", "64", "--json", "--seed", "5").stdout
    b = _run("task1_float32_v0", "-m", "64", "-n", "64", "-k", "64", "--json", "--seed", "5").stdout
    ja = [ln for ln in a.splitlines() if ln.startswith("{")][0]
    assert '"iters": 10' in ja and '"version": 0' in ja  # the CPU path is forced to 10 rounds
    assert a.splitlines()[2].split("Average Error:")[1] == b.splitlines()[2].split("Average Error:")[1]


def test_task1_cli_errors():
    assert _run("task1_float16_v0", "--bogus", check=False).returncode != 0
    assert _run("task1_float16_v0", "-m", "x", check=False).returncode != 0
    assert _run("task1_float16_v0", "--dist", "cauchy", check=False).returncode != 0
    h = _run("task1_float16_v0", "-h")
    assert "--n_warmup" in h.stdout and "--n_test" in h.stdout


def test_gpu_binaries_exist_per_version():
    import vibekernel_amd as vk
    for v in vk.versions("f16"):
        assert os.path.exists(os.path.join(HARNESS, "bin", f"task1_float16_v{v}"))
    for v in vk.versions("f32"):
        assert os.path.exists(os.path.join(HARNESS, "bin", f"task1_float32_v{v}"))


def test_check_handwritten_passes():
    p = subprocess.run([os.path.join(HARNESS, "check_handwritten.sh")], capture_output=True, text=True)
    assert p.returncode == 0, p.stdout


def test_check_handwritten_flags_a_library(tmp_path):
    # a fake kernel tree that includes a GEMM library must be rejected
    (tmp_path / "csrc").mkdir()
    (tmp_path / "csrc" / "k.hip").write_text('#include <rocblas/rocblas.h>\n')
    p = subprocess.run([os.path.join(HARNESS, "check_handwritten.sh"), str(tmp_path)], capture_output=True,
                       text=True)
    assert p.returncode == 1


def _decls(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vkb?_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("vk_v0.h", "libvk_v0.so"), ("vk_bench.h", "libvk_bench.so")])
def test_harness_abi_exports(header, lib):
    import vibekernel_amd as vk
    vk.load()  # the bench library depends on libvk_gemm.so and the HIP runtime
    L = ctypes.CDLL(os.path.join(LIB, lib))
    decls = _decls(header)
    assert decls
    for fn in decls:
        assert hasattr(L, fn), f"{fn} declared in include/{header} but not exported by {lib}"
