"""The error statistic the task1 harness prints ("Average Error",
TestData::calculateAvgErr in include/playground/test_data.hpp; the reference's
is results/naive_cycle4/include/playground/test_data.hpp:145-162) pinned bit
for bit against the oracle's restatement (oracle.mean_rel_err), and the
harness binaries' --dump / --err-legacy paths at the binary level.

tests/native/stat_check.cpp runs the product's own statistic on arrays this
test writes: equal bits for nonzero statistics, the GT == 0 skip rule, long
sequential fp32 sums, and the same aborts (non-finite C, legacy GT == 0, no
valid term) where the oracle reports a non-OK status."""
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "vibekernel_amd", "harness")
LIB = os.path.join(ROOT, "vibekernel_amd", "lib")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
RESULT_RE = re.compile(r"TFLOPS: (?P<tf>[0-9.eE+-]+); *Average Error: (?P<err>[0-9.eE+-]+|nan|inf)")


@pytest.fixture(scope="module")
def stat_bins(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not found")
    out = tmp_path_factory.mktemp("stat")
    bins = {}
    for dt, flag in (("f16", ["-DTEST_FLOAT16"]), ("f32", [])):
        exe = str(out / f"stat_check_{dt}")
        subprocess.run([HIPCC, "-O2", "-std=c++17", *flag, "-I" + os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "native", "stat_check.cpp"),
                        os.path.join(HARNESS, "matmul_v0.cpp"), "-L" + LIB, "-lvk_v0",
                        "-Wl,-rpath," + LIB, "-o", exe], check=True, capture_output=True, timeout=300)
        bins[dt] = exe
    return bins


def _product_stat(stat_bins, tmp_path, GT, C, legacy=False):
    dt = "f16" if GT.dtype == np.float16 else "f32"
    path = tmp_path / "io.bin"
    with open(path, "wb") as f:
        np.array([GT.size], np.uint64).tofile(f)
        GT.ravel().tofile(f)
        C.ravel().tofile(f)
    args = [stat_bins[dt], str(path)] + (["--legacy"] if legacy else [])
    p = subprocess.run(args, capture_output=True, text=True, timeout=120)
    if p.returncode != 0:
        assert "Check failed" in p.stderr, p.stderr
        return None
    tag, bits = p.stdout.split()
    assert tag == "ok"
    return np.array([int(bits, 16)], np.uint32).view(np.float32)[0]


def _oracle_stat(oracle, GT, C, legacy=False):
    v, st = oracle.mean_rel_err(GT, C, oracle.ERR_LEGACY if legacy else oracle.ERR_SKIP_ZERO)
    return (np.float32(v) if st == oracle.STATUS_OK else None), st


def _noisy(rng, GT, rel):
    return (GT.astype(np.float64) * (1 + rel * rng.standard_normal(GT.shape))).astype(GT.dtype)


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("count,rel", [(1, 1e-3), (4097, 1e-3), (100_000, 3e-2), (1 << 20, 1e-4)])
def test_statistic_bits_equal_oracle(stat_bins, oracle, tmp_path, dtype, count, rel):
    rng = np.random.default_rng(count)
    GT = rng.standard_normal(count).astype(dtype)
    C = _noisy(rng, GT, rel)
    got = _product_stat(stat_bins, tmp_path, GT, C)
    want, st = _oracle_stat(oracle, GT, C)
    assert st == oracle.STATUS_OK and want > 0
    assert got is not None and got.view(np.uint32) == want.view(np.uint32), (got, want)
    # and both are the mean relative error: within fp32 summation error of fp64
    ref = np.mean(np.abs((GT.astype(np.float64) - C) / GT.astype(np.float64)))
    assert abs(float(got) - ref) <= 1e-6 * count * ref + 1e-12


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_statistic_skips_exact_zeros(stat_bins, oracle, tmp_path, dtype):
    rng = np.random.default_rng(3)
    GT = rng.standard_normal(5000).astype(dtype)
    GT[::7] = 0
    C = _noisy(rng, GT, 1e-2)
    C[::7] = dtype(0.5)  # a nonzero C where GT == 0: skipped, not counted
    got = _product_stat(stat_bins, tmp_path, GT, C)
    want, st = _oracle_stat(oracle, GT, C)
    assert st == oracle.STATUS_OK and got.view(np.uint32) == want.view(np.uint32)
    # legacy mode: the first GT == 0 term makes the sum non-finite -> abort in
    # the product, non-OK status in the oracle
    assert _product_stat(stat_bins, tmp_path, GT, C, legacy=True) is None
    assert _oracle_stat(oracle, GT, C, legacy=True)[1] != oracle.STATUS_OK


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("bad", ["nan", "inf", "-inf"])
def test_statistic_aborts_on_non_finite_c(stat_bins, oracle, tmp_path, dtype, bad):
    rng = np.random.default_rng(4)
    GT = rng.standard_normal(300).astype(dtype)
    C = _noisy(rng, GT, 1e-3)
    C[123] = dtype(float(bad))
    assert _product_stat(stat_bins, tmp_path, GT, C) is None
    assert _oracle_stat(oracle, GT, C)[1] in (oracle.STATUS_NAN, oracle.STATUS_INF)


def test_statistic_aborts_without_a_valid_term(stat_bins, oracle, tmp_path):
    GT = np.zeros(64, np.float32)
    C = np.ones(64, np.float32)
    assert _product_stat(stat_bins, tmp_path, GT, C) is None
    assert _oracle_stat(oracle, GT, C)[1] == oracle.STATUS_EMPTY


def _read_dump(path):
    with open(path, "rb") as f:
        m, n, k, esz = np.fromfile(f, np.uint32, 4)
        dt = np.float16 if esz == 2 else np.float32
        A = np.fromfile(f, dt, int(m) * int(k)).reshape(m, k)
        B = np.fromfile(f, dt, int(k) * int(n)).reshape(k, n)
        GT = np.fromfile(f, dt, int(m) * int(n)).reshape(m, n)
        C = np.fromfile(f, dt, int(m) * int(n)).reshape(m, n)
    return A, B, GT, C


def run_task1(binary, *args, check=True):
    p = subprocess.run([os.path.join(HARNESS, "bin", binary), *args], capture_output=True, text=True,
                       timeout=300)
    if check:
        assert p.returncode == 0, p.stdout + p.stderr
    return p


@pytest.mark.parametrize("binary", ["task1_float16_v0", "task1_float32_v0"])
def test_v0_binary_dump_and_printed_error(oracle, tmp_path, binary):
    dump = str(tmp_path / "run.bin")
    p = run_task1(binary, "-m", "70", "-n", "90", "-k", "50", "--dist", "uniform", "--dump", dump)
    A, B, GT, C = _read_dump(dump)
    want = oracle.hgemm(A, B) if A.dtype == np.float16 else oracle.sgemm(A, B)
    assert np.array_equal(GT.view(np.uint16 if A.dtype == np.float16 else np.uint32),
                          want.view(np.uint16 if A.dtype == np.float16 else np.uint32))
    assert np.array_equal(C, GT)  # v0 measured against its own ground truth, as in the reference
    printed = np.float32(RESULT_RE.search(p.stdout).group("err"))
    v, st = oracle.mean_rel_err(GT, C)
    assert st == oracle.STATUS_OK and printed == np.float32(v) == 0


def test_legacy_flag_aborts_on_zero_ground_truth(tmp_path):
    # --dist int with k = 1: products of integers in [-2, 2], a third of them 0
    ok = run_task1("task1_float16_v0", "-m", "32", "-n", "32", "-k", "1", "--dist", "int")
    assert RESULT_RE.search(ok.stdout).group("err") == "0"
    bad = run_task1("task1_float16_v0", "-m", "32", "-n", "32", "-k", "1", "--dist", "int", "--err-legacy",
                    check=False)
    assert bad.returncode != 0 and "Check failed" in bad.stderr
    assert "Result >>>" not in bad.stdout


def test_json_line_carries_cores_and_clock_field():
    p = run_task1("task1_float32_v0", "-m", "64", "-n", "64", "-k", "64", "--json")
    import json
    j = json.loads([ln for ln in p.stdout.splitlines() if ln.startswith("{")][0])
    assert j["host_cores"] >= 1 and "clock" in j and "pct_peak" in j and "cus" in j
