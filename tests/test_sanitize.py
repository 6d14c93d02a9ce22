"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, no GPU
(tests/native/Makefile, target san): the product's version 0 and the CPU
oracle on ragged shapes (tests/native/san_cpu.cpp), the C ABI's host side --
registry, validation, query, workspace plans -- (tests/native/san_abi.cpp, the
HIP sources built with the sanitizers on their host side only), and the
split-tail schedule check (tests/native/splittail_check.cpp).  Each binary
aborts on the first report (-fno-sanitize-recover=all)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NATIVE = os.path.join(ROOT, "tests", "native")


@pytest.fixture(scope="module")
def san_dir(tmp_path_factory):
    if not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not found")
    out = str(tmp_path_factory.mktemp("san"))
    p = subprocess.run(["make", "-C", NATIVE, "-j3", "san", f"OUT={out}"], capture_output=True, text=True,
                       timeout=900)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-3000:]
    return out


@pytest.mark.parametrize("binary,expect", [("san_cpu", "ok "), ("san_abi", "ok "), ("san_splittail", "ok ")])
def test_sanitized_host_code(san_dir, binary, expect):
    env = dict(os.environ, UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               ASAN_OPTIONS="abort_on_error=1:detect_leaks=" + ("0" if binary == "san_abi" else "1"))
    # san_abi: the HIP runtime the library links keeps allocations for the
    # process's lifetime, which the leak checker would report.
    p = subprocess.run([os.path.join(san_dir, binary)], capture_output=True, text=True, timeout=600, env=env)
    assert p.returncode == 0, (p.stdout[-2000:] + p.stderr[-4000:])
    assert p.stdout.strip().splitlines()[-1].startswith(expect), p.stdout[-500:]
    assert "runtime error" not in p.stderr and "AddressSanitizer" not in p.stderr, p.stderr[-3000:]
