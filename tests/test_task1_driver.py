"""The task1.sh driver flow (build + run + log) on the CPU version 0, checked
against the reference's log layout
(results/ralph_loop_fable/logs/task1_float16_v19_20260610_082246.log:1-11 of
the reference; command surface CLAUDE_For_KernelAgent.md:37-43):

    Run started at: <date -u>
    FLOAT_TYPE: float32
    VERSION: 0
    ======================================
    [Playground] Start Testing for GEMM Version 0 with DType float32 ...
    [Playground] Calculating Finished
    [Playground] Result >>> TFLOPS: <x>; Average Error: <y>
    ======================================
    Run completed at: <date -u>
    Log saved to: logs/task1_float32_v0_<YYYYmmdd_HHMMSS>.log
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "vibekernel_amd", "harness")
DATE_RE = r"[A-Z][a-z]{2} [A-Z][a-z]{2} [ 0-9]\d \d\d:\d\d:\d\d UTC \d{4}"


@pytest.mark.parametrize("flt,dt", [("f32", "float32"), ("f16", "float16")])
def test_task1_run_log_layout(flt, dt):
    env = dict(os.environ, LC_ALL="C")
    p = subprocess.run([os.path.join(HARNESS, "task1.sh"), "run", "--float", flt, "--ver", "0", "--",
                        "-m", "128", "-n", "96", "-k", "64"], capture_output=True, text=True, timeout=600,
                       env=env)
    assert p.returncode == 0, p.stdout + p.stderr
    lines = p.stdout.rstrip("\n").split("\n")
    assert len(lines) == 10, lines
    assert re.fullmatch("Run started at: " + DATE_RE, lines[0]), lines[0]
    assert lines[1] == f"FLOAT_TYPE: {dt}"
    assert lines[2] == "VERSION: 0"
    assert lines[3] == "=" * 38 == lines[7]
    assert lines[4] == f"[Playground] Start Testing for GEMM Version 0 with DType {dt} ..."
    assert lines[5] == "[Playground] Calculating Finished"
    # the reference's own parser (results/parse_run.sh:58-59)
    m = re.search(r"TFLOPS: ([0-9.eE+-]+); *Average Error: ([0-9.eE+-]+)", lines[6])
    assert m and float(m.group(1)) > 0 and float(m.group(2)) == 0.0
    assert re.fullmatch("Run completed at: " + DATE_RE, lines[8]), lines[8]
    lm = re.fullmatch(rf"Log saved to: (logs/task1_{dt}_v0_\d{{8}}_\d{{6}}\.log)", lines[9])
    assert lm, lines[9]
    log = os.path.join(HARNESS, lm.group(1))
    try:
        with open(log) as f:
            assert f.read() == p.stdout  # the log is exactly what was printed
    finally:
        os.remove(log)


def test_task1_usage_errors():
    sh = os.path.join(HARNESS, "task1.sh")
    assert subprocess.run([sh, "run", "--float", "f64"], capture_output=True).returncode == 2
    assert subprocess.run([sh, "bogus"], capture_output=True).returncode == 2
    assert subprocess.run([sh, "run", "--nope"], capture_output=True).returncode == 2
