"""In-tree build of every native artefact (no JIT cache, no pip install).

* libvk_gemm.so  -- vibekernel_amd/csrc/Makefile (hipcc --offload-arch=gfx950)
* libvk_gemm_timeline.so -- the same with version 7's per-workgroup timestamps
  (measurement only: vibekernel_amd/harness/timeline.py)
* task1 harness   -- vibekernel_amd/harness/Makefile (binaries per version)
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
HARNESS = os.path.join(HERE, "harness")


def _make(path: str, jobs: int = 8, force: bool = True, target: str = "all") -> None:
    if not os.path.exists(os.path.join(path, "Makefile")):
        return
    cmd = ["make", "-C", path, f"-j{jobs}", target]
    if force:
        cmd.insert(3, "-B")
    subprocess.run(cmd, check=True)


def build_library(force: bool = True) -> str:
    _make(CSRC, force=force)
    lib = os.path.join(HERE, "lib", "libvk_gemm.so")
    if not os.path.exists(lib):
        raise RuntimeError("libvk_gemm.so was not produced")
    # the measurement build with per-workgroup timestamps (timeline.py)
    _make(CSRC, force=force, target="timeline")
    return lib


def build_harness(force: bool = True) -> None:
    _make(HARNESS, force=force)


def build_all(force: bool = True) -> None:
    build_library(force)
    build_harness(force)
