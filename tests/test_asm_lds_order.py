"""Device-assembly checks of every HIP kernel in libvk_gemm.so (gfx950,
compiled here with the library's flags to a temporary directory): no
instruction reads a VGPR that an LDS read is still writing, and every
LDS-DMA load has its wait state after an M0 write.

The fragment reads of the matrix-core kernels are inline asm
(lds_read_h8_off / lds_read_tr16_off in vk_device.hpp), which the compiler
does not track: their results must be consumed only after an
s_waitcnt lgkmcnt(N) that retires them, or an s_barrier (the kernels'
lds_barrier waits lgkmcnt(0) first).  A register copy the compiler inserts
between such a read and the wait -- as a branch on the phase in a k-loop
once produced -- reads stale data, with no error and results that pass or
fail with timing.  The scan follows each kernel in program order, keeps the
pending LDS operations as an in-order queue (lgkmcnt(N) leaves the N most
recent), and flags any read of a pending destination.  It is exact for the
straight-line k-loop bodies; across branches it follows the fall-through
path.  The scanner itself is pinned on small hand-written sequences.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "vibekernel_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S"]


def _regs(spec):
    spec = spec.split()[0] if spec else ""
    m = re.match(r"v\[(\d+):(\d+)\]$", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", spec)
    return {int(m.group(1))} if m else set()


def scan(text):
    """{kernel: [(instruction, registers)]} of reads of pending LDS results."""
    out = {}
    cur = None
    fifo = []
    for line in text.splitlines():
        t = line.strip()
        m = re.match(r"^(_Z\S+):", t)
        if m:
            cur, fifo = m.group(1), []
            out[cur] = []
            continue
        if cur is None or not t or t[0] in ";.":
            continue
        op = t.split()[0]
        if op == "s_endpgm":
            cur = None
            continue
        if op == "s_barrier":
            fifo = []
            continue
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", t)
            if m:
                del fifo[:max(0, len(fifo) - int(m.group(1)))]
            elif t == "s_waitcnt 0":
                fifo = []
            continue
        args = [a.strip() for a in t[len(op):].split(",")]
        if op.startswith("ds_read"):
            srcs = args[1:]
        elif op.startswith("ds_"):
            srcs = args
        elif op.startswith("s_"):
            srcs = []
        else:
            srcs = args[1:]
        used = set()
        for a in srcs:
            used |= _regs(a)
        pending = set().union(*fifo) if fifo else set()
        if used & pending:
            out[cur].append((t, sorted(used & pending)))
        if op.startswith("ds_"):
            fifo.append(_regs(args[0]) if op.startswith("ds_read") else set())
        elif op.startswith("v_") and args:
            written = _regs(args[0])
            fifo = [f - written for f in fifo]
    return out


def m0_hazards(text):
    """LDS-DMA loads (global_load_lds_*, buffer_load_* ... lds) issued right
    after an SALU write of M0, which on the GFX9 family needs one wait state
    between them (the kernels' inline asm puts an s_nop 0 there)."""
    bad = []
    prev = ""
    for line in text.splitlines():
        t = line.strip()
        if not t or t[0] in ";." or t.endswith(":"):
            continue
        op = t.split()[0]
        dma = op.startswith("global_load_lds") or (op.startswith("buffer_load") and t.endswith(" lds"))
        if dma and prev.startswith("s_") and prev.split()[1:2] == ["m0,"]:
            bad.append((prev, t))
        prev = t
    return bad


def test_m0_scanner():
    assert m0_hazards("\ts_mov_b32 m0, s4\n\tglobal_load_lds_dwordx4 v1, s[2:3]")
    assert not m0_hazards("\ts_mov_b32 m0, s4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[2:3]")
    assert m0_hazards("\ts_mov_b32 m0, s4\n\tbuffer_load_dwordx4 v1, s[4:7], s8 offen lds")


def test_scanner_flags_a_read_before_the_wait():
    bad = """_Zk:
\tds_read_b128 v[4:7], v1 offset:0
\tds_read_b128 v[8:11], v1 offset:16
\tv_mov_b64_e32 v[20:21], v[4:5]
\ts_endpgm"""
    assert scan(bad)["_Zk"] and scan(bad)["_Zk"][0][1] == [4, 5]


def test_scanner_accepts_waits_and_barriers():
    ok = """_Zk:
\tds_read_b128 v[4:7], v1 offset:0
\tds_read_b128 v[8:11], v1 offset:16
\ts_waitcnt lgkmcnt(1)
\tv_mov_b64_e32 v[20:21], v[4:5]
\ts_waitcnt lgkmcnt(0)
\tv_add_u32_e32 v30, v8, v9
\tds_read_b64_tr_b16 v[12:13], v2 offset:0
\ts_barrier
\tv_mfma_f32_16x16x32_f16 v[40:43], v[12:15], v[4:7], v[40:43]
\ts_endpgm"""
    assert scan(ok) == {"_Zk": []}
    # lgkmcnt(1) retires only the older of two reads
    early = ok.replace("v_mov_b64_e32 v[20:21], v[4:5]", "v_mov_b64_e32 v[20:21], v[8:9]")
    assert scan(early)["_Zk"]


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not found")
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    d = tmp_path_factory.mktemp("asm")
    procs = []
    for f in srcs:
        out = str(d / (f[:-4] + ".s"))
        procs.append((f, out, subprocess.Popen([HIPCC] + FLAGS + [os.path.join(CSRC, f), "-o", out],
                                               stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)))
    texts = {}
    for f, out, p in procs:
        _, err = p.communicate(timeout=600)
        assert p.returncode == 0, err.decode()[-2000:]
        texts[f] = open(out).read()
    return texts


def test_no_kernel_reads_an_unretired_lds_result(device_asm):
    found = {}
    kernels = 0
    for f, text in device_asm.items():
        for k, hits in scan(text).items():
            kernels += 1
            if hits:
                found[f"{f}: {k}"] = hits[:3]
    assert kernels > 40  # every kernel instance of the library was scanned
    assert not found, found


def test_m0_wait_state_before_every_lds_dma(device_asm):
    found = {f: m0_hazards(text)[:3] for f, text in device_asm.items() if m0_hazards(text)}
    assert not found, found
