"""Device-assembly checks of every HIP kernel in libvk_gemm.so (gfx950,
compiled here with the library's flags to a temporary directory): no
instruction reads a VGPR that an LDS read or a memory load is still
writing, and every LDS-DMA load has its wait state after an M0 write.

The fragment reads of the matrix-core kernels are inline asm
(lds_read_h8_off / lds_read_tr16_off in vk_device.hpp), and so are the A
fragment loads of version 14 (buf_load_h8 in f16_skinny_wk.hip), which the
compiler does not track: their results must be consumed only after an
s_waitcnt lgkmcnt(N) (LDS) or vmcnt(N) (memory) that retires them, or, for
LDS reads, an s_barrier (the kernels' lds_barrier waits lgkmcnt(0) first).
A register copy the compiler inserts between such a read and the wait -- as
a branch on the phase in a k-loop once produced -- reads stale data, with no
error and results that pass or fail with timing.  The scan follows each
kernel in program order, keeps the pending LDS operations and the pending
memory operations (loads, stores and direct-to-LDS loads: gfx9 counts all of
them in vmcnt) as two in-order queues (a wait with count N leaves the N most
recent), and flags any read of a pending destination and any write into one (the
pending data would land on top of the new value) other than by a later
operation of the same counter.  It is exact for the
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


def _vmem(op):
    return op.startswith(("buffer_", "global_", "flat_", "scratch_"))


_CAP = 64  # ages beyond every counter's range


def _age(state, dests):
    """One more operation of a counter: every pending destination of it gets
    one more younger operation; the new one's destinations start at 0."""
    out = {r: min(a + 1, _CAP) for r, a in state.items()}
    for r in dests:
        out[r] = 0
    return out


def _step(t, st, hits):
    """Apply instruction t to the state (lgkm, vm): two maps register -> age
    (younger operations of the same counter issued since its operation)."""
    lg, vm = st
    op = t.split()[0]
    if op == "s_barrier":
        return {}, vm
    if op == "s_waitcnt":
        if t == "s_waitcnt 0":
            return {}, {}
        m = re.search(r"lgkmcnt\((\d+)\)", t)
        if m:
            n = int(m.group(1))
            lg = {r: a for r, a in lg.items() if a < n}
        m = re.search(r"vmcnt\((\d+)\)", t)
        if m:
            n = int(m.group(1))
            vm = {r: a for r, a in vm.items() if a < n}
        return lg, vm
    args = [a.strip() for a in t[len(op):].split(",")]
    dma = _vmem(op) and (op.startswith("global_load_lds") or t.endswith(" lds"))
    vload = _vmem(op) and "load" in op and not dma
    if op.startswith("ds_read") or vload:
        srcs = args[1:]
    elif op.startswith("ds_") or _vmem(op):
        srcs = args
    elif op.startswith("s_"):
        srcs = []
    else:
        srcs = args[1:]
    used = set()
    for a in srcs:
        used |= _regs(a)
    bad = used & (set(lg) | set(vm))
    # A register written while a load into it is pending: the load's data
    # lands afterwards.  Only a later operation of the same in-order counter
    # may write it (its data lands last).
    if op.startswith("ds_read"):
        bad |= _regs(args[0]) & set(vm)
    elif vload:
        bad |= _regs(args[0]) & set(lg)
    elif op.startswith("v_") and args:
        bad |= _regs(args[0]) & (set(lg) | set(vm))
    if bad:
        hits.append((t, sorted(bad)))
    if op.startswith("ds_"):
        lg = _age(lg, _regs(args[0]) if op.startswith("ds_read") else set())
    elif _vmem(op):
        vm = _age(vm, _regs(args[0]) if vload else set())
    return lg, vm


def _join(x, y):
    """Pending on either path, with the fewer younger operations."""
    out = dict(x)
    for r, a in y.items():
        out[r] = min(a, out[r]) if r in out else a
    return out


def _blocks(lines):
    """Basic blocks [(label, [instructions], [successor labels])] of one
    kernel's instruction lines (labels split blocks, branches end them)."""
    blocks, label, body = [], "<entry>", []
    n = 0

    def close(succ):
        nonlocal label, body, n
        blocks.append((label, body, succ))
        n += 1
        label, body = f"<after{n}>", []

    for t in lines:
        m = re.match(r"^([.\w$]+):", t)
        if m:
            if body or label.startswith("<after"):
                close([m.group(1)])
            label = m.group(1)
            continue
        body.append(t)
        op = t.split()[0]
        if op == "s_endpgm":
            close([])
        elif op == "s_branch":
            close([t.split()[1]])
        elif op.startswith("s_cbranch"):
            close([t.split()[1], None])  # None: the next block
    close([])
    out = []
    for i, (lab, body, succ) in enumerate(blocks):
        nxt = blocks[i + 1][0] if i + 1 < len(blocks) else None
        out.append((lab, body, [nxt if s is None else s for s in succ if (s is not None or nxt)]))
    return out


def scan(text):
    """{kernel: [(instruction, registers)]} of reads of pending LDS or memory
    load results, over every path of each kernel's control-flow graph."""
    kernels, cur = {}, None
    for line in text.splitlines():
        t = line.strip()
        m = re.match(r"^(_Z\S+):", t)
        if m:
            cur = m.group(1)
            kernels[cur] = []
            continue
        if cur is None:
            continue
        if t.startswith(".Lfunc_end"):
            cur = None
            continue
        if not t or t[0] == ";" or (t[0] == "." and not re.match(r"^\.L\w+:", t)):
            continue
        kernels[cur].append(t.split(";")[0].strip())
    out = {}
    for k, lines in kernels.items():
        blocks = _blocks(lines)
        index = {lab: i for i, (lab, _, _) in enumerate(blocks)}
        state_in = {0: ({}, {})}
        work = [0]
        while work:
            i = work.pop()
            st = state_in[i]
            for t in blocks[i][1]:
                st = _step(t, st, [])
            for s in blocks[i][2]:
                j = index.get(s)
                if j is None:
                    continue
                new = st if j not in state_in else (_join(state_in[j][0], st[0]), _join(state_in[j][1], st[1]))
                if j not in state_in or new != state_in[j]:
                    state_in[j] = new
                    work.append(j)
        hits = []
        for i, (_, body, _) in enumerate(blocks):
            if i not in state_in:
                continue
            st = state_in[i]
            for t in body:
                st = _step(t, st, hits)
        out[k] = hits
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


def test_scanner_tracks_memory_loads():
    ok = """_Zk:
\tbuffer_load_dwordx4 v[4:7], v1, s[8:11], s2 offen
\ts_mov_b32 m0, s5
\ts_nop 0
\tglobal_load_lds_dwordx4 v2, s[12:13]
\tbuffer_load_dwordx4 v[8:11], v1, s[8:11], s3 offen
\ts_waitcnt vmcnt(2)
\tv_mfma_f32_16x16x32_f16 v[40:43], v[4:7], v[20:23], v[40:43]
\ts_waitcnt vmcnt(0)
\tv_mfma_f32_16x16x32_f16 v[40:43], v[8:11], v[20:23], v[40:43]
\ts_endpgm"""
    assert scan(ok) == {"_Zk": []}
    # vmcnt(2) with the direct-to-LDS load counted leaves only the first load
    # retired; vmcnt(1) would not retire the second one either
    early = ok.replace("s_waitcnt vmcnt(0)", "s_waitcnt vmcnt(1)")
    assert scan(early)["_Zk"][0][1] == [8, 9, 10, 11]
    # a copy of a load's result before any wait
    copy = ok.replace("\ts_waitcnt vmcnt(2)\n", "\tv_mov_b32_e32 v30, v5\n\ts_waitcnt vmcnt(2)\n")
    assert scan(copy)["_Zk"][0][1] == [5]
    # a register reused while a load into it is pending
    waw = ok.replace("\ts_waitcnt vmcnt(2)\n", "\tv_mov_b32_e32 v9, 0\n\ts_waitcnt vmcnt(2)\n")
    assert scan(waw)["_Zk"][0][1] == [9]
    # a store counts too: issued after the second load, it lets vmcnt(1)
    # retire that load
    st = ok.replace("\ts_waitcnt vmcnt(0)", "\tglobal_store_dwordx4 v[50:51], v[60:63], off\n\ts_waitcnt vmcnt(1)")
    assert scan(st) == {"_Zk": []}


def test_scanner_follows_branches_and_loops():
    # blocks laid out out of order: the wait sits in a block placed later in
    # the text but run first
    ok = """_Zk:
\tbuffer_load_dwordx4 v[4:7], v1, s[8:11], s2 offen
\ts_branch .LBB0_2
.LBB0_1:
\tv_mfma_f32_16x16x32_f16 v[40:43], v[4:7], v[20:23], v[40:43]
\ts_endpgm
.LBB0_2:
\ts_waitcnt vmcnt(0)
\ts_branch .LBB0_1
.Lfunc_end0:"""
    assert scan(ok) == {"_Zk": []}
    assert scan(ok.replace("vmcnt(0)", "vmcnt(1)"))["_Zk"]
    # a loop whose back edge carries a load issued after the wait
    loop = """_Zk:
\ts_mov_b32 s0, 4
.LBB0_1:
\ts_waitcnt vmcnt(1)
\tv_mfma_f32_16x16x32_f16 v[40:43], v[4:7], v[20:23], v[40:43]
\tbuffer_load_dwordx4 v[4:7], v1, s[8:11], s2 offen
\ts_sub_u32 s0, s0, 1
\ts_cbranch_scc0 .LBB0_1
\ts_waitcnt vmcnt(0)
\ts_endpgm
.Lfunc_end0:"""
    assert scan(loop)["_Zk"]
    assert scan(loop.replace("vmcnt(1)", "vmcnt(0)", 1)) == {"_Zk": []}


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
