"""C ABI of libvk_gemm.so, checked without a GPU: the library loads, exports
every entry point include/vk_gemm.h declares, and validates arguments the way
the header documents (no kernel is launched by any of these calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    text = open(os.path.join(ROOT, "include", "vk_gemm.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vk_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    from vibekernel_amd import _abi
    L = _abi.load()
    declared = _header_functions()
    assert declared, "no declarations parsed"
    for fn in declared:
        assert hasattr(L, fn), f"{fn} declared in include/vk_gemm.h but not exported"
    assert sorted(_abi.EXPORTED_SYMBOLS) == declared


def test_abi_version_and_registry():
    from vibekernel_amd import _abi
    assert _abi.abi_version() == 1
    f16 = _abi.versions(_abi.DTYPE_F16)
    f32 = _abi.versions(_abi.DTYPE_F32)
    assert 1 in f16 and 2 in f16 and 1 in f32
    assert 0 not in f16  # v0 (CPU ground truth) lives with the harness, not here
    for v in f16:
        assert _abi.name(v, _abi.DTYPE_F16).startswith(f"f16_v{v}_")
    assert _abi.name(99, _abi.DTYPE_F16) is None


F16, F32 = 1, 2
P = 1 << 20  # a 16-byte-aligned fake address: vk_gemm_check never dereferences


@pytest.mark.parametrize("args,expected", [
    ((2, F16, F16, 4096, 4096, 4096, P, P, P), 0),
    ((2, F16, F32, 4096, 4096, 4096, P, P, P), 0),
    ((2, F16, F16, 4096, 4096, 4000, P, P, P), -3),    # k % 64
    ((2, F16, F16, 4000, 4096, 4096, P, P, P), -3),    # m % 256
    ((2, F16, F16, 4096, 4096, 4096, P + 2, P, P), -4),  # A misaligned
    ((2, F16, F16, 4096, 4096, 4096, 0, P, P), -5),    # NULL A
    ((2, F16, F16, 0, 4096, 4096, 0, 0, 0), 0),        # empty: nothing to write
    ((2, F16, F16, 256, 256, 0, 0, 0, P), 0),          # k == 0: C := 0, A/B unused
    ((2, F16, F16, 256, 256, 0, 0, 0, 0), -5),         # k == 0 still needs C
    ((42, F16, F16, 256, 256, 256, P, P, P), -1),      # unknown version
    ((1, F32, F16, 256, 256, 256, P, P, P), -2),       # f32 in, f16 out unsupported
    ((1, F16, 7, 256, 256, 256, P, P, P), -2),         # bad dtype code
    ((1, F16, F16, 17, 33, 65, P + 2, P + 4, P + 6), 0),  # v1: any shape, 2-byte aligned
    ((1, F16, F16, 2 ** 31, 1, 1, P, P, P), -8),       # beyond 32-bit indexing
    ((10, F16, F16, 4000, 4000, 4000, P, P, P), 0),    # v10: any m, n and k multiples of 8
    ((10, F16, F32, 1, 8, 8, P, P, P), 0),
    ((10, F16, F16, 4000, 4004, 4000, P, P, P), -3),   # n % 8
    ((10, F16, F16, 4000, 4000, 4100, P, P, P), -3),   # k % 8
    ((10, F16, F16, 4000, 4000, 4000, P + 8, P, P), -4),  # 16-byte rows
    ((3, F32, F32, 1000, 1000, 1000, P, P, P), 0),     # f32 v3: any m, n and k multiples of 4
    ((3, F32, F32, 1000, 1002, 1000, P, P, P), -3),
])
def test_vk_gemm_check(args, expected):
    from vibekernel_amd import _abi
    assert _abi.check(*args) == expected


def test_status_strings():
    from vibekernel_amd import _abi
    for code in range(-8, 1):
        s = _abi.status_string(code)
        assert s and s != "unknown status"
    assert _abi.status_string(-99) == "unknown status"


def test_caps_consistent():
    from vibekernel_amd import _abi
    for v in _abi.versions(_abi.DTYPE_F16):
        c = _abi.query(v, _abi.DTYPE_F16)
        assert c.version == v and c.lds_bytes <= 160 * 1024 and c.threads % 64 == 0
        assert _abi.DTYPE_F16 in c.out_dtypes
    with pytest.raises(_abi.VkError):
        _abi.query(123, _abi.DTYPE_F16)


def test_workspace_bytes_zero_for_plain_versions():
    from vibekernel_amd import _abi
    for v in _abi.versions(_abi.DTYPE_F16):
        c = _abi.query(v, _abi.DTYPE_F16)
        if not c.uses_workspace:
            assert _abi.workspace_bytes(v, _abi.DTYPE_F16, 4096, 4096, 4096) == 0


def test_splittail_workspace_follows_schedule():
    """Version 9 needs a workspace only where its schedule splits tiles: the
    8 KB counter block plus one 256 KB partial slot per split-tail unit (no
    device here: an MI355X's 256 CUs are assumed)."""
    from vibekernel_amd import _abi
    f16 = _abi.DTYPE_F16
    assert _abi.query(9, f16).uses_workspace == 1
    assert _abi.workspace_bytes(9, f16, 4096, 4096, 4096) == 0     # one full wave
    assert _abi.workspace_bytes(9, f16, 4096, 11008, 4096) == 0    # tail of 176 tiles: left whole
    assert _abi.workspace_bytes(9, f16, 2048, 2048, 4096) == 8192 + 256 * 256 * 1024  # 64 tiles x 4 pieces
    assert _abi.workspace_bytes(9, f16, 768, 2560, 4096) == 8192 + 120 * 256 * 1024   # 30 tiles x 4 pieces
    assert _abi.workspace_bytes(9, f16, 2560, 2560, 2048) == 0     # 100 tiles of 32 k-tiles: no gain modelled
    assert _abi.workspace_bytes(9, f16, 256, 256, 512) == 0        # 8 k-tiles: too shallow to split


def test_edge_split_plan_follows_shape():
    """Version 10 takes version 9's split tails where the plan splits, with
    the tiles and k-tiles past M, N or K counted whole."""
    from vibekernel_amd import _abi
    f16 = _abi.DTYPE_F16
    assert _abi.query(10, f16).uses_workspace == 1
    assert _abi.workspace_bytes(10, f16, 4000, 4000, 4000) == 0   # 256 tiles: one full wave
    assert _abi.workspace_bytes(10, f16, 1000, 1000, 1000) == 0   # 16 k-tiles: too shallow to split
    assert _abi.workspace_bytes(10, f16, 1000, 1000, 4000) == 8192 + 64 * 256 * 1024  # 16 tiles x 4 pieces
    assert _abi.workspace_bytes(10, f16, 4096, 4096, 4096) == 0


def test_f32_split_workspace_follows_shape():
    """fp32 versions 2 and 3 take 128 x 128 tiles unless 256 x 256 ones fill
    the CUs in as few rounds, 64 x 64 tiles where the 128 x 128 ones are
    fewer than the CUs, and split K (pieces of at least 2 k-tiles of 32)
    where the chosen tiles fill at most half of the CUs, or the tiles of a
    part-empty last round where version 9's schedule does: the 8 KB counter
    block plus one partial slot (the tile in fp32: 64 or 16 KB) per piece
    (256 CUs assumed)."""
    from vibekernel_amd import _abi
    f32 = _abi.DTYPE_F32
    for v in (2, 3):
        assert _abi.query(v, f32).uses_workspace == 1
        assert _abi.workspace_bytes(v, f32, 4096, 4096, 4096) == 0   # 256 tiles of 256 x 256
        assert _abi.workspace_bytes(v, f32, 2048, 2048, 2048) == 0   # 256 tiles of 128 x 128: whole
        assert _abi.workspace_bytes(v, f32, 1024, 1024, 1024) == 0   # 256 tiles of 64 x 64: whole
        assert _abi.workspace_bytes(v, f32, 1536, 1536, 1536) == 8192 + 192 * 16384  # 576 tiles of 64 x 64: 64 in the tail x 3
        assert _abi.workspace_bytes(v, f32, 512, 512, 512) == 8192 + 256 * 16384      # 64 x 64: 64 tiles x 4 pieces
        assert _abi.workspace_bytes(v, f32, 256, 256, 1024) == 8192 + 128 * 16384     # 16 tiles x 8 pieces
        assert _abi.workspace_bytes(v, f32, 4096, 4352, 4096) == 8192 + 256 * 65536  # 1088 tiles: 64 in the tail x 4
        assert _abi.workspace_bytes(v, f32, 2304, 2048, 2048) == 8192 + 128 * 65536  # 288 tiles: 32 in the tail x 4
        assert _abi.workspace_bytes(v, f32, 2304, 2304, 2048) == 8192 + 204 * 65536  # 324 tiles: 68 in the tail x 3
        assert _abi.workspace_bytes(v, f32, 2304, 2048, 1024) == 0   # 32 k-tiles: the tail left whole
        assert _abi.workspace_bytes(v, f32, 256, 256, 32) == 0       # one k-tile
        assert _abi.workspace_bytes(v, f32, 4096, 4096, 1040) == 0   # 256 tiles of 256 x 256 (eight-wave kernel)
        assert _abi.workspace_bytes(v, f32, 512, 512, 1040) == 8192 + 256 * 16384     # 33 k-tiles, the last masked
    assert _abi.workspace_bytes(3, f32, 1000, 1000, 1024) == 0       # 256 edge tiles of 64 x 64
    assert _abi.workspace_bytes(3, f32, 300, 260, 96) == 0           # 3 k-tiles: too shallow to split
    assert _abi.workspace_bytes(3, f32, 300, 260, 128) == 8192 + 50 * 16384      # 25 tiles x 2 pieces


def test_version15_takes_any_shape_with_padded_workspace():
    """Version 15 runs version 10 on copies of A, B and C whose rows are padded
    to multiples of 8 halves: any shape, a workspace of version 10's own plus
    the copies it needs (A' when K % 8, B' when N % 8 or K % 8, C' in fp32
    when N % 8), each at a 256-byte boundary (256 CUs assumed)."""
    from vibekernel_amd import _abi
    from vibekernel_amd.gemm import pick_version
    f16 = _abi.DTYPE_F16
    up = lambda x: -(-x // 256) * 256
    for shape in [(1000, 1001, 1000), (17, 33, 65), (4096, 4096, 4095), (1, 1, 1)]:
        assert _abi.check(15, f16, f16, *shape, P, P, P) == 0
        assert _abi.check(15, f16, F32, *shape, P, P, P) == 0
    assert _abi.check(15, f16, f16, 1000, 1001, 1000, P + 8, P, P) == -4  # 16-byte aligned operands
    m, n, k = 1000, 1001, 1000   # N off: B' and C'; version 10's plan for 1000 x 1008 x 1000 splits nothing
    assert _abi.workspace_bytes(10, f16, m, 1008, k) == 0
    assert _abi.workspace_bytes(15, f16, m, n, k) == up(k * 1008 * 2) + up(m * 1008 * 4)
    m, n, k = 4096, 4096, 4095  # K off: A' and B'; C goes straight to version 10
    assert _abi.workspace_bytes(15, f16, m, n, k) == up(m * 4096 * 2) + up(4096 * n * 2)
    assert _abi.workspace_bytes(15, f16, 4096, 4096, 4096) == 0  # aligned: version 10 as it is
    assert pick_version(1000, 1001, 1000) == 15 and pick_version(4096, 50257, 4096) == 15
    assert pick_version(17, 33, 65) == 1    # below 2^24 multiply-adds: version 1, no copies
    assert pick_version(1024, 1024, 1024) == 11


def test_single_hip_runtime_in_process():
    """The library must bind to the HIP runtime the process already uses
    (PyTorch's), never map a second one."""
    from vibekernel_amd import _abi
    _abi.load()
    assert len(_abi.hip_runtimes_loaded()) == 1, _abi.hip_runtimes_loaded()


def test_workspace_bytes_version14():
    """Version 14's split plan on 256 CUs: ks = the largest power of two up
    to 8 that keeps ceil(N / 64) * ks workgroups on the CUs with at least 8
    k-steps of 32 per piece, or more pieces where they fill idle CUs with at
    least 32 steps each; the workspace is 4 KB of counters plus ks pieces x
    the column blocks x 4 waves x 1 KB per 16-row block."""
    from vibekernel_amd import _abi
    f16 = _abi.DTYPE_F16
    ws = lambda m, n, k: _abi.workspace_bytes(14, f16, m, n, k)
    assert ws(128, 8192, 8192) == 4096 + 2 * 128 * 4 * 8 * 1024   # 128 column blocks x 2
    assert ws(16, 8192, 8192) == 4096 + 2 * 128 * 4 * 1 * 1024
    assert ws(64, 4096, 4096) == 4096 + 4 * 64 * 4 * 4 * 1024     # 64 x 4
    assert ws(100, 2048, 4096) == 4096 + 8 * 32 * 4 * 7 * 1024    # 32 x 8
    assert ws(64, 264, 1024) == 4096 + 4 * 5 * 4 * 4 * 1024       # 8 steps per piece at ks = 4
    assert ws(128, 16384, 4096) == 0   # 256 column blocks: one per CU already
    assert ws(96, 8192, 1056) == 4096 + 2 * 128 * 4 * 6 * 1024    # 33 steps: pieces of 16 and 17
    assert ws(1, 5120, 4096) == 4096 + 3 * 80 * 4 * 1 * 1024      # 80 x 3 = 240 workgroups, 42 steps each
    assert ws(16, 3072, 4096) == 4096 + 4 * 48 * 4 * 1 * 1024     # 5 pieces would have 25 steps
    assert ws(48, 1000, 2016) == 4096 + 4 * 16 * 4 * 3 * 1024     # 63 steps: at least 8 per piece
    assert ws(17, 72, 160) == 0        # 5 steps: fewer than 8 per piece


def test_pick_version_follows_shape():
    import vibekernel_amd as vk
    assert vk.pick_version(16, 8192, 8192) == 8
    assert vk.pick_version(16, 4096, 4096) == 14   # 2048 < N <= 4096: K split over the waves too
    assert vk.pick_version(16, 4096, 14336) == 8   # up to 32 rows with K > 12288: version 8
    assert vk.pick_version(64, 4096, 14336) == 14
    assert vk.pick_version(128, 3072, 2048) == 14
    assert vk.pick_version(128, 2048, 8192) == 14  # N <= 2048 from 65 rows
    assert vk.pick_version(96, 4096, 8192) == 14   # 65-128 rows: K up to 8192
    assert vk.pick_version(128, 4096, 11264) == 8
    assert vk.pick_version(1, 1536, 8192) == 14    # up to 8 rows at 1024 < N <= 2048, K <= 8192
    assert vk.pick_version(16, 2048, 8192) == 8
    assert vk.pick_version(1, 1024, 2048) == 8
    assert vk.pick_version(160, 4096, 4096) == 11  # from 129 rows: 128 x 128 tiles where they suit
    assert vk.pick_version(64, 2048, 8192) == 8
    assert vk.pick_version(16, 1024, 2048) == 8
    assert vk.pick_version(1, 5120, 4096) == 8     # 80 column blocks of 64 x 2 pieces: CUs idle
    assert vk.pick_version(16, 4104, 4096) == 8    # just past N = 4096
    assert vk.pick_version(16, 8224, 8192) == 8  # n % 128 != 0: the last column block cut short
    assert vk.pick_version(16, 8220, 8192) == 15  # n % 8 != 0: version 10 on padded copies
    assert vk.pick_version(128, 8192, 8192) == 8  # batch-128 decode: still the split-K kernel
    assert vk.pick_version(144, 8192, 8192) == 11  # from 129 rows: 128 x 128 tiles where they suit
    assert vk.pick_version(1, 8192, 8192) == 8    # one row: the same kernel, rows past M read as zeros
    assert vk.pick_version(256, 8192, 8192) == 11  # 128 x 128 tiles, K split over idle CUs
    assert vk.pick_version(192, 4096, 4096) == 11
    assert vk.pick_version(136, 14336, 4096) == 11
    assert vk.pick_version(192, 28672, 8192) == 8  # 448 tiles of 128 x 128 off the grid: over 1.5 waves
    assert vk.pick_version(300, 8192, 8192) == 11  # beyond 256 rows, off the grid: 192 tiles of 128 x 128
    assert vk.pick_version(4096, 4096, 4096) == 7  # 256 tiles: one full wave
    assert vk.pick_version(4096, 4096, 4096, "f16", "f32") == 7
    assert vk.pick_version(4096, 11008, 4096) == 7  # 688 tiles = 2.69 waves: tail left whole
    assert vk.pick_version(2048, 2048, 4096) == 11  # 64 tiles of 256 x 256, 256 of 128 x 128: one wave
    assert vk.pick_version(512, 512, 512) == 11     # 16 tiles of 128 x 128 where 256 x 256 gives 4, no split
    assert vk.pick_version(1024, 1024, 8192) == 11  # 64 tiles of 128 x 128, K split 4 ways over the idle CUs
    assert vk.pick_version(512, 512, 8192) == 11    # 16 tiles of 128 x 128, K split 8 ways
    assert vk.pick_version(3840, 4096, 4096) == 7   # 240 of 256 CUs busy: not worth a split
    assert vk.pick_version(4096, 4096, 4128) == 10  # k % 64 != 0: v7 with a masked last k-tile
    assert vk.pick_version(100, 300, 70) == 1
    assert vk.pick_version(4000, 4000, 4000) == 10  # off the 256 x 256 x 64 grid: v7 with edges
    assert vk.pick_version(1000, 1000, 1000) == 11  # 64 tiles of 128 x 128 with edges
    assert vk.pick_version(2600, 2600, 72) == 10    # 441 tiles of 128 x 128: over 1.5 waves
    assert vk.pick_version(512, 512, 512, "f32") == 2   # fp32 on the matrix cores
    assert vk.pick_version(500, 512, 512, "f32") == 3   # m % 256 != 0: the matrix cores with edges
    assert vk.pick_version(500, 510, 512, "f32") == 1   # n % 4 != 0: the VALU kernel


def test_pick_version_raises_when_no_version_accepts():
    """No version takes fp32 input with fp16 output, and none takes a shape
    whose 32-bit offsets overflow: the pick raises VkError (status -3), not a
    None that the C-ABI call would reject with a ctypes error."""
    import vibekernel_amd as vk
    with pytest.raises(vk.VkError) as e:
        vk.pick_version(256, 256, 256, "f32", "f16")
    assert e.value.status == -3
    with pytest.raises(vk.VkError):
        vk.pick_version(1 << 24, 3, 4096)  # A alone beyond 2^31 bytes


def test_leave_one_out_instances_registered():
    """fp16 71-77 are version 7 with one ingredient off: listed by the
    library, named after version 7, accepting exactly version 7's shapes, and
    left out of vibekernel_amd.versions() and the pick unless asked for."""
    import vibekernel_amd as vk
    from vibekernel_amd import _abi
    text = open(os.path.join(ROOT, "include", "vk_gemm.h")).read()
    first = int(re.search(r"#define VK_F16_LEAVE_ONE_OUT_FIRST (\d+)", text).group(1))
    last = int(re.search(r"#define VK_F16_LEAVE_ONE_OUT_LAST (\d+)", text).group(1))
    assert list(_abi.LEAVE_ONE_OUT) == list(range(first, last + 1))
    lib = _abi.versions(_abi.DTYPE_F16)
    c7 = vk.query(7)
    for v in _abi.LEAVE_ONE_OUT:
        assert v in lib
        assert _abi.name(v, _abi.DTYPE_F16).startswith(f"f16_v{v}_v7_")
        c = vk.query(v)
        for f in ("div_m", "div_n", "div_k", "max_m", "align_bytes", "tile", "threads", "out_dtypes",
                  "uses_workspace", "tolerance_tier"):
            assert getattr(c, f) == getattr(c7, f), (v, f)
        assert c.lds_bytes <= 160 * 1024
        for shape in ((4096, 4096, 4096), (256, 256, 64), (4096, 4096, 4000), (4000, 4096, 4096)):
            assert _abi.check(v, F16, F16, *shape, P, P, P) == _abi.check(7, F16, F16, *shape, P, P, P)
        assert v not in vk.versions("f16")
        assert v in vk.versions("f16", leave_one_out=True)
    assert vk.pick_version(4096, 4096, 4096) == 7


def test_timeline_build_is_separate():
    """The measurement build (libvk_gemm_timeline.so) exports the timestamp
    reader; the product library does not carry it."""
    import subprocess
    lib = os.path.join(ROOT, "vibekernel_amd", "lib")
    prod = subprocess.run(["nm", "-D", os.path.join(lib, "libvk_gemm.so")], capture_output=True, text=True).stdout
    tl = subprocess.run(["nm", "-D", os.path.join(lib, "libvk_gemm_timeline.so")], capture_output=True,
                        text=True).stdout
    assert " T vk_gemm" in prod and " T vk_gemm" in tl
    assert "vk_timeline_read" not in prod
    assert " T vk_timeline_read" in tl
