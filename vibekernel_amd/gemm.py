"""Python mirror of the reference operator interface.

Reference (paths relative to the reference repository root):
``results/naive_cycle4/include/playground/matmul.hpp:11-23``::

    template <typename DType, uint8_t Version>
    void matmul(size_t m, size_t n, size_t k, const DType* A, const DType* B, DType* C);
    #define PLAYGOUND_MATMUL_CALL(Version, m, n, k, A, B, C) \
        matmul<remove_cvref_t<decltype(*A)>, Version>(m, n, k, A, B, C)

:func:`matmul` keeps the argument order and meaning: ``m, n, k`` then row-major
``A`` (m x k), ``B`` (k x n) and the output ``C`` (m x n), which is fully
overwritten (alpha = 1, beta = 0).  As in ``PLAYGOUND_MATMUL_CALL`` the input
dtype comes from ``A``; the output dtype comes from ``C`` (fp16 as in the
reference, or fp32).  Operands are device tensors; the call is asynchronous on
the current stream (or ``stream``).  Where the reference returns void with no
error channel, this raises :class:`VkError`.

Every call goes through libvk_gemm.so; there is no other implementation.
"""
from __future__ import annotations

from . import _abi
from ._abi import DTYPE_F16, DTYPE_F32, VkError


def _torch():
    import torch  # imported lazily: the ABI layer itself does not need torch
    return torch


def _dtype_code(t) -> int:
    torch = _torch()
    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.float32:
        return DTYPE_F32
    raise VkError(-2, f"unsupported dtype {t.dtype}")


def _stream_handle(stream, device):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream(device)
    return ctypes_void_p(stream.cuda_stream)


def ctypes_void_p(v):
    import ctypes
    return ctypes.c_void_p(v)


def matmul(m: int, n: int, k: int, A, B, C, version: int, stream=None) -> None:
    """C = A . B with kernel ``version`` (row-major, fp32 accumulation)."""
    for name, t in (("A", A), ("B", B), ("C", C)):
        if not t.is_cuda:
            raise VkError(-5, f"{name} must be a device tensor")
        if not t.is_contiguous():
            raise VkError(-4, f"{name} must be contiguous (row-major, dense)")
    if A.numel() < m * k or B.numel() < k * n or C.numel() < m * n:
        raise VkError(-3, "operand smaller than m x k / k x n / m x n")
    in_dt = _dtype_code(A)
    if _dtype_code(B) != in_dt:
        raise VkError(-2, "A and B must have the same dtype")
    out_dt = _dtype_code(C)
    st = _abi.gemm(version, in_dt, out_dt, m, n, k, A.data_ptr(), B.data_ptr(), C.data_ptr(),
                   _stream_handle(stream, C.device))
    if st != _abi.VK_OK:
        raise VkError(st, f"matmul(version={version}, m={m}, n={n}, k={k})")


def gemm(A, B, version: int | None = None, out_dtype=None, stream=None):
    """Allocate C and run :func:`matmul`; A is (m, k), B is (k, n).  With no
    version, :func:`pick_version` chooses one for the shape and dtypes."""
    torch = _torch()
    m, k = A.shape
    k2, n = B.shape
    if k != k2:
        raise VkError(-3, f"inner dimensions differ: {k} vs {k2}")
    C = torch.empty((m, n), dtype=out_dtype or A.dtype, device=A.device)
    if version is None:
        dt = "f16" if A.dtype == torch.float16 else "f32"
        version = pick_version(m, n, k, dt, "f16" if C.dtype == torch.float16 else "f32")
    matmul(m, n, k, A, B, C, version, stream)
    return C


def versions(dtype: str = "f16", leave_one_out: bool = False) -> list:
    """The library's versions for an input dtype; the leave-one-out instances
    of version 7 (fp16 71-77, measurement only) only when asked for."""
    vs = _abi.versions(DTYPE_F16 if dtype == "f16" else DTYPE_F32)
    if dtype == "f16" and not leave_one_out:
        vs = [v for v in vs if v not in _abi.LEAVE_ONE_OUT]
    return vs


def name(version: int, dtype: str = "f16"):
    return _abi.name(version, DTYPE_F16 if dtype == "f16" else DTYPE_F32)


def query(version: int, dtype: str = "f16"):
    return _abi.query(version, DTYPE_F16 if dtype == "f16" else DTYPE_F32)


def _num_cus() -> int:
    """Compute units of the current device (256 on MI355X, assumed when no
    device is visible)."""
    try:
        torch = _torch()
        if torch.cuda.is_available():
            return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    except Exception:
        pass
    return 256


def pick_version(m: int, n: int, k: int, dtype: str = "f16", out: str | None = None) -> int:
    """The fastest version that accepts this shape (checked with vk_gemm_check
    on 4 KiB-aligned placeholder addresses; nothing is launched): for fp16
    the skinny kernels up to M = 128 (version 14 where it suits, else version
    8; version 4 up to 64) and version 8 from 129 to 255 rows where version 11
    does not suit, then the
    128 x 128 tiles of version 11 where they suit the grid, then the 256x256 kernels
    (fastest first; version 10 takes shapes off the 256 x 256 x 64 grid
    whose N and K are multiples of 8), then version 15 (version 10 through
    row-padded copies, for N or K off the multiples of 8, from M N K = 2^24
    on), then the any-shape kernel.  Version 11
    is taken, with T its 128 x 128 tiles on C compute units:
      * on the 256 x 256 x 64 grid, where T <= C (one wave; with 2 T <= C it
        splits K over the idle CUs itself).  Measured on MI355X, us per
        launch against version 9's split tail: 1024 x 4096 x 4096 33.6
        against 46.2 (version 7: 64.5), 1024 x 1024 x 8192 29.1 against
        43.9, 512 x 512 x 8192 19.7 against 41.7, 512 x 4096 x 4096 24.7
        against 35.1; beyond one wave 1536 x 4096 x 4096 (T = 384) took 58.7
        against 50.6;
      * off it, where T <= 3 C / 2 (version 10, whose split pieces do not stay
        on one XCD there and whose edge tiles are twice as wide, measured
        slower on every such shape: 1000 x 1000 x 1000 23.0 us against 9.8,
        2000 x 3000 x 1000 (T = 384) 25.2 against 21.2, 1000 x 1000 x 4000
        (T = 64) 36.6 against 23.0).
    From M = 129 version 11 also beats the skinny split-K version 8 wherever
    it is taken (us per launch, one box: 192 x 4096 x 4096 22.5 against
    30.2, 192 x 8192 x 8192 39.8 against 46.0, 192 x 14336 x 4096 32.9
    against 42.4, 256 x 8192 x 8192 39.8 against 55.6; another box, v11
    against v8 at N x K = 4096 x 4096 / 4096 x 8192 / 8192 x 4096 / 8192 x
    8192 / 14336 x 4096 / 4096 x 14336: M = 136 21.1 / 27.1 / 24.1 / 37.1 /
    28.9 / 37.9 against 25.9 / 31.5 / 27.0 / 37.4 / 32.8 / 39.4; M = 160
    21.1 / 27.8 / 24.5 / 39.0 / 31.1 / 39.5 against 26.2 / 31.9 / 27.6 /
    38.5 / 33.8 / 39.8; M = 184 21.9 / 28.3 / 24.8 / 39.8 / 32.6 / 38.9
    against 30.3 / 38.7 / 32.5 / 45.6 / 41.1 / 46.9).
    Version 14 (K split over the waves of a workgroup, 64-column blocks) is
    taken up to M = 64 where 2048 < N <= 4096 (but not up to M = 32 with
    K > 12288) and up to M = 8 where 1024 < N <= 2048 and K <= 8192, and
    from M = 65 to 128 where N <= 4096 and K <= 8192.  Against version 8
    (us per launch, one box): M = 72 / 96 / 128 at N x K = 4096 x 6144
    16.8 / 19.3 / 22.9 against 20.2 / 22.6 / 25.0, at 4096 x 8192 19.2 /
    22.2 / 26.6 against 22.7 / 24.3 / 27.7, at 2048 x 8192 16.5 / 18.2 /
    21.5 against 18.9 / 20.5 / 24.1, at 3072 x 6144 17.4 / 19.5 / 23.1
    against 18.3 / 20.0 / 22.9; at K = 11264 mixed (4096 columns: 23.7 /
    27.9 / 34.2 against 26.7 / 28.3 / 31.3); M = 1 / 4 / 8 at N x K = 1536 x
    8192 8.6 / 9.0 / 9.2 against 10.0 / 10.2 / 10.3, 2048 x 8192 9.6 / 10.1
    / 10.6 against 10.4 / 10.7 / 10.7, 2048 x 4096 8.7 / 9.0 / 9.2 against
    8.9 / 9.1 / 9.2, but 2048 x 14336 16.0 / 16.5 / 16.4 against 15.7 /
    15.9 / 16.0 and M = 16 at N = 2048 (K = 4096 / 8192 / 14336: 9.3 / 11.1
    / 16.4 against 9.1 / 10.8 / 16.0).  At K = 14336, N = 4096 version 8 is faster up
    to M = 32 (us per launch against version 14, 2 rounds on one box: M = 1
    22.3 against 22.6, 16 22.5 against 23.6, 32 23.8 against 24.1; N =
    3072, M = 16 19.1 against 20.1; N = 2560, M = 16 17.8 against 18.0) and
    version 14 from M = 48 (26.1 against 25.4; M = 64 28.4 against 27.2);
    at K = 11264 they are within 2 % (M = 16 19.4 / 19.8, M = 1 19.1 /
    18.9) and at K = 8192 version 14 wins (M = 1 16.4 / 15.5, 16 16.9 /
    16.0, 32 18.4 / 16.5).  Measured on MI355X
    against version 8 (us per launch, one box, M = 1 / 16 / 64 / 128):
    N = 4096, K = 4096 8.1 / 9.1 / 14.4 / 18.4 against 9.5 / 9.9 / 16.2 /
    21.8; N = 3072, K = 2048 7.2 / 7.6 / 11.6 / 14.4 against 8.1 / 8.3 /
    13.5 / 20.3; N = 4096, K = 14336 22.1 / 22.9 / 27.1 / 39.0 against
    22.2 / 22.5 / 28.5 / 35.3; N = 2048, K = 8192 at M = 128 21.0 against
    23.4, at M = 16 10.2 against 10.5; N = 1024, K = 2048 8.3 / 8.6 / 12.4 /
    15.9 against 6.7 / 7.0 / 10.9 / 17.6.  Every 64 columns re-read all of
    A (at M = 128 twice B's bytes), which costs it at large M and K; from
    N = 5120 its power-of-two K split also leaves CUs idle (80 column blocks
    x 2): 128 x 8192 x 8192 41.8 against 32.9.
    The split-tail version 9 comes first among the 256x256 kernels only where
    its schedule splits tiles on this device (it then needs a workspace);
    elsewhere it would run version 7's whole tiles.  The reference picks
    versions at build time only (CMakeLists.txt MATMUL_VERSION); this is a
    convenience of the front end."""
    in_dt = DTYPE_F16 if dtype == "f16" else DTYPE_F32
    out_dt = DTYPE_F16 if (out or dtype) == "f16" else DTYPE_F32
    order = [14, 8, 4, 11, 9, 7, 10, 6, 5, 3, 2, 15, 1] if in_dt == DTYPE_F16 else [2, 3, 1]
    avail = set(_abi.versions(in_dt))

    def takes(v):
        return v in avail and _abi.check(v, in_dt, out_dt, m, n, k, 4096, 4096, 4096) == _abi.VK_OK

    def v11_suits():
        cus = _num_cus()
        tiles = -(-m // 128) * -(-n // 128)
        if m % 256 == 0 and n % 256 == 0 and k % 64 == 0:
            return tiles <= cus
        return 2 * tiles <= 3 * cus

    def v14_suits():
        if m > 128 or n > 4096:
            return False
        if m <= 32 and k > 12288:
            return False
        if m <= 64:
            return n > 2048 or (m <= 8 and n > 1024 and k <= 8192)
        return k <= 8192

    for v in order:
        if v not in avail:
            continue
        if v == 14 and not v14_suits():
            continue
        if v == 8 and m > 128 and in_dt == DTYPE_F16 and v11_suits() and takes(11):
            continue
        if v == 9 and _abi.workspace_bytes(v, in_dt, m, n, k) == 0:
            continue
        if v == 11 and not v11_suits():
            continue
        if v == 15 and m * n * k < (1 << 24):
            continue  # small shapes: version 1 without the copies
        if takes(v):
            return v
    raise VkError(-3, f"no {dtype} version accepts m={m}, n={n}, k={k} with {out or dtype} output")
