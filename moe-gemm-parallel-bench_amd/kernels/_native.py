"""ctypes binding of libmoegemm.so (the C ABI declared in include/moegemm.h).

The library is built in-tree next to this file (``csrc/Makefile`` or ``__graft_entry__.build()``).
Nothing here falls back to another implementation: when the library or a GPU is missing, every
launch raises ``RuntimeError``, mirroring the reference's "Triton with an active CUDA driver is
required" error (reference kernels/grouped_gemm.py:626-627, kernels/matmul.py:342-343).
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().with_name("libmoegemm.so")

ABI_VERSION = 9
OK = 0
ERR_INVALID = -1
ERR_NO_KERNEL = -2
ERR_LAUNCH = -3

DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2
PRECISION_IEEE = 0
PRECISION_TF32 = 1

DTYPE_NAMES = {DTYPE_F16: "fp16", DTYPE_BF16: "bf16", DTYPE_F32: "fp32"}

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p

# Exported symbol -> (restype, argtypes).  tests/test_native_abi.py checks this against the header.
SIGNATURES = {
    "moegemm_abi_version": (ctypes.c_int, []),
    "moegemm_last_error": (ctypes.c_char_p, []),
    "moegemm_kernel_count": (ctypes.c_int, [ctypes.c_int]),
    "moegemm_kernel_info": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.POINTER(_i32)]),
    "moegemm_grouped_gemm": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "moegemm_grouped_gemm_stealing": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i32, _vp],
    ),
    "moegemm_grouped_gemm_swiglu": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "moegemm_kernel_swiglu": (ctypes.c_int, [ctypes.c_int, ctypes.c_int]),
    "moegemm_splitk_workspace_bytes": (ctypes.c_int, [_i32, _i32, _i32, _i32, ctypes.POINTER(_i64)]),
    "moegemm_matmul_splitk": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i32, _vp],
    ),
    "moegemm_matmul_splitk_noalloc": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "moegemm_grouped_gemm_splitk": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         _i32, _i32, _i32, _vp, _i64, _i32, _vp],
    ),
    "moegemm_streamk_workspace_bytes": (ctypes.c_int, [_i32, _i32, _i32, _i32, ctypes.POINTER(_i64)]),
    "moegemm_matmul_streamk": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i32, _vp],
    ),
    "moegemm_grouped_gemm_streamk": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         _i32, _i32, _i32, _vp, _i64, _i32, _vp],
    ),
    "moegemm_grouped_mm_offs": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i32, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "moegemm_grouped_mm_offs_swiglu": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "moegemm_grouped_mm_offs_stealing": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i32, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i32, _vp],
    ),
    "moegemm_matmul": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
}


class NativeUnavailable(RuntimeError):
    """libmoegemm.so is missing or does not match this binding."""


@lru_cache(maxsize=1)
def library() -> ctypes.CDLL:
    path = Path(os.environ.get("MOEGEMM_LIBRARY", LIBRARY_PATH))
    if not path.exists():
        raise NativeUnavailable(
            f"native library {path} is not built; run `make -C moe-gemm-parallel-bench_amd/csrc` "
            "or __graft_entry__.build()"
        )
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as exc:  # missing ROCm runtime, wrong architecture, ...
        raise NativeUnavailable(f"cannot load {path}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.moegemm_abi_version()
    if version != ABI_VERSION:
        raise NativeUnavailable(f"{path} has ABI version {version}, this binding expects {ABI_VERSION}")
    return lib


def available() -> bool:
    try:
        library()
        return True
    except NativeUnavailable:
        return False


def last_error() -> str:
    return library().moegemm_last_error().decode("utf-8", "replace")


def check(status: int) -> None:
    """Map a native status to the reference's exception types."""
    if status == OK:
        return
    message = last_error()
    if status == ERR_INVALID:
        raise ValueError(message)
    raise RuntimeError(message)


@lru_cache(maxsize=None)
def compiled_kernels(dtype_code: int) -> tuple[tuple[int, int, int, int, int, int, int], ...]:
    """(block_m, block_n, block_k, num_warps, num_stages, lds_bytes, waves_m) per compiled kernel."""
    lib = library()
    out = (_i32 * 7)()
    rows = []
    for index in range(lib.moegemm_kernel_count(dtype_code)):
        check(lib.moegemm_kernel_info(dtype_code, index, out))
        rows.append(tuple(int(v) for v in out))
    return tuple(rows)


@lru_cache(maxsize=None)
def swiglu_tiles(dtype_code: int) -> frozenset:
    """Tile keys (block_m, block_n, block_k, num_warps, num_stages) that can run the SwiGLU epilogue."""
    lib = library()
    keys = set()
    for index, row in enumerate(compiled_kernels(dtype_code)):
        status = lib.moegemm_kernel_swiglu(dtype_code, index)
        if status < 0:
            check(status)
        if status == 1:
            keys.add(tuple(row[:5]))
    return frozenset(keys)


def splitk_workspace_bytes(tiles: int, splits: int, block_m: int, block_n: int) -> int:
    out = _i64(0)
    check(library().moegemm_splitk_workspace_bytes(tiles, splits, block_m, block_n, ctypes.byref(out)))
    return int(out.value)


def streamk_workspace_bytes(tail_tiles: int, grid: int, block_m: int, block_n: int) -> int:
    out = _i64(0)
    check(library().moegemm_streamk_workspace_bytes(tail_tiles, grid, block_m, block_n, ctypes.byref(out)))
    return int(out.value)


PANEL_ROWS = 256  # the largest block_m of the menu
_TWO_GIB = 1 << 31


def panels_fit(k: int, sam: int, sbk: int, scm: int) -> bool:
    """Byte-range limits of the LDS-DMA kernels' 32-bit buffer offsets, as the library checks them:
    A and C are addressed through one resource per tile of at most PANEL_ROWS rows (any number of
    rows in all), B through one resource running to the end of the [k, n] matrix."""
    return PANEL_ROWS * sam * 2 < _TWO_GIB and PANEL_ROWS * scm * 2 < _TWO_GIB and k * sbk * 2 < _TWO_GIB


def streamk_tail(tiles: int, grid: int, k: int, block_k: int) -> int:
    """Tail tiles of a stream-K launch (0 when stream-K does not apply): the remainder r of
    ``tiles`` over a ``grid`` of workgroups, so the whole tiles fill exact rounds and the r tail
    tiles are spread over every workgroup.  0 when there is no remainder, or when the tail is too
    thin for the library's limit of 64 pieces per tile."""
    if tiles <= 0 or grid <= 0:
        return 0
    tail = tiles % grid
    if tail == 0:
        return 0
    kt = -(-k // block_k)
    per_run = tail * kt // grid
    if per_run < 1 or -(-kt // per_run) + 1 > 64:
        return 0
    return tail


# Split-K workspaces, one per (device, stream).  A workspace is never released once handed out, so
# a captured graph that recorded its address stays valid; a larger need allocates a new one.
_SPLITK_WORKSPACES: dict[tuple[int, int], list] = {}
_SPLITK_MIN_BYTES = 32 << 20


def _refuse_allocation_under_capture(what: str) -> None:
    """A buffer made inside graph capture would be zeroed only when the graph replays, so an eager
    launch on that stream before the first replay would read stale counters: refuse instead."""
    import torch

    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"the {what} for this stream does not exist yet and cannot be created during graph "
                           "capture; make the first call on this stream outside capture")


def splitk_workspace(device, stream_handle: int, nbytes: int):
    """A zero-initialised uint8 device tensor of at least ``nbytes`` for this device and stream."""
    import torch

    key = (torch.device(device).index or 0, int(stream_handle))
    held = _SPLITK_WORKSPACES.setdefault(key, [])
    if not held or held[-1].numel() < nbytes:
        _refuse_allocation_under_capture("split-K workspace")
        held.append(torch.zeros(max(nbytes, _SPLITK_MIN_BYTES), dtype=torch.uint8, device=device))
    return held[-1]


# Work-stealing tile queues, one per (device, stream), zeroed once and never released (launches
# leave them zero; a captured graph keeps a valid address).
QUEUE_BYTES = 4352
NOALLOC_SCRATCH_BYTES = 64 * 1024 * 1024 + 256 * 1024  # MOEGEMM_NOALLOC_SCRATCH_BYTES
TILE_SCHEDULES = ("static", "stealing")
# Schedules of homogeneous grouped launches: also "streamk" (whole tiles in exact rounds, then a
# stream-K tail; fp16/bf16 vector layouts).
GROUPED_SCHEDULES = TILE_SCHEDULES + ("streamk",)
_TILE_QUEUES: dict[tuple[int, int], object] = {}


def tile_queue(device, stream_handle: int):
    """The zero-initialised MOEGEMM_QUEUE_BYTES device buffer for this device and stream."""
    import torch

    key = (torch.device(device).index or 0, int(stream_handle))
    queue = _TILE_QUEUES.get(key)
    if queue is None:
        _refuse_allocation_under_capture("work-stealing tile queue")
        queue = torch.zeros(QUEUE_BYTES // 4, dtype=torch.int32, device=device)
        _TILE_QUEUES[key] = queue
    return queue


def dtype_code(dtype) -> int:
    import torch

    codes = {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}
    if dtype not in codes:
        raise ValueError(f"unsupported dtype {dtype}; expected float16, bfloat16 or float32")
    return codes[dtype]


def precision_code(input_precision: str, dtype_code_value: int) -> int:
    if input_precision not in ("ieee", "tf32"):
        raise ValueError(f"input_precision must be 'ieee' or 'tf32', got {input_precision!r}")
    # Like tl.dot, TF32 only changes fp32 operands; 16-bit operands are exact in any mode.
    if input_precision == "tf32" and dtype_code_value == DTYPE_F32:
        return PRECISION_TF32
    return PRECISION_IEEE


def current_stream_handle(device) -> int:
    import torch

    return int(torch.cuda.current_stream(device).cuda_stream)
