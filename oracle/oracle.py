"""CPU ORACLE - TEST INFRASTRUCTURE ONLY.

Python side of the oracle: a ctypes binding of ``grouped_gemm_oracle.c`` (built by ``make`` in
this directory into ``liboracle.so``) plus numpy restatements of the reference's table layout and
launch rules.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module, and only as the checker; the product path never does.

Functions and the reference code they restate:
  * ``gemm``                        kernels/matmul.py:223-273 (fp32-exact products, fp32/fp64
                                    accumulation, cast on store); pinned by tests/test_oracle.py
                                    against the golden fixtures (torch CPU float64), closed forms,
                                    brute force and numpy.
  * ``grouped_gemm`` / ``grouped_gemm_tables``  kernels/grouped_gemm.py:399-482 over the tables of
                                    :530-544 (pointer tables, dims (m, n, k), strides (am, ak, bk,
                                    bn, cm, cn)); pinned against the golden fixtures, a brute force
                                    and numpy on heterogeneous and strided groups, and by planted
                                    table mistakes (dims order, stride order) that must fail.
  * ``tables``                      kernels/grouped_gemm.py:530-544 (pointer order, dims (m, n, k),
                                    strides (am, ak, bk, bn, cm, cn)); pinned by brute force.
  * ``is_homogeneous``              kernels/grouped_gemm.py:550-552; pinned by reference tests'
                                    expectations (tests/test_gpu.py:99-125 of the reference).
  * ``dispatch``                    kernels/grouped_gemm.py:629-640, 682, 709, 739, 760 (scheduler names).
  * ``grid_size``                   kernels/grouped_gemm.py:597-599.
  * ``tile_order``                  kernels/grouped_gemm.py:353-360 (GROUP_M traversal + persistent
                                    stride); pinned by a coverage/bijection check.
  * ``w13_reference``               benchmark_moe.py:258-266 (cat of gate and up products).
  * ``offsets_groups`` / ``grouped_mm_offsets``  the expert-sorted 2-D A / 3-D B / int32 ``offs``
                                    layout of kernels/torch_grouped_gemm.py:139-158 with the
                                    semantics of torch.nn.functional.grouped_mm (group e owns rows
                                    offs[e-1]:offs[e]; rows past offs[-1] are unspecified there and
                                    zero here); pinned against
                                    torch's CPU grouped_mm and a brute force in tests/test_oracle.py.
  * ``swiglu_reference``            silu(A @ B[:, :F]) * (A @ B[:, F:]) over packed Gate+Up weights
                                    (the step after benchmark_moe.py:258-266's W13 product,
                                    README.md:55-57): exact sums, float64 activation, one rounding;
                                    pinned against torch CPU float64 and a planted gate/up swap.
  * ``offsets_tile_bound``          the host's tile-count bound for that layout (each group adds at
                                    most one partial M tile); pinned by exhaustive small cases.
  * ``to_bf16_bits`` / ``to_f16_bits``  round-to-nearest-even casts; pinned against torch/numpy.
  * ``c_decode``                    the C decoders behind every operand read; pinned over all
                                    65536 bit patterns against numpy's float16 and the bf16 shift.
  * ``gemm_fast_bf16``              the same fp32 running sum as ``gemm(accum="f32")``, blocked and
                                    threaded (an extra CPU timing in bench.py); pinned bit for bit
                                    against a numpy float32 running sum with torch's cast, against
                                    ``gemm(accum="f32")``, within the float32 accumulation bound of
                                    the golden sums, and by a planted dropped term.
"""

from __future__ import annotations

import ctypes
import math
import subprocess
from functools import lru_cache
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"

F16, BF16, F32 = 0, 1, 2
ACCUM_F64, ACCUM_F32 = 0, 1
_DTYPES = {"fp16": F16, "bf16": BF16, "fp32": F32}


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not LIBRARY.exists():
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    handle = ctypes.CDLL(str(LIBRARY))
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    handle.oracle_gemm.argtypes = [vp, vp, vp, i32, i32, i32, i64, i64, i64, i64, i64, i64, i32, i32, i32, vp]
    handle.oracle_gemm.restype = ctypes.c_int
    handle.oracle_grouped_gemm.argtypes = [i32, vp, vp, vp, vp, vp, i32, i32, i32]
    handle.oracle_grouped_gemm.restype = ctypes.c_int
    handle.oracle_gemm_rowmajor_fast.argtypes = [vp, vp, vp, i32, i32, i32, i32, vp, i32]
    handle.oracle_gemm_rowmajor_fast.restype = ctypes.c_int
    handle.oracle_float_to_bf16.argtypes = [ctypes.c_float]
    handle.oracle_float_to_bf16.restype = ctypes.c_uint16
    handle.oracle_float_to_f16.argtypes = [ctypes.c_float]
    handle.oracle_float_to_f16.restype = ctypes.c_uint16
    handle.oracle_tf32_round.argtypes = [ctypes.c_float]
    handle.oracle_tf32_round.restype = ctypes.c_float
    handle.oracle_f16_to_float.argtypes = [ctypes.c_uint16]
    handle.oracle_f16_to_float.restype = ctypes.c_float
    handle.oracle_bf16_to_float.argtypes = [ctypes.c_uint16]
    handle.oracle_bf16_to_float.restype = ctypes.c_float
    return handle


def c_decode(bits: np.ndarray, dtype: str) -> np.ndarray:
    """The C library's own 16-bit decoders (the ones oracle_gemm reads operands with)."""
    handle = lib()
    fn = handle.oracle_bf16_to_float if dtype == "bf16" else handle.oracle_f16_to_float
    flat = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    return np.array([fn(int(v)) for v in flat], dtype=np.float32).reshape(np.shape(bits))


# --------------------------------------------------------------------------------------------
# Element encodings.  16-bit matrices are carried as numpy uint16 bit patterns.

def bf16_bits_to_float(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_float(bits: np.ndarray) -> np.ndarray:
    return bits.view(np.float16).astype(np.float32)


def to_float(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_float(bits)
    if dtype == "fp16":
        return f16_bits_to_float(bits)
    return bits.astype(np.float32)


def to_bf16_bits(values: np.ndarray) -> np.ndarray:
    handle = lib()
    flat = np.ascontiguousarray(values, dtype=np.float32).ravel()
    return np.array([handle.oracle_float_to_bf16(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(values))


def to_f16_bits(values: np.ndarray) -> np.ndarray:
    handle = lib()
    flat = np.ascontiguousarray(values, dtype=np.float32).ravel()
    return np.array([handle.oracle_float_to_f16(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(values))


def tf32_round(values: np.ndarray) -> np.ndarray:
    handle = lib()
    flat = np.ascontiguousarray(values, dtype=np.float32).ravel()
    return np.array([handle.oracle_tf32_round(float(v)) for v in flat], dtype=np.float32).reshape(np.shape(values))


# --------------------------------------------------------------------------------------------
# GEMM

def _element_size(dtype: str) -> int:
    return 4 if dtype == "fp32" else 2


def gemm(a: np.ndarray, b: np.ndarray, dtype: str, *, tf32: bool = False, accum: str = "f64",
         out_strides: tuple[int, int] | None = None, return_sums: bool = False):
    """C = A @ B for one problem.  ``a``/``b`` are uint16 bit patterns (fp16/bf16) or float32,
    with any (element) strides numpy allows; returns C in the operand encoding (and optionally
    the unrounded sums as float64)."""
    code = _DTYPES[dtype]
    store = np.float32 if dtype == "fp32" else np.uint16
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype != store or b.dtype != store:
        raise TypeError(f"{dtype} operands must be numpy {np.dtype(store).name} arrays")
    m, k = a.shape
    kb, n = b.shape
    if k != kb:
        raise ValueError("inner dimensions differ")
    es = _element_size(dtype)
    c = np.zeros((m, n), dtype=store)
    sums = np.zeros((m, n), dtype=np.float64) if return_sums else None
    rc = lib().oracle_gemm(
        a.ctypes.data, b.ctypes.data, c.ctypes.data, m, n, k,
        a.strides[0] // es, a.strides[1] // es, b.strides[0] // es, b.strides[1] // es, n, 1,
        code, int(tf32), ACCUM_F32 if accum == "f32" else ACCUM_F64,
        sums.ctypes.data if sums is not None else None,
    )
    if rc:
        raise ValueError("oracle_gemm rejected its arguments")
    return (c, sums) if return_sums else c


def grouped_gemm_tables(a_list, b_list, c_list, dims, strides, dtype: str, *, tf32: bool = False,
                        accum: str = "f64") -> None:
    """The reference's table form (kernels/grouped_gemm.py:530-544, read at :427-449): host pointer
    tables over the arrays' first elements, ``dims`` int32 [G,3] = (m, n, k) and ``strides`` int64
    [G,6] = (am, ak, bk, bn, cm, cn) in elements.  C_e is written through ``c_list[e]``'s memory as
    the tables describe it; the arrays are not checked against the tables (as on the device)."""
    groups = len(a_list)
    if not groups or len(b_list) != groups or len(c_list) != groups:
        raise ValueError("grouped GEMM requires matching, non-empty operand lists")
    dims = np.ascontiguousarray(dims, dtype=np.int32)
    strides = np.ascontiguousarray(strides, dtype=np.int64)
    if dims.shape != (groups, 3) or strides.shape != (groups, 6):
        raise ValueError("dims must be [G,3] and strides [G,6]")
    table = ctypes.c_void_p * groups
    a_ptrs = table(*(int(x.ctypes.data) for x in a_list))
    b_ptrs = table(*(int(x.ctypes.data) for x in b_list))
    c_ptrs = table(*(int(x.ctypes.data) for x in c_list))
    rc = lib().oracle_grouped_gemm(groups, ctypes.addressof(a_ptrs), ctypes.addressof(b_ptrs),
                                   ctypes.addressof(c_ptrs), dims.ctypes.data, strides.ctypes.data,
                                   _DTYPES[dtype], int(tf32), ACCUM_F32 if accum == "f32" else ACCUM_F64)
    if rc:
        raise ValueError("oracle_grouped_gemm rejected its tables")


def grouped_gemm(a_list, b_list, dtype: str, *, tf32: bool = False, accum: str = "f64"):
    """C_e = A_e @ B_e for every problem, through the table form: dims and strides are taken from
    the operand views exactly as the reference's builder takes them from its tensors
    (kernels/grouped_gemm.py:536-544), so strided views keep their strides.  Returns the C list
    (row-major, operand encoding)."""
    if not a_list or len(a_list) != len(b_list):
        raise ValueError("grouped GEMM requires matching, non-empty operand lists")
    store = np.float32 if dtype == "fp32" else np.uint16
    es = _element_size(dtype)
    c_list, dims, strides = [], [], []
    for a, b in zip(a_list, b_list):
        a, b = np.asarray(a), np.asarray(b)
        if a.dtype != store or b.dtype != store:
            raise TypeError(f"{dtype} operands must be numpy {np.dtype(store).name} arrays")
        (m, k), (kb, n) = a.shape, b.shape
        if k != kb:
            raise ValueError("inner dimensions differ")
        c = np.zeros((m, n), dtype=store)
        c_list.append(c)
        dims.append((m, n, k))
        strides.append((a.strides[0] // es, a.strides[1] // es, b.strides[0] // es, b.strides[1] // es,
                        c.strides[0] // es, c.strides[1] // es))
    grouped_gemm_tables(a_list, b_list, c_list, dims, strides, dtype, tf32=tf32, accum=accum)
    return c_list


def w13_reference(a: np.ndarray, b: np.ndarray, dtype: str, **kwargs) -> np.ndarray:
    """Packed Gate+Up reference: [A @ B[:, :F] | A @ B[:, F:]] (benchmark_moe.py:258-266)."""
    n = b.shape[1]
    if n % 2:
        raise ValueError("packed W13 needs an even output width")
    half = n // 2
    gate = gemm(a, np.ascontiguousarray(b[:, :half]), dtype, **kwargs)
    up = gemm(a, np.ascontiguousarray(b[:, half:]), dtype, **kwargs)
    return np.concatenate([gate, up], axis=1)


def swiglu_reference(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    """H = silu(A @ B[:, :F]) * (A @ B[:, F:]) for packed B = [gate | up], rounded once to dtype."""
    n = b.shape[1]
    if n % 2:
        raise ValueError("packed Gate+Up weights need an even width")
    half = n // 2
    _, gate = gemm(a, np.ascontiguousarray(b[:, :half]), dtype, return_sums=True)
    _, up = gemm(a, np.ascontiguousarray(b[:, half:]), dtype, return_sums=True)
    h = gate / (1.0 + np.exp(-gate)) * up
    h32 = h.astype(np.float32)
    if dtype == "bf16":
        return to_bf16_bits(h32)
    if dtype == "fp16":
        return to_f16_bits(h32)
    return h32


def offsets_groups(offs, rows: int) -> list[tuple[int, int]]:
    """(first row, row count) of each group: offsets clamped to [0, rows], decreasing = empty."""
    groups = []
    prev = 0
    for end in (int(v) for v in offs):
        lo, hi = min(max(prev, 0), rows), min(max(end, 0), rows)
        groups.append((lo, max(hi - lo, 0)))
        prev = end
    return groups


def grouped_mm_offsets(a: np.ndarray, b3: np.ndarray, offs, dtype: str, **kwargs) -> np.ndarray:
    """C [rows, N] with C[r0:r0+m] = A[r0:r0+m] @ B[e] per group; rows no group covers are zero."""
    rows, k = a.shape
    groups, kb, n = b3.shape
    if k != kb or len(offs) != groups:
        raise ValueError("expert-sorted operands disagree on K or the group count")
    store = np.float32 if dtype == "fp32" else np.uint16
    c = np.zeros((rows, n), dtype=store)
    for e, (r0, m) in enumerate(offsets_groups(offs, rows)):
        if m:
            c[r0:r0 + m] = gemm(a[r0:r0 + m], b3[e], dtype, **kwargs)
    return c


def offsets_tile_bound(rows: int, group_count: int, n: int, block_m: int, block_n: int) -> int:
    if rows <= 0:
        return 0
    m_tiles = min(rows // block_m + group_count, group_count * math.ceil(rows / block_m))
    return m_tiles * math.ceil(n / block_n)


def gemm_fast_bf16(a_bits: np.ndarray, b_bits: np.ndarray, threads: int, dtype: str = "bf16") -> np.ndarray:
    """OpenMP fp32-accumulating contiguous GEMM (CPU baseline timing only)."""
    m, k = a_bits.shape
    _, n = b_bits.shape
    a_bits = np.ascontiguousarray(a_bits, dtype=np.uint16)
    b_bits = np.ascontiguousarray(b_bits, dtype=np.uint16)
    c = np.empty((m, n), dtype=np.uint16)
    scratch = np.empty((m, n), dtype=np.float32)
    rc = lib().oracle_gemm_rowmajor_fast(a_bits.ctypes.data, b_bits.ctypes.data, c.ctypes.data, m, n, k,
                                         _DTYPES[dtype], scratch.ctypes.data, threads)
    if rc:
        raise ValueError("oracle_gemm_rowmajor_fast rejected its arguments")
    return c


# --------------------------------------------------------------------------------------------
# Tables and launch rules

def tables(shapes, strides_list=None):
    """dims [G,3] = (m, n, k) and strides [G,6] = (am, ak, bk, bn, cm, cn) as the reference builds them."""
    dims = np.array([[m, n, k] for m, k, n in shapes], dtype=np.int32)
    if strides_list is None:
        strides_list = [(k, 1, n, 1, n, 1) for m, k, n in shapes]
    strides = np.array(strides_list, dtype=np.int64)
    return dims, strides


def is_homogeneous(shapes, contiguous_flags) -> bool:
    return all(s == shapes[0] for s in shapes) and all(contiguous_flags)


def dispatch(problem_count: int, homogeneous: bool) -> str:
    if problem_count == 1:
        return "single_problem_matmul"
    return "homogeneous_persistent" if homogeneous else "generic_persistent"


def tile_count(shapes, block_m: int, block_n: int) -> int:
    return sum(math.ceil(m / block_m) * math.ceil(n / block_n) for m, _, n in shapes)


def grid_size(shapes, block_m: int, block_n: int, sm_count: int, cta_multiplier: int) -> int:
    return max(1, min(tile_count(shapes, block_m, block_n), sm_count * cta_multiplier))


def group_m_tile(local: int, m_tiles: int, n_tiles: int, group_m: int) -> tuple[int, int]:
    width = group_m * n_tiles
    first_m = (local // width) * group_m
    size = min(m_tiles - first_m, group_m)
    return first_m + local % size, (local % width) // size


def tile_order(shapes, block_m: int, block_n: int, group_m: int, grid: int):
    """For each program id, the (problem, m-tile, n-tile) list it visits in order."""
    offsets = [0]
    per_problem = []
    for m, _, n in shapes:
        mt, nt = math.ceil(m / block_m), math.ceil(n / block_n)
        per_problem.append((mt, nt))
        offsets.append(offsets[-1] + mt * nt)
    total = offsets[-1]
    visits = []
    for pid in range(grid):
        mine = []
        for t in range(pid, total, grid):
            e = int(np.searchsorted(offsets, t, side="right") - 1)
            mt, nt = per_problem[e]
            mine.append((e, *group_m_tile(t - offsets[e], mt, nt, group_m)))
        visits.append(mine)
    return visits
