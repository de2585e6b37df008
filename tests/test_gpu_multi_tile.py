"""GPU tests of workgroups that run several tiles in a row (static and work-stealing schedules).

Each tile's epilogue stages C in the LDS slots that the next tile's copies refill, so a tile must
leave nothing behind for its successor.  Exact-integer results (small integers in A and B, so the
fp32 sums are exact and the store rounds them as the float64 reference rounded to the dtype does)
are checked for every compiled 16-bit tile at grids that give each workgroup several tiles, with
ragged M, N and K so that the last tiles store partial rows and columns; NaN guard bands around
each C catch a store outside it.  Homogeneous groups mix 16-byte-aligned and 8-byte-aligned C
(whole-row and half-row stores alternate within a launch), and single GEMMs write into a column
slice of a wider matrix whose other columns must stay untouched.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DTYPES = (torch.bfloat16, torch.float16)
GUARD = 4096


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")
    torch.manual_seed(5)


def _ints(shape, dtype):
    return torch.randint(-2, 3, shape, device="cuda").to(dtype)


def _tiles(dtype):
    from kernels import _native

    return [tuple(row[:5]) for row in _native.compiled_kernels(_native.dtype_code(dtype))]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_homogeneous_every_tile_small_grids_mixed_alignment(dtype):
    from kernels import _native
    from kernels.grouped_gemm import _vector_layout, build_grouped_workspace

    groups, m, k, n = 5, 300, 200, 392
    ws = build_grouped_workspace([(m, k, n)] * groups, dtype, seed=1)
    storages = []
    for e in range(groups):
        ws.a[e].copy_(_ints((m, k), dtype))
        ws.b[e].copy_(_ints((k, n), dtype))
        lead = GUARD + (4 if e % 2 else 0)  # odd problems: C only 8-byte aligned
        storage = torch.full((lead + m * n + GUARD,), float("nan"), device="cuda", dtype=dtype)
        ws.c[e] = storage[lead:lead + m * n].view(m, n)
        ws.c_ptrs[e] = ws.c[e].data_ptr()
        storages.append((storage, lead))
    assert ws.homogeneous
    code = _native.dtype_code(dtype)
    assert _vector_layout(ws, code)
    expected = [(a.double() @ b.double()).to(dtype) for a, b, _ in ws.problem_tensors()]
    for bm, bn, bk, warps, stages in _tiles(dtype):
        tiles = groups * -(-m // bm) * -(-n // bn)
        for grid in sorted({1, 3, 8, 13, max(1, tiles // 3)}):
            print(f"multi-tile homogeneous tile={(bm, bn, bk, warps, stages)} tiles={tiles} grid={grid}", flush=True)
            for storage, _ in storages:
                storage.fill_(float("nan"))
            status = _native.library().moegemm_grouped_gemm(
                ws.a_ptrs.data_ptr(), ws.b_ptrs.data_ptr(), ws.c_ptrs.data_ptr(), ws.dims.data_ptr(),
                ws.strides.data_ptr(), groups, m, n, k, 1, tiles, code, 0, bm, bn, bk, 4, warps, stages, grid, 1,
                0, _native.current_stream_handle(ws.a[0].device))
            _native.check(status)
            torch.cuda.synchronize()
            for e, ((storage, lead), ref) in enumerate(zip(storages, expected)):
                label = f"tile {(bm, bn, bk, warps, stages)} grid {grid} problem {e}"
                assert torch.equal(ws.c[e], ref), label
                assert torch.isnan(storage[:lead]).all() and torch.isnan(storage[lead + m * n:]).all(), label


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("pitch_pad", [8, 4], ids=["c16", "c8"])
def test_single_every_tile_column_slice_small_grids(dtype, pitch_pad):
    from kernels import _native

    m, k, n = 333, 136, 520
    pitch = n + pitch_pad
    a, b = _ints((m, k), dtype), _ints((k, n), dtype)
    expected = (a.double() @ b.double()).to(dtype)
    wide = torch.empty((m + 2, pitch), device="cuda", dtype=dtype)
    c = wide[1:m + 1, :n]  # rows 0 and m + 1 and the last pitch_pad columns are guards
    code = _native.dtype_code(dtype)
    for bm, bn, bk, warps, stages in _tiles(dtype):
        tiles = -(-m // bm) * -(-n // bn)
        for grid in sorted({1, 5, 16, max(1, tiles // 2)}):
            print(f"multi-tile single tile={(bm, bn, bk, warps, stages)} pitch={pitch} tiles={tiles} grid={grid}",
                  flush=True)
            wide.fill_(float("nan"))
            status = _native.library().moegemm_matmul(
                a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, a.stride(0), a.stride(1), b.stride(0),
                b.stride(1), c.stride(0), c.stride(1), code, 0, bm, bn, bk, 4, warps, stages, grid,
                0, _native.current_stream_handle(a.device))
            _native.check(status)
            torch.cuda.synchronize()
            label = f"tile {(bm, bn, bk, warps, stages)} grid {grid}"
            assert torch.equal(c, expected), label
            assert torch.isnan(wide[0]).all() and torch.isnan(wide[m + 1]).all(), label
            assert torch.isnan(wide[:, n:]).all(), label


@pytest.mark.parametrize("schedule", ["static", "stealing"])
@pytest.mark.parametrize("k", [64, 128, 136, 192, 256, 328])
def test_chained_two_stage_tiles_every_k_slice_count(k, schedule):
    """Two-stage tiles chain each tile's copies into the next tile's first K slice (single and
    homogeneous launches).  On the stealing schedule the workgroup claims its units one ahead.  K
    from one slice (no chaining) to several with a tail, ragged M and N, several tiles per
    workgroup and C alternating 16- and 8-byte alignment (staged tiles chain only for 16-byte
    aligned C): exact integers, intact guard bands, and a re-armed queue after every launch."""
    from kernels import _native
    from kernels.grouped_gemm import build_grouped_workspace

    dtype = torch.bfloat16
    groups, m, n = 6, 70, 392
    ws = build_grouped_workspace([(m, k, n)] * groups, dtype, seed=2)
    storages = []
    for e in range(groups):
        ws.a[e].copy_(_ints((m, k), dtype))
        ws.b[e].copy_(_ints((k, n), dtype))
        lead = GUARD + (4 if e % 3 == 1 else 0)
        storage = torch.full((lead + m * n + GUARD,), float("nan"), device="cuda", dtype=dtype)
        ws.c[e] = storage[lead:lead + m * n].view(m, n)
        ws.c_ptrs[e] = ws.c[e].data_ptr()
        storages.append((storage, lead))
    code = _native.dtype_code(dtype)
    expected = [(a.double() @ b.double()).to(dtype) for a, b, _ in ws.problem_tensors()]
    two_stage = [t for t in _tiles(dtype) if t[4] == 2 and t[0] <= 64]
    assert two_stage
    for bm, bn, bk, warps, stages in two_stage:
        tiles = groups * -(-m // bm) * -(-n // bn)
        for grid in sorted({1, 5, 8, max(1, tiles // 4)}):
            print(f"chained {schedule} k={k} tile={(bm, bn, bk, warps, stages)} tiles={tiles} grid={grid}", flush=True)
            for storage, _ in storages:
                storage.fill_(float("nan"))
            args = (ws.a_ptrs.data_ptr(), ws.b_ptrs.data_ptr(), ws.c_ptrs.data_ptr(), ws.dims.data_ptr(),
                    ws.strides.data_ptr(), groups, m, n, k, 1, tiles, code, 0, bm, bn, bk, 4, warps, stages, grid, 1)
            stream = _native.current_stream_handle(ws.a[0].device)
            if schedule == "stealing":
                queue = torch.zeros(_native.QUEUE_BYTES // 4, dtype=torch.int32, device="cuda")
                status = _native.library().moegemm_grouped_gemm_stealing(*args, queue.data_ptr(), 0, stream)
            else:
                status = _native.library().moegemm_grouped_gemm(*args, 0, stream)
            _native.check(status)
            torch.cuda.synchronize()
            if schedule == "stealing":
                assert not queue.any(), f"queue not re-armed: {queue.tolist()}"
            for e, ((storage, lead), ref) in enumerate(zip(storages, expected)):
                label = f"{schedule} k {k} tile {(bm, bn, bk, warps, stages)} grid {grid} problem {e}"
                assert torch.equal(ws.c[e], ref), label
                assert torch.isnan(storage[:lead]).all() and torch.isnan(storage[lead + m * n:]).all(), label


@pytest.mark.parametrize("schedule", ["static", "stealing"])
@pytest.mark.parametrize("k", [64, 96, 128, 136, 160, 232])
def test_chained_ping_pong_tiles_every_k_slice_count(k, schedule):
    """The 8-wave 256x256 ping-pong tiles chain across tiles on the static schedule: a tile's last
    three memory phases copy the next tile's first slices, C leaves through one stage, and the next
    tile's first waits count the previous tile's stores.  K from two slices (unchained) through
    four (the first chained count) to several with a tail; several tiles per workgroup, ragged M
    and N, C alternating 16- and 8-byte alignment (8-byte aligned C runs the unchained epilogue, so
    chained and unchained tiles alternate in one workgroup).  The stealing schedule runs these
    tiles unchained.  Exact integers, intact guard bands, re-armed queue."""
    from kernels import _native
    from kernels.grouped_gemm import build_grouped_workspace

    dtype = torch.bfloat16
    groups, m, n = 4, 300, 520
    ws = build_grouped_workspace([(m, k, n)] * groups, dtype, seed=3)
    storages = []
    for e in range(groups):
        ws.a[e].copy_(_ints((m, k), dtype))
        ws.b[e].copy_(_ints((k, n), dtype))
        lead = GUARD + (4 if e % 3 == 1 else 0)
        storage = torch.full((lead + m * n + GUARD,), float("nan"), device="cuda", dtype=dtype)
        ws.c[e] = storage[lead:lead + m * n].view(m, n)
        ws.c_ptrs[e] = ws.c[e].data_ptr()
        storages.append((storage, lead))
    code = _native.dtype_code(dtype)
    expected = [(a.double() @ b.double()).to(dtype) for a, b, _ in ws.problem_tensors()]
    ping_pong = [t for t in _tiles(dtype) if t[:2] == (256, 256) and t[3] == 8 and t[4] >= 3]
    assert ping_pong
    for bm, bn, bk, warps, stages in ping_pong:
        tiles = groups * -(-m // bm) * -(-n // bn)
        for grid in (1, 5, 8):
            print(f"ping-pong chained {schedule} k={k} tile={(bm, bn, bk, warps, stages)} tiles={tiles} grid={grid}",
                  flush=True)
            for storage, _ in storages:
                storage.fill_(float("nan"))
            args = (ws.a_ptrs.data_ptr(), ws.b_ptrs.data_ptr(), ws.c_ptrs.data_ptr(), ws.dims.data_ptr(),
                    ws.strides.data_ptr(), groups, m, n, k, 1, tiles, code, 0, bm, bn, bk, 4, warps, stages, grid, 1)
            stream = _native.current_stream_handle(ws.a[0].device)
            if schedule == "stealing":
                queue = torch.zeros(_native.QUEUE_BYTES // 4, dtype=torch.int32, device="cuda")
                status = _native.library().moegemm_grouped_gemm_stealing(*args, queue.data_ptr(), 0, stream)
            else:
                status = _native.library().moegemm_grouped_gemm(*args, 0, stream)
            _native.check(status)
            torch.cuda.synchronize()
            if schedule == "stealing":
                assert not queue.any(), f"queue not re-armed: {queue.tolist()}"
            for e, ((storage, lead), ref) in enumerate(zip(storages, expected)):
                label = f"{schedule} k {k} tile {(bm, bn, bk, warps, stages)} grid {grid} problem {e}"
                assert torch.equal(ws.c[e], ref), label
                assert torch.isnan(storage[:lead]).all() and torch.isnan(storage[lead + m * n:]).all(), label


@pytest.mark.parametrize("k", [64, 128, 136, 232])
def test_ping_pong_swiglu_several_tiles_per_workgroup(k):
    """The packed W13 SwiGLU epilogue on the ping-pong tiles with several tiles per workgroup
    stores bit for bit what one tile per workgroup stores, keeps the guard bands around every H
    intact, and matches the oracle's SwiGLU within the normwise bound.  (SwiGLU launches run
    these tiles unchained: chaining them measured no gain.)"""
    import numpy as np

    from helpers import from_oracle, normwise, to_oracle
    from kernels import _native
    from kernels.grouped_gemm import build_fused_gate_up_workspace
    from oracle import oracle

    dtype = torch.bfloat16
    groups, m, f = 4, 300, 264
    n = 2 * f
    ws = build_fused_gate_up_workspace([(m, k, n)] * groups, dtype, seed=4)
    storages = []
    for e in range(groups):
        ws.a[e].copy_(_ints((m, k), dtype))
        ws.b[e].copy_(_ints((k, n), dtype))
        lead = GUARD + (4 if e % 2 else 0)  # odd problems: H only 8-byte aligned
        storage = torch.full((lead + m * f + GUARD,), float("nan"), device="cuda", dtype=dtype)
        storages.append((storage, lead))
    h_ptrs = torch.tensor([s[lead:].data_ptr() for s, lead in storages], device="cuda", dtype=torch.int64)
    code = _native.dtype_code(dtype)
    ping_pong = [t for t in _tiles(dtype) if t[:2] == (256, 256) and t[3] == 8 and t[4] >= 3]
    assert ping_pong
    for bm, bn, bk, warps, stages in ping_pong:
        tiles = groups * -(-m // bm) * -(-f // (bn // 2))
        results = {}
        for grid in (tiles, 1, 5, 8):
            print(f"ping-pong swiglu k={k} tile={(bm, bn, bk, warps, stages)} tiles={tiles} grid={grid}", flush=True)
            for storage, _ in storages:
                storage.fill_(float("nan"))
            status = _native.library().moegemm_grouped_gemm_swiglu(
                ws.a_ptrs.data_ptr(), ws.b_ptrs.data_ptr(), h_ptrs.data_ptr(), ws.dims.data_ptr(),
                ws.strides.data_ptr(), groups, m, n, k, 1, tiles, code, bm, bn, bk, 4, warps, stages, grid, 1,
                0, _native.current_stream_handle(ws.a[0].device))
            _native.check(status)
            torch.cuda.synchronize()
            results[grid] = [s[lead:lead + m * f].clone() for s, lead in storages]
            for e, (storage, lead) in enumerate(storages):
                label = f"k {k} tile {(bm, bn, bk, warps, stages)} grid {grid} problem {e}"
                assert torch.isnan(storage[:lead]).all() and torch.isnan(storage[lead + m * f:]).all(), label
                assert torch.equal(results[grid][e], results[tiles][e]), label
        for e in (0, groups - 1):
            ref = from_oracle(oracle.swiglu_reference(np.ascontiguousarray(to_oracle(ws.a[e])),
                                                      np.ascontiguousarray(to_oracle(ws.b[e])), "bf16"), "bf16")
            assert normwise(results[tiles][e].view(m, f).cpu(), ref) <= 1e-2, f"k {k} problem {e}"
