"""CPU tests of the C ABI boundary: the library loads, exports what include/moegemm.h declares,
and rejects bad arguments with the documented codes before any GPU work."""

from __future__ import annotations

import ctypes
import math
import re
from pathlib import Path

import pytest

from kernels import _native
from kernels.matmul import _MENU_16BIT, _MENU_F32

HEADER = Path(__file__).resolve().parents[1] / "include" / "moegemm.h"


def _declarations() -> dict[str, int]:
    """Function name -> parameter count, parsed from the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    found = {}
    for match in re.finditer(r"\b(moegemm_\w+)\s*\(([^)]*)\)\s*;", text):
        params = match.group(2).strip()
        found[match.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return found


def test_header_declares_every_bound_symbol_and_nothing_else():
    declared = _declarations()
    assert set(declared) == set(_native.SIGNATURES)
    for name, count in declared.items():
        assert len(_native.SIGNATURES[name][1]) == count, name


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.library()
    for name in _declarations():
        assert hasattr(lib, name), name
    assert lib.moegemm_abi_version() == _native.ABI_VERSION
    header_version = int(re.search(r"#define MOEGEMM_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert header_version == _native.ABI_VERSION


def test_buffer_sizes_agree_between_header_and_binding():
    """The caller-allocated stealing queue and the no-alloc scratch limit have one size in C and Python."""
    text = HEADER.read_text()
    queue = int(re.search(r"#define MOEGEMM_QUEUE_BYTES (\d+)", text).group(1))
    assert queue == _native.QUEUE_BYTES
    assert queue % 256 == 0 and queue >= 17 * 256  # 17 counters, one per 256-byte block
    scratch = re.search(r"#define MOEGEMM_NOALLOC_SCRATCH_BYTES \(([^)]*)\)", text).group(1)
    assert re.fullmatch(r"[0-9 *+]+", scratch), scratch
    total = sum(math.prod(int(f) for f in term.split("*")) for term in scratch.split("+"))
    assert total == _native.NOALLOC_SCRATCH_BYTES


def test_compiled_menus_match_python_candidate_pools():
    assert [row[:5] for row in _native.compiled_kernels(_native.DTYPE_BF16)] == list(_MENU_16BIT)
    assert [row[:5] for row in _native.compiled_kernels(_native.DTYPE_F16)] == list(_MENU_16BIT)
    assert [row[:5] for row in _native.compiled_kernels(_native.DTYPE_F32)] == list(_MENU_F32)
    for code in (_native.DTYPE_F16, _native.DTYPE_BF16, _native.DTYPE_F32):
        for row in _native.compiled_kernels(code):
            assert 0 < row[5] <= 160 * 1024  # LDS bytes fit one CU


def _grouped(**overrides):
    args = dict(a=1, b=1, c=1, dims=1, strides=1, g=4, m=16, n=64, k=64, homog=1, tiles=4, dtype=1, prec=0,
                bm=256, bn=256, bk=64, group=8, warps=8, stages=2, grid=4, vec=1, b_stream=0, stream=None)
    args.update(overrides)
    lib = _native.library()
    return lib.moegemm_grouped_gemm(args["a"], args["b"], args["c"], args["dims"], args["strides"], args["g"],
                                    args["m"], args["n"], args["k"], args["homog"], args["tiles"], args["dtype"],
                                    args["prec"], args["bm"], args["bn"], args["bk"], args["group"], args["warps"],
                                    args["stages"], args["grid"], args["vec"], args["b_stream"], args["stream"])


@pytest.mark.parametrize("override, code, needle", [
    ({"dtype": 7}, _native.ERR_INVALID, "dtype"),
    ({"prec": 1}, _native.ERR_INVALID, "tf32"),
    ({"prec": 5}, _native.ERR_INVALID, "precision"),
    ({"group": 0}, _native.ERR_INVALID, "group_size_m"),
    ({"bm": 48}, _native.ERR_NO_KERNEL, "no compiled kernel"),
    ({"stages": 3}, _native.ERR_NO_KERNEL, "no compiled kernel"),
    ({"g": 0}, _native.ERR_INVALID, "problem_count"),
    ({"a": None}, _native.ERR_INVALID, "pointer tables"),
    ({"m": 0}, _native.ERR_INVALID, "shape"),
    ({"homog": 0, "dims": None}, _native.ERR_INVALID, "dims"),
    ({"homog": 0, "tiles": -1}, _native.ERR_INVALID, "total_tiles"),
    ({"b_stream": 2}, _native.ERR_INVALID, "b_stream"),
    ({"b_stream": -1}, _native.ERR_INVALID, "b_stream"),
])
def test_grouped_entry_rejects_bad_arguments_without_launching(override, code, needle):
    assert _grouped(**override) == code
    assert needle in _native.last_error()


def test_grouped_entry_with_no_tiles_is_a_no_op():
    assert _grouped(homog=0, tiles=0) == _native.OK


def test_matmul_entry_rejects_bad_arguments_without_launching():
    lib = _native.library()
    call = lambda **kw: lib.moegemm_matmul(
        kw.get("a", 1), 1, 1, kw.get("m", 4), 4, 4, 4, 1, 4, 1, 4, 1, kw.get("dtype", 1), 0,
        kw.get("bm", 16), 64, 128, 1, 4, 4, 0, 0, None)
    assert call(m=0) == _native.ERR_INVALID and "shape" in _native.last_error()
    assert call(a=None) == _native.ERR_INVALID and "non-null" in _native.last_error()
    assert call(bm=24) == _native.ERR_NO_KERNEL
    assert call(dtype=3) == _native.ERR_INVALID


@pytest.mark.parametrize("m,sam,sbk,scm", [
    (1 << 20, 4096, 64, 64),        # A of 8 GiB: any number of rows
    (300, (1 << 22) - 8, 64, 64),   # the largest A pitch whose 256 rows stay under 2 GiB
    (300, 1 << 22, 64, 64),
    (300, 256, 64, (1 << 22) - 8),  # the same bound on C
    (300, 256, 64, 1 << 22),
    (300, 256, (1 << 22) - 8, 64),  # B [256, n] under 2 GiB
    (300, 256, 1 << 22, 64),
])
def test_fast_layout_byte_limits_match_the_python_mirror(m, sam, sbk, scm):
    """The split-K entry checks the LDS-DMA layout before its workspace, so a layout the library
    accepts fails on the missing workspace instead, and neither reaches a launch."""
    k, n = 256, 64
    status = _native.library().moegemm_matmul_splitk(
        4096, 8192, 12288, m, n, k, sam, 1, sbk, 1, scm, 1, _native.DTYPE_BF16, 256, 256, 32, 8, 8, 4, 2, 0,
        None, 0, 0, None)
    assert status == _native.ERR_INVALID
    accepted = "workspace" in _native.last_error()
    assert accepted != ("vector layout" in _native.last_error())
    assert accepted == _native.panels_fit(k, sam, sbk, scm)


def test_status_mapping_to_python_exceptions():
    assert _grouped(dtype=9) == _native.ERR_INVALID
    with pytest.raises(ValueError):
        _native.check(_native.ERR_INVALID)
    assert _grouped(bm=48) == _native.ERR_NO_KERNEL
    with pytest.raises(RuntimeError):
        _native.check(_native.ERR_NO_KERNEL)
    _native.check(_native.OK)


def test_launches_fail_loudly_without_a_gpu(monkeypatch):
    import torch

    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped
    from kernels.matmul import launch_matmul

    workspace = build_grouped_workspace([(8, 16, 32)] * 2, torch.bfloat16, device="cpu")
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError, match="GPU"):
        launch_grouped(workspace)
    with pytest.raises(ValueError):  # CPU tensors are rejected as a device mismatch first
        launch_matmul(workspace.a[0], workspace.b[0], workspace.c[0])


def test_missing_library_is_a_runtime_error(monkeypatch, tmp_path):
    monkeypatch.setenv("MOEGEMM_LIBRARY", str(tmp_path / "absent.so"))
    _native.library.cache_clear()
    try:
        with pytest.raises(RuntimeError, match="not built"):
            _native.library()
        assert not _native.available()
    finally:
        monkeypatch.delenv("MOEGEMM_LIBRARY")
        _native.library.cache_clear()
    assert isinstance(_native.library(), ctypes.CDLL)


def test_swiglu_tiles_are_exactly_the_even_fragment_tiles():
    """The C library's epilogue flag equals the fragment-pairing rule (even N fragments per wave)."""
    for code in (_native.DTYPE_F16, _native.DTYPE_BF16):
        expected = set()
        for bm, bn, bk, warps, stages, _lds, waves_m in _native.compiled_kernels(code):
            wtm, wtn = bm // waves_m, bn // (warps // waves_m)
            mi = 32 if wtm >= 32 and wtn >= 32 else 16
            if (wtn // mi) % 2 == 0:
                expected.add((bm, bn, bk, warps, stages))
        assert _native.swiglu_tiles(code) == frozenset(expected)
    assert _native.swiglu_tiles(_native.DTYPE_F32) == frozenset()
    assert _native.library().moegemm_kernel_swiglu(_native.DTYPE_BF16, 10_000) < 0


def test_splitk_workspace_has_a_fixed_counter_area():
    """Partials start at the same offset for every launch shape, so launches of different tile
    counts sharing one workspace never write partials over each other's tile counters."""
    sizes = {(tiles, splits, bm, bn): _native.splitk_workspace_bytes(tiles, splits, bm, bn)
             for tiles in (0, 1, 16, 128, 512, 65536) for splits in (2, 16) for bm, bn in ((16, 64), (256, 256))}
    offsets = {nbytes - tiles * splits * bm * bn * 4 for (tiles, splits, bm, bn), nbytes in sizes.items()}
    assert len(offsets) == 1
    (counter_bytes,) = offsets
    assert counter_bytes >= 65536 * 4 and counter_bytes % 256 == 0


def test_splitk_entry_rejects_more_tiles_than_counters_without_launching():
    lib = _native.library()
    m, n, k = 4096, 16448, 1024  # 256 x 257 tiles of 16 x 64: one more column than the counters hold
    status = lib.moegemm_matmul_splitk(256, 256, 256, m, n, k, k, 1, n, 1, n, 1, _native.DTYPE_BF16,
                                       16, 64, 128, 1, 4, 4, 2, 0, None, 0, 0, None)
    assert status == _native.ERR_INVALID and "output tiles" in _native.last_error()


def test_stealing_entries_reject_a_missing_or_misaligned_queue_without_launching():
    lib = _native.library()
    args = (1, 1, 1, 1, 1, 4, 16, 64, 64, 1, 4, _native.DTYPE_BF16, 0, 16, 64, 128, 1, 4, 4, 4, 1)
    assert lib.moegemm_grouped_gemm_stealing(*args, None, 0, None) == _native.ERR_INVALID
    assert "tile queue" in _native.last_error()
    assert lib.moegemm_grouped_gemm_stealing(*args, 4, 0, None) == _native.ERR_INVALID
    assert "256-byte aligned" in _native.last_error()
    offs_args = (256, 256, 256, 256, 2, 16, 64, 64, 64, 64 * 64, 64, 64, _native.DTYPE_BF16, 0, 16, 64, 128, 1, 4, 4, 4)
    assert lib.moegemm_grouped_mm_offs_stealing(*offs_args, None, 0, None) == _native.ERR_INVALID
    assert "tile queue" in _native.last_error()
    assert lib.moegemm_grouped_mm_offs_stealing(*offs_args, 260, 0, None) == _native.ERR_INVALID
    assert "256-byte aligned" in _native.last_error()


def test_stream_buffers_are_not_created_during_graph_capture(monkeypatch):
    import torch

    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="outside capture"):
        _native.tile_queue("cpu", 987654321)
    with pytest.raises(RuntimeError, match="outside capture"):
        _native.splitk_workspace("cpu", 987654321, 1024)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    queue = _native.tile_queue("cpu", 987654321)  # made outside capture: reused afterwards, even under capture
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert _native.tile_queue("cpu", 987654321) is queue
    _native._TILE_QUEUES.pop((0, 987654321))
    _native._SPLITK_WORKSPACES.pop((0, 987654321), None)
