"""GPU tests of operands past the 32-bit byte ranges of the LDS-DMA kernels' buffer resources.

The fast kernels address A and C through one buffer resource per tile (at most 256 rows) and B
through one resource running to the end of the matrix, all with 32-bit byte offsets.  So A and C
may hold any number of rows as long as 256 of their rows stay under 2 GiB, and B must stay under
2 GiB; the library sends any other layout to the general kernel, which uses 64-bit pointers.

Cases, through the C ABI:
* a single GEMM and an expert-sorted launch whose A is 4.36 GB, so tiles start past the 2 GiB and
  4 GiB byte offsets: the ping-pong tile, a chained two-stage tile, the stream-K tail and work
  stealing;
* A and C row pitches just under the per-tile limit (fast kernel) and past it (general kernel).
  A C pitch of 2^23 + 64 elements makes 256 rows span more than 4 GiB, which the fast kernel's
  32-bit store offsets cannot address, so the library must route it to the general kernel.

Inputs are small integers: every product and sum is an integer below 2^24, so the float64 torch
product rounded to bf16 is the exact expected output, compared bit for bit.  Guard rows and
columns outside the written region must keep their NaN fill.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

PINGPONG = (256, 256, 32, 8, 4)
TWO_STAGE = (16, 256, 64, 4, 2)
CHUNK = 65536
NAN = float("nan")


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


def _lib():
    from kernels import _native

    return _native, _native.library()


def _grid():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _fill_ints(t, seed):
    """Integers in [-2, 2] into a 2-D (possibly row-strided) bf16 view, CHUNK rows at a time."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    for i in range(0, t.shape[0], CHUNK):
        j = min(t.shape[0], i + CHUNK)
        t[i:j] = torch.randint(-2, 3, (j - i, t.shape[1]), device="cuda", dtype=torch.int8, generator=g).to(t.dtype)
    return t


def _assert_product(c, a, b, label):
    """c == a @ b rounded to c's dtype, bit for bit, CHUNK rows at a time."""
    b64 = b.double()
    for i in range(0, a.shape[0], CHUNK):
        j = min(a.shape[0], i + CHUNK)
        expected = (a[i:j].double() @ b64).to(c.dtype)
        bad = (c[i:j] != expected).any(dim=1).nonzero().flatten()
        assert bad.numel() == 0, f"{label}: rows {(bad[:8] + i).tolist()} differ"


def _matmul(a, b, c, tile, grid):
    native, lib = _lib()
    bm, bn, bk, warps, stages = tile
    return lib.moegemm_matmul(
        a.data_ptr(), b.data_ptr(), c.data_ptr(), a.shape[0], b.shape[1], a.shape[1], a.stride(0), a.stride(1),
        b.stride(0), b.stride(1), c.stride(0), c.stride(1), native.DTYPE_BF16, 0, bm, bn, bk, 8, warps, stages,
        grid, 0, native.current_stream_handle(a.device))


def _offsets(a, b3, out, offs, tile, grid, queue=None):
    native, lib = _lib()
    bm, bn, bk, warps, stages = tile
    args = (a.data_ptr(), b3.data_ptr(), out.data_ptr(), offs.data_ptr(), b3.shape[0], a.shape[0], b3.shape[2],
            a.shape[1], a.stride(0), b3.stride(0), b3.stride(1), out.stride(0), native.DTYPE_BF16, 0,
            bm, bn, bk, 8, warps, stages, grid)
    stream = native.current_stream_handle(a.device)
    if queue is None:
        return lib.moegemm_grouped_mm_offs(*args, 0, stream)
    return lib.moegemm_grouped_mm_offs_stealing(*args, queue.data_ptr(), 0, stream)


def test_single_gemm_with_a_over_4gib():
    native, lib = _lib()
    m, k, n = 532_557, 4096, 256
    assert m * k * 2 > 1 << 32 and native.panels_fit(k, k, n, n)
    a = _fill_ints(torch.empty((m, k), device="cuda", dtype=torch.bfloat16), 1)
    b = _fill_ints(torch.empty((k, n), device="cuda", dtype=torch.bfloat16), 2)
    guarded = torch.empty((m + 1, n), device="cuda", dtype=torch.bfloat16)
    c = guarded[:m]
    grid = _grid()
    for tile in (PINGPONG, TWO_STAGE):
        print(f"large single m={m} k={k} n={n} tile={tile} grid={grid}", flush=True)
        guarded.fill_(NAN)
        native.check(_matmul(a, b, c, tile, grid))
        torch.cuda.synchronize()
        _assert_product(c, a, b, f"single {tile}")
        assert torch.isnan(guarded[m]).all()
    bm, bn, bk, warps, stages = PINGPONG
    tiles = -(-m // bm) * -(-n // bn)
    tail = native.streamk_tail(tiles, grid, k, bk)
    assert tail > 0
    ws = torch.zeros(native.streamk_workspace_bytes(tail, grid, bm, bn), dtype=torch.uint8, device="cuda")
    print(f"large single stream-K tiles={tiles} tail={tail} grid={grid}", flush=True)
    guarded.fill_(NAN)
    native.check(lib.moegemm_matmul_streamk(
        a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, a.stride(0), 1, b.stride(0), 1, c.stride(0), 1,
        native.DTYPE_BF16, bm, bn, bk, 8, warps, stages, tail, grid, ws.data_ptr(), ws.numel(),
        0, native.current_stream_handle(a.device)))
    torch.cuda.synchronize()
    _assert_product(c, a, b, "single stream-K")
    assert torch.isnan(guarded[m]).all()


@pytest.mark.parametrize("schedule", ["static", "stealing"])
def test_expert_sorted_with_a_over_4gib(schedule):
    native, _ = _lib()
    rows, k, n = 532_557, 4096, 256
    # Group ends straddle the 2 GiB (row 262,144) and 4 GiB (row 524,288) byte offsets of A; group 1
    # is empty.
    ends = [70_001, 70_001, 200_003, 262_161, 400_009, 524_293, 530_000, rows]
    groups = len(ends)
    a = _fill_ints(torch.empty((rows, k), device="cuda", dtype=torch.bfloat16), 3)
    b3 = _fill_ints(torch.empty((groups * k, n), device="cuda", dtype=torch.bfloat16), 4).view(groups, k, n)
    offs = torch.tensor(ends, dtype=torch.int32, device="cuda")
    guarded = torch.full((rows + 1, n), NAN, device="cuda", dtype=torch.bfloat16)
    out = guarded[:rows]
    queue = torch.zeros(native.QUEUE_BYTES // 4, dtype=torch.int32, device="cuda") if schedule == "stealing" else None
    print(f"large offsets {schedule} rows={rows} k={k} n={n} groups={groups} tile={PINGPONG}", flush=True)
    native.check(_offsets(a, b3, out, offs, PINGPONG, _grid(), queue))
    torch.cuda.synchronize()
    prev = 0
    for e, end in enumerate(ends):
        if end > prev:
            _assert_product(out[prev:end], a[prev:end], b3[e], f"offsets {schedule} group {e}")
        prev = end
    assert torch.isnan(guarded[rows]).all()
    if queue is not None:
        assert not queue.any(), "queue not re-armed"


@pytest.mark.parametrize("pitch", [(1 << 22) - 8, (1 << 23) + 64], ids=["fast", "general"])
@pytest.mark.parametrize("operand", ["a", "c"])
def test_row_pitch_at_the_panel_limit(operand, pitch):
    native, _ = _lib()
    m, k, n = 300, 256, 64
    sam = pitch if operand == "a" else k
    scm = pitch if operand == "c" else n
    assert native.panels_fit(k, sam, n, scm) == (pitch < 1 << 22)
    a_store = torch.empty((m, sam), device="cuda", dtype=torch.bfloat16)
    a = _fill_ints(a_store[:, :k], 5)
    b = _fill_ints(torch.empty((k, n), device="cuda", dtype=torch.bfloat16), 6)
    b3 = _fill_ints(torch.empty((2 * k, n), device="cuda", dtype=torch.bfloat16), 7).view(2, k, n)
    c_store = torch.empty((m, scm), device="cuda", dtype=torch.bfloat16)
    c = c_store[:, :n]
    ends = [120, m]
    offs = torch.tensor(ends, dtype=torch.int32, device="cuda")
    grid = _grid()
    for tile in (PINGPONG, TWO_STAGE):
        label = f"pitch {operand}={pitch} tile={tile}"
        print(f"{label} single", flush=True)
        c_store.fill_(NAN)
        native.check(_matmul(a, b, c, tile, grid))
        torch.cuda.synchronize()
        _assert_product(c, a, b, f"{label} single")
        assert torch.isnan(c_store[:, n:]).all(), f"{label} single: written past column {n}"
        print(f"{label} expert-sorted", flush=True)
        c_store.fill_(NAN)
        native.check(_offsets(a, b3, c, offs, tile, grid))
        torch.cuda.synchronize()
        _assert_product(c[:120], a[:120], b3[0], f"{label} group 0")
        _assert_product(c[120:], a[120:], b3[1], f"{label} group 1")
        assert torch.isnan(c_store[:, n:]).all(), f"{label} expert-sorted: written past column {n}"
