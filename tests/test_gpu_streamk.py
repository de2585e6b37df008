"""GPU parity tests of the stream-K tail (whole tiles in exact rounds, then the remaining tiles' K
slices spread over every workgroup) through the C ABI and the Python launchers.

Inputs are small random integers, so every product and every fp32 partial sum is exact whatever
the order of the sums: the result must equal the float64 product rounded once to the output
dtype, bit for bit.  A piece that summed the wrong K range, a partial read from another tile's
slot, a lost or doubled piece, a tile stored to the wrong place or a counter left armed changes
that result.  Covered: every compiled 16-bit tile; tails that are part of one round, a whole
round and more (pieces that are whole tiles); K tails; grids that are and are not multiples of 8;
the Mixtral-8x7B W13 EP shape at M_e = 1024 (448 tiles of 256x256 on 256 CUs); repeated launches
and a captured graph replayed with eager work in between on one workspace; fp16; the library's
argument checks; and the Python launchers' "streamk" schedule.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


def _ints(shape, gen, dtype, lo=-2, hi=3):
    return torch.randint(lo, hi, shape, generator=gen, device="cuda").to(dtype)


def _exact(a, b, dtype):
    """The float64 product rounded once to the output dtype (exact for these integer inputs)."""
    return (a.double() @ b.double()).to(dtype)


def _lib():
    from kernels import _native

    return _native, _native.library()


def _workspace(tail, grid, bm, bn):
    native, _ = _lib()
    return torch.zeros(native.streamk_workspace_bytes(tail, grid, bm, bn), dtype=torch.uint8, device="cuda")


def _matmul_streamk(a, b, c, tile, tail, grid, ws, group_m=8):
    native, lib = _lib()
    bm, bn, bk, warps, stages = tile
    return lib.moegemm_matmul_streamk(
        a.data_ptr(), b.data_ptr(), c.data_ptr(), a.shape[0], b.shape[1], a.shape[1],
        a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1), native.dtype_code(a.dtype),
        bm, bn, bk, group_m, warps, stages, tail, grid, ws.data_ptr(), ws.numel(),
        0, native.current_stream_handle(a.device))


def _grouped_streamk(a_list, b_list, c_list, tile, tail, grid, ws, group_m=8):
    native, lib = _lib()
    bm, bn, bk, warps, stages = tile
    ptr = lambda ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device="cuda")  # noqa: E731
    tables = (ptr(a_list), ptr(b_list), ptr(c_list))
    m, k = a_list[0].shape
    n = b_list[0].shape[1]
    status = lib.moegemm_grouped_gemm_streamk(
        tables[0].data_ptr(), tables[1].data_ptr(), tables[2].data_ptr(), len(a_list), m, n, k,
        native.dtype_code(a_list[0].dtype), bm, bn, bk, group_m, warps, stages, tail, grid, 1,
        ws.data_ptr(), ws.numel(), 0, native.current_stream_handle(a_list[0].device))
    return status, tables  # the tables must outlive the launch


def _tiles16():
    native, _ = _lib()
    return [tuple(row[:5]) for row in native.compiled_kernels(native.DTYPE_BF16)]


@pytest.mark.parametrize("tile", _tiles16(), ids=lambda t: "x".join(map(str, t)))
def test_every_tile_single_streamk_tail_exact(tile):
    """A single GEMM with M, N and K tails, 15 tiles: on a grid of 4, three rounds of whole tiles
    and a tail of 3, or a tail of all 15 (runs that hold whole tiles); on grids of 16 and 20 (20 is
    not a multiple of 8, so runs are numbered without the XCD order) every tile is cut into pieces
    across the runs."""
    bm, bn, bk, warps, stages = tile
    gen = torch.Generator(device="cuda").manual_seed(bm * 1000 + bn + bk)
    mt, nt = 3, 5
    m, n, k = mt * bm - bm // 2 + 1, nt * bn - 8, 6 * bk + 24  # M, N and K tails
    a, b = _ints((m, k), gen, torch.bfloat16), _ints((k, n), gen, torch.bfloat16)
    exact = _exact(a, b, torch.bfloat16)
    tiles = mt * nt
    for grid in (4, 16, 20):
        for tail in sorted({tiles % grid or grid // 2, tiles}):
            if tail * ((k + bk - 1) // bk) < grid:
                continue
            print(f"streamk single tile={tile} grid={grid} tail={tail} m={m} n={n} k={k}", flush=True)
            c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
            ws = _workspace(tail, grid, bm, bn)
            assert _matmul_streamk(a, b, c, tile, tail, grid, ws) == 0, _lib()[0].last_error()
            torch.cuda.synchronize()
            assert torch.equal(c, exact), f"tile {tile} grid {grid} tail {tail}"
            assert int(ws[: 256 * 1024].view(torch.int32).abs().sum()) == 0, "counters must be left zero"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_streamk_tails_exact(dtype):
    """Homogeneous groups on the ping-pong tile and a two-stage tile: tails of part of a round,
    of all tiles (fewer tiles than workgroups) and of runs that hold whole tiles."""
    gen = torch.Generator(device="cuda").manual_seed(7)
    g, m, k, n = 5, 300, 1000, 520
    a = [_ints((m, k), gen, dtype) for _ in range(g)]
    b = [_ints((k, n), gen, dtype) for _ in range(g)]
    exact = [_exact(x, y, dtype) for x, y in zip(a, b)]
    for tile in ((256, 256, 32, 8, 4), (64, 128, 64, 4, 2), (128, 256, 64, 8, 3)):
        bm, bn, bk = tile[:3]
        tiles = g * -(-m // bm) * -(-n // bn)
        kt = -(-k // bk)
        for grid, tail in ((8, tiles % 8 or 4), (20, tiles % 20 or 10), (32, tiles % 32 or 16), (8, tiles),
                           (256, tiles)):
            per_run = tail * kt // grid
            if per_run < 1 or -(-kt // per_run) + 1 > 64:
                continue  # a plan the library rejects (covered by test_library_rejects_bad_streamk_plans)
            print(f"streamk grouped {dtype} tile={tile} tiles={tiles} grid={grid} tail={tail}", flush=True)
            c = [torch.full((m, n), float("nan"), device="cuda", dtype=dtype) for _ in range(g)]
            ws = _workspace(tail, grid, bm, bn)
            status, _tables = _grouped_streamk(a, b, c, tile, tail, grid, ws)
            assert status == 0, _lib()[0].last_error()
            torch.cuda.synchronize()
            for e in range(g):
                assert torch.equal(c[e], exact[e]), f"tile {tile} grid {grid} tail {tail} problem {e}"


def test_mixtral_w13_ep_me1024_shape_exact():
    """[1024,4096]@[4096,28672]: 448 tiles of 256x256 on 256 workgroups, 192 of them in the tail."""
    gen = torch.Generator(device="cuda").manual_seed(11)
    m, k, n = 1024, 4096, 28672
    a, b = _ints((m, k), gen, torch.bfloat16), _ints((k, n), gen, torch.bfloat16)
    exact = _exact(a, b, torch.bfloat16)
    c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    tile = (256, 256, 32, 8, 4)
    ws = _workspace(192, 256, 256, 256)
    print("streamk Mixtral W13 EP M_e=1024 tail=192 grid=256", flush=True)
    assert _matmul_streamk(a, b, c, tile, 192, 256, ws) == 0, _lib()[0].last_error()
    torch.cuda.synchronize()
    assert torch.equal(c, exact)


def test_repeated_launches_and_graph_replay_share_one_workspace():
    """Launches of different shapes and tails in a row, then a captured launch replayed three times
    with eager launches in between, all on one workspace: every launch must leave the counters
    zero, and every result must be exact."""
    gen = torch.Generator(device="cuda").manual_seed(5)
    tile = (256, 256, 32, 8, 4)
    grid = 64
    ws = _workspace(64, grid, 256, 256)
    shapes = [(700, 1504, 2104), (300, 2000, 1800), (1100, 640, 1304)]  # K, N multiples of 8
    operands = []
    for m, k, n in shapes:
        a, b = _ints((m, k), gen, torch.bfloat16), _ints((k, n), gen, torch.bfloat16)
        tiles = -(-m // 256) * -(-n // 256)
        operands.append((a, b, _exact(a, b, torch.bfloat16), tiles % grid or grid // 4))
    for a, b, exact, tail in operands:
        c = torch.full(exact.shape, float("nan"), device="cuda", dtype=torch.bfloat16)
        print(f"streamk repeated shape={tuple(a.shape)}x{b.shape[1]} tail={tail}", flush=True)
        assert _matmul_streamk(a, b, c, tile, tail, grid, ws) == 0, _lib()[0].last_error()
        torch.cuda.synchronize()
        assert torch.equal(c, exact)
    a0, b0, exact0, tail0 = operands[0]
    a1, b1, exact1, tail1 = operands[1]
    c0 = torch.full(exact0.shape, float("nan"), device="cuda", dtype=torch.bfloat16)
    c1 = torch.empty(exact1.shape, device="cuda", dtype=torch.bfloat16)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        assert _matmul_streamk(a0, b0, c0, tile, tail0, grid, ws) == 0  # warm up on the capture stream
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            assert _matmul_streamk(a0, b0, c0, tile, tail0, grid, ws) == 0
    torch.cuda.current_stream().wait_stream(stream)
    for replay in range(3):
        print(f"streamk graph replay {replay}", flush=True)
        c0.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c0, exact0), f"replay {replay}"
        c1.fill_(float("nan"))
        assert _matmul_streamk(a1, b1, c1, tile, tail1, grid, ws) == 0
        torch.cuda.synchronize()
        assert torch.equal(c1, exact1), f"eager launch after replay {replay}"
    assert int(ws[: 256 * 1024].view(torch.int32).abs().sum()) == 0


def test_library_rejects_bad_streamk_plans():
    native, lib = _lib()
    a = torch.zeros((512, 512), device="cuda", dtype=torch.bfloat16)
    b = torch.zeros((512, 512), device="cuda", dtype=torch.bfloat16)
    c = torch.zeros((512, 512), device="cuda", dtype=torch.bfloat16)
    tile = (256, 256, 32, 8, 4)
    ws = _workspace(4, 256, 256, 256)
    # 4 tiles: a tail past the tile count, an empty tail, and a tail too thin for 256 runs (16 K
    # slices per tile).
    for tail, grid in ((5, 8), (0, 8), (1, 256)):
        assert _matmul_streamk(a, b, c, tile, tail, grid, ws) == native.ERR_INVALID
    small = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    assert _matmul_streamk(a, b, c, tile, 4, 8, small) == native.ERR_INVALID
    assert "workspace" in native.last_error()
    odd = torch.zeros(ws.numel() + 512, dtype=torch.uint8, device="cuda")[16:]
    assert _matmul_streamk(a, b, c, tile, 4, 8, odd) == native.ERR_INVALID
    assert "aligned" in native.last_error()
    at = a.t()  # not the vector layout (non-unit inner stride)
    assert _matmul_streamk(at, b, c, tile, 4, 8, ws) == native.ERR_INVALID
    assert _matmul_streamk(a.float(), b.float(), c.float(), (128, 128, 32, 4, 2), 4, 8, ws) in (
        native.ERR_INVALID, native.ERR_NO_KERNEL)


def test_python_launchers_run_the_streamk_schedule():
    from kernels.grouped_gemm import launch_grouped, workspace_from_tensors
    from kernels.matmul import STREAMK, KernelConfig, _launch_fixed, last_matmul_schedule

    gen = torch.Generator(device="cuda").manual_seed(3)
    g, m, k, n = 3, 512, 2048, 2560  # 3 x 2 x 10 = 60 tiles of 256x256: a partial round on any GPU
    a = [_ints((m, k), gen, torch.bfloat16) for _ in range(g)]
    b = [_ints((k, n), gen, torch.bfloat16) for _ in range(g)]
    exact = [_exact(x, y, torch.bfloat16) for x, y in zip(a, b)]
    c = [torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16) for _ in range(g)]
    ws = workspace_from_tensors(a, b, c)
    cfg = KernelConfig(256, 256, 32, 8, 8, 4, 1)
    print("streamk launch_grouped pinned", flush=True)
    launch_grouped(ws, config=cfg, autotune=False, tile_schedule="streamk")
    torch.cuda.synchronize()
    assert ws.tile_schedule == "streamk" and ws.split_k == 1
    for e in range(g):
        assert torch.equal(ws.c[e], exact[e])
    print("streamk launch_grouped autotuned", flush=True)
    for ce in ws.c:
        ce.fill_(float("nan"))
    launch_grouped(ws)  # the tuner also measures the streamk candidates
    torch.cuda.synchronize()
    assert ws.tile_schedule in ("static", "stealing", "streamk")
    for e in range(g):
        assert torch.equal(ws.c[e], exact[e])
    print("streamk single GEMM launcher", flush=True)
    from kernels import _native

    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    assert _launch_fixed(a[0], b[0], out, m, n, k, cfg, _native.DTYPE_BF16, _native.PRECISION_IEEE, STREAMK) == 1
    torch.cuda.synchronize()
    assert last_matmul_schedule() == STREAMK
    assert torch.equal(out, exact[0])
