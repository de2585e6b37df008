"""GPU tests of the work-stealing tile scheduler through the C ABI.

Exact-integer known answers (A = 1, B_e = e + 1, so C_e = K (e + 1) exactly) with C poisoned with
NaN before each launch, so a tile that no workgroup took stays NaN; after every launch the queue
must be back to all zeros (the last workgroup re-arms it), which is what lets the next launch and
graph replays run without clearing it.  Grids cover one workgroup, grids that are not a multiple
of 8 (one queue), multiples of 8 (one queue per XCD, with stealing once a queue drains) and one
workgroup per tile; the modes cover homogeneous groups, generic (heterogeneous) groups, and the
offsets layout with more groups than one device prefix chunk (a stolen tile can precede the loaded
chunk) and with offsets clamped so that the device finds fewer tiles than the host bound.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


def _queue():
    from kernels import _native

    return torch.zeros(_native.QUEUE_BYTES // 4, dtype=torch.int32, device="cuda")


def _known_group(shapes, dtype=torch.bfloat16):
    from kernels.grouped_gemm import workspace_from_tensors

    a = [torch.ones((m, k), device="cuda", dtype=dtype) for m, k, _ in shapes]
    b = [torch.full((k, n), float(e % 31 + 1), device="cuda", dtype=dtype) for e, (_, k, n) in enumerate(shapes)]
    c = [torch.empty((m, n), device="cuda", dtype=dtype) for m, _, n in shapes]
    expected = [float(k * (e % 31 + 1)) for e, (_, k, _) in enumerate(shapes)]
    return workspace_from_tensors(a, b, c), expected


def _launch_stealing(ws, cfg, grid, queue):
    from kernels import _native
    from kernels.grouped_gemm import _vector_layout

    dtype_code = _native.dtype_code(ws.a[0].dtype)
    m, k, n = ws.shapes[0]
    status = _native.library().moegemm_grouped_gemm_stealing(
        ws.a_ptrs.data_ptr(), ws.b_ptrs.data_ptr(), ws.c_ptrs.data_ptr(), ws.dims.data_ptr(), ws.strides.data_ptr(),
        ws.problem_count, m, n, k, 1 if ws.homogeneous else 0, ws.tile_count_for(cfg), dtype_code, 0,
        cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages, grid,
        1 if _vector_layout(ws, dtype_code) else 0, queue.data_ptr(), 0, _native.current_stream_handle(ws.a[0].device))
    _native.check(status)


def _check(ws, expected, label):
    for index, (c, value) in enumerate(zip(ws.c, expected)):
        assert torch.all(c == value), f"{label}: problem {index} (NaN = tile never taken)"


@pytest.mark.parametrize("homogeneous", [True, False], ids=["homogeneous", "generic"])
def test_every_grid_size_takes_every_tile_and_rearms_the_queue(homogeneous):
    from kernels.matmul import KernelConfig

    shapes = [(100, 256, 320)] * 12 if homogeneous else [(100 + 7 * e, 64 * (1 + e % 3), 320 - 64 * (e % 2))
                                                          for e in range(12)]
    ws, expected = _known_group(shapes)
    assert ws.homogeneous == homogeneous
    queue = _queue()
    for cfg in (KernelConfig(32, 128, 64, 8, 4, 4, 1), KernelConfig(128, 128, 64, 8, 4, 4, 1),
                KernelConfig(256, 256, 32, 8, 8, 4, 1)):  # the last runs the ping-pong schedule
        tiles = ws.tile_count_for(cfg)
        for grid in sorted({1, 3, 8, 13, 24, 64, tiles - 1, tiles}):
            for repeat in range(2):
                print(f"stealing {'homogeneous' if homogeneous else 'generic'} tile={cfg.tile_key} "
                      f"tiles={tiles} grid={grid} repeat={repeat}", flush=True)
                for c in ws.c:
                    c.fill_(float("nan"))
                _launch_stealing(ws, cfg, grid, queue)
                torch.cuda.synchronize()
                _check(ws, expected, f"tile {cfg.tile_key} grid {grid}")
                assert not queue.any(), f"queue not re-armed: {queue.tolist()}"


def test_offsets_many_groups_steal_across_prefix_chunks_and_clamped_count():
    from kernels import _native
    from kernels.grouped_mm import offsets_tile_bound
    from kernels.matmul import KernelConfig

    groups, k, n = 1300, 32, 48  # > 512 groups: the device prefix sum spans three chunks
    sizes = [(e * 7) % 5 for e in range(groups)]
    ends, total = [], 0
    for size in sizes:
        total += size
        ends.append(total)
    rows = total
    mat_a = torch.ones((rows, k), device="cuda", dtype=torch.bfloat16)
    mat_b = torch.stack([torch.full((k, n), float(e % 31 + 1), device="cuda", dtype=torch.bfloat16)
                         for e in range(groups)])
    expected = torch.empty((rows, n), dtype=torch.float64)
    prev = 0
    for e, end in enumerate(ends):
        expected[prev:end] = float(k * (e % 31 + 1))
        prev = end
    queue = _queue()
    cfg = KernelConfig(16, 64, 128, 8, 4, 4, 1)
    bound = offsets_tile_bound(rows, groups, n, cfg.block_m, cfg.block_n)
    for label, offs_list in (("exact", ends), ("clamped", ends[:600] + [ends[599]] * (groups - 600))):
        offs = torch.tensor(offs_list, device="cuda", dtype=torch.int32)
        covered = offs_list[-1]
        for grid in (8, 16, 24, 40):
            print(f"stealing offsets {label} G={groups} rows={rows} bound={bound} grid={grid}", flush=True)
            out = torch.full((rows, n), float("nan"), device="cuda", dtype=torch.bfloat16)
            status = _native.library().moegemm_grouped_mm_offs_stealing(
                mat_a.data_ptr(), mat_b.data_ptr(), out.data_ptr(), offs.data_ptr(), groups, rows, n, k,
                mat_a.stride(0), mat_b.stride(0), mat_b.stride(1), out.stride(0), _native.DTYPE_BF16, 0,
                cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages, grid,
                queue.data_ptr(), 0, _native.current_stream_handle(mat_a.device))
            _native.check(status)
            torch.cuda.synchronize()
            got = out.double().cpu()
            assert torch.equal(got[:covered], expected[:covered]), f"{label} grid {grid}"
            assert torch.isnan(got[covered:]).all(), f"{label} grid {grid}: rows past offs[-1] written"
            assert not queue.any(), f"queue not re-armed: {queue.tolist()}"


def test_graph_replays_need_no_queue_reset():
    from kernels.grouped_gemm import launch_grouped
    from kernels.matmul import KernelConfig

    ws, expected = _known_group([(64, 128, 256)] * 6)
    cfg = KernelConfig(32, 128, 64, 8, 4, 4, 1)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        launch_grouped(ws, config=cfg, autotune=False, tile_schedule="stealing")  # allocates this stream's queue
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            launch_grouped(ws, config=cfg, autotune=False, tile_schedule="stealing")
    torch.cuda.synchronize()
    for replay in range(4):
        print(f"stealing graph replay {replay}", flush=True)
        for c in ws.c:
            c.fill_(float("nan"))
        launch_grouped(ws, config=cfg, autotune=False, tile_schedule="stealing")  # eager, default stream's queue
        for c in ws.c:
            c.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _check(ws, expected, f"replay {replay}")


@pytest.mark.parametrize("case", [("W1", "EP", 8), ("W1", "EP", 512), ("W2", "TP", 8)], ids=lambda c: "_".join(map(str, c)))
def test_dsv3_full_size_forced_stealing_exact(case):
    from kernels.grouped_gemm import build_fused_gate_up_workspace, build_grouped_workspace, launch_grouped
    from utils.metrics import moe_shapes

    projection, parallel, m = case
    shapes = moe_shapes(projection, parallel, m, 7168, 2048, 256, 8)
    builder = build_fused_gate_up_workspace if projection == "W1" else build_grouped_workspace
    ws = builder(shapes, torch.bfloat16, 1234)
    k = ws.shapes[0][1]
    for index, (a, b, c) in enumerate(ws.problem_tensors()):
        a.fill_(1)
        b.fill_(index % 31 + 1)
    print(f"stealing DSV3 {projection} {parallel} M_e={m} autotuned", flush=True)
    launch_grouped(ws, tile_schedule="stealing")
    assert ws.tile_schedule == "stealing" and ws.split_k == 1
    for c in ws.c:
        c.fill_(float("nan"))
    launch_grouped(ws, config=ws.config, autotune=False, tile_schedule="stealing")
    torch.cuda.synchronize()
    _check(ws, [float(k * (e % 31 + 1)) for e in range(ws.problem_count)], f"DSV3 {case} {ws.config}")


def test_autotuner_measures_both_schedules():
    from kernels import _native
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped

    ws = build_grouped_workspace([(48, 512, 768)] * 16, torch.bfloat16, seed=3)
    print("stealing autotuned schedule choice", flush=True)
    launch_grouped(ws)
    assert ws.tile_schedule in _native.TILE_SCHEDULES
    torch.cuda.synchronize()
    for index in (0, 15):
        reference = ws.a[index].float() @ ws.b[index].float()
        err = float((ws.c[index].float() - reference).abs().max() / reference.abs().max())
        assert err <= 1e-2, f"problem {index}: normwise {err}"
