"""GPU parity tests of the expert-sorted layout (2-D A, 3-D B, int32 offsets) through the C ABI.

The checker is ``oracle.grouped_mm_offsets`` (pinned against torch's CPU grouped_mm in
tests/test_oracle.py).  Exact integers are compared bit for bit; seeded random inputs use the
normwise bound max|C - R| / max|R| (bf16 <= 1e-2, fp16 <= 2e-3, fp32 <= 1e-5).  Cases: ragged
offsets with empty groups and rows past the last offset (which must stay untouched), every
compiled 16-bit tile, more groups than one LDS prefix chunk, offsets past the end of A (clamped
on the device), a DeepSeek-V3 EP W13 shard on sampled rows, and a captured graph replayed with
offsets rewritten in place between replays (the kernel reads them at run time).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import DTYPE_NAME, from_oracle, normwise, to_oracle
from oracle import oracle

pytestmark = pytest.mark.gpu

NORMWISE = {"bf16": 1e-2, "fp16": 2e-3, "fp32": 1e-5}
DTYPES = (torch.float16, torch.bfloat16, torch.float32)


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")
    torch.manual_seed(11)


def _oracle(mat_a, mat_b, offs_list):
    name = DTYPE_NAME[mat_a.dtype]
    c = oracle.grouped_mm_offsets(np.ascontiguousarray(to_oracle(mat_a)), np.ascontiguousarray(to_oracle(mat_b)),
                                  offs_list, name)
    return from_oracle(c, name)


def _small_ints(shape, dtype=torch.bfloat16):
    return torch.randint(-2, 3, shape, device="cuda").to(dtype)


def _operands(rows, k, n, groups, dtype, *, integer=False):
    if integer:
        mat_a = torch.ones((rows, k), device="cuda", dtype=dtype)
        mat_b = torch.stack([torch.full((k, n), float(e + 1), device="cuda", dtype=dtype) for e in range(groups)])
    else:
        mat_a = torch.randn((rows, k), device="cuda", dtype=dtype) / math.sqrt(k)
        mat_b = torch.randn((groups, k, n), device="cuda", dtype=dtype) / math.sqrt(k)
    return mat_a, mat_b


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DTYPE_NAME[d])
def test_ragged_offsets_random_inputs(dtype):
    from kernels.grouped_mm import grouped_mm

    rows, k, n = 203, 136, 72
    offs_list = [17, 17, 90, 91, 160]  # empty group, single-row group, rows 160..202 past the end
    print(f"offsets ragged dtype={DTYPE_NAME[dtype]} rows={rows} k={k} n={n} offs={offs_list}", flush=True)
    mat_a, mat_b = _operands(rows, k, n, len(offs_list), dtype)
    offs = torch.tensor(offs_list, device="cuda", dtype=torch.int32)
    out = torch.full((rows, n), float("nan"), device="cuda", dtype=dtype)
    grouped_mm(mat_a, mat_b, offs, out=out)
    torch.cuda.synchronize()
    covered = offs_list[-1]
    expected = _oracle(mat_a, mat_b, offs_list)
    assert torch.isfinite(out[:covered]).all()
    assert normwise(out[:covered], expected[:covered]) <= NORMWISE[DTYPE_NAME[dtype]]
    assert torch.isnan(out[covered:]).all(), "rows past offs[-1] were written"


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DTYPE_NAME[d])
def test_exact_integers_every_compiled_tile(dtype):
    from kernels import _native
    from kernels.grouped_mm import grouped_mm
    from kernels.matmul import KernelConfig

    rows, k, n = 150, 96, 80
    offs_list = [0, 33, 33, 120, 150]
    mat_a, mat_b = _operands(rows, k, n, len(offs_list), dtype, integer=True)
    offs = torch.tensor(offs_list, device="cuda", dtype=torch.int32)
    expected = torch.empty((rows, n), dtype=torch.float64)
    prev = 0
    for e, end in enumerate(offs_list):
        expected[prev:end] = float(k * (e + 1))
        prev = end
    for bm, bn, bk, warps, stages, *_ in _native.compiled_kernels(_native.dtype_code(dtype)):
        cfg = KernelConfig(bm, bn, bk, 8, warps, stages, 1)
        print(f"offsets exact dtype={DTYPE_NAME[dtype]} tile={cfg.tile_key}", flush=True)
        out = torch.full((rows, n), float("nan"), device="cuda", dtype=dtype)
        grouped_mm(mat_a, mat_b, offs, out=out, config=cfg)
        torch.cuda.synchronize()
        assert torch.equal(out.double().cpu(), expected), f"tile {cfg.tile_key}"


def test_many_groups_cross_prefix_chunks_and_clamped_offsets():
    from kernels.grouped_mm import grouped_mm
    from kernels.matmul import KernelConfig

    groups, k, n = 1300, 32, 48  # > 1024 groups: the device prefix sum spans several chunks
    rng = np.random.default_rng(5)
    sizes = rng.integers(0, 5, size=groups)
    ends = np.cumsum(sizes).astype(np.int64)
    rows = int(ends[-1])
    mat_a, mat_b = _operands(rows, k, n, groups, torch.bfloat16, integer=True)
    offs_list = [int(v) for v in ends]
    offs = torch.tensor(offs_list, device="cuda", dtype=torch.int32)
    expected = torch.empty((rows, n), dtype=torch.float64)
    prev = 0
    for e, end in enumerate(offs_list):
        # B holds bf16(e + 1); k times it is exact in the fp32 accumulator
        expected[prev:end] = k * float(torch.tensor(float(e + 1)).to(torch.bfloat16))
        prev = end
    for cfg in (KernelConfig(16, 64, 128, 8, 4, 4, 1), KernelConfig(64, 64, 64, 8, 4, 4, 1)):
        print(f"offsets many groups G={groups} rows={rows} tile={cfg.tile_key}", flush=True)
        out = torch.full((rows, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        grouped_mm(mat_a, mat_b, offs, out=out, config=cfg)
        torch.cuda.synchronize()
        # exact-integer values k*(e+1) exceed bf16's 8-bit mantissa; compare to their bf16 rounding
        assert torch.equal(out.double().cpu(), expected.to(torch.bfloat16).double())
    # Offsets past the end of A are clamped on the device: the last group ends at `rows`.
    clamped = offs_list[:-1] + [rows + 1000]
    offs.copy_(torch.tensor(clamped, dtype=torch.int32))
    out = torch.full((rows, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    print("offsets clamped last offset", flush=True)
    grouped_mm(mat_a, mat_b, offs, out=out, config=KernelConfig(16, 64, 128, 8, 4, 4, 1))
    torch.cuda.synchronize()
    assert torch.equal(out.double().cpu(), expected.to(torch.bfloat16).double())


def test_dsv3_ep_w13_shard_sampled_rows():
    from kernels.grouped_mm import build_offsets_workspace, launch_grouped_offsets

    rng = np.random.default_rng(9)
    sizes = [int(v) for v in rng.integers(300, 700, size=32)]  # ragged routing around M_e = 512
    shapes = [(m, 7168, 4096) for m in sizes]
    print(f"offsets DSV3 EP W13 rows={sum(sizes)}", flush=True)
    ws = build_offsets_workspace(shapes, torch.bfloat16, seed=1234, operation="gate_up")
    launch_grouped_offsets(ws)
    torch.cuda.synchronize()
    assert ws.scheduler == "offsets_persistent" and ws.config is not None
    for index, (a_e, b_e, c_e) in enumerate(ws.problem_tensors()):
        if index not in (0, 13, 31):
            continue
        rows = torch.tensor([0, a_e.shape[0] // 2, a_e.shape[0] - 1])
        expected = a_e[rows].float() @ b_e.float()
        got = c_e[rows].float()
        assert normwise(got.cpu(), expected.cpu()) <= 1e-2


def test_graph_replay_reads_offsets_at_run_time():
    from kernels.grouped_mm import grouped_mm
    from kernels.matmul import KernelConfig

    rows, k, n, groups = 96, 64, 64, 3
    mat_a, mat_b = _operands(rows, k, n, groups, torch.float16, integer=True)
    offs = torch.tensor([10, 50, 96], device="cuda", dtype=torch.int32)
    out = torch.zeros((rows, n), device="cuda", dtype=torch.float16)
    cfg = KernelConfig(32, 128, 64, 8, 4, 4, 1)
    grouped_mm(mat_a, mat_b, offs, out=out, config=cfg)  # warm outside capture
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            grouped_mm(mat_a, mat_b, offs, out=out, config=cfg)
    torch.cuda.synchronize()
    for offs_list in ([10, 50, 96], [40, 41, 96], [0, 0, 96], [96, 96, 96]):
        print(f"offsets graph replay offs={offs_list}", flush=True)
        offs.copy_(torch.tensor(offs_list, dtype=torch.int32))
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        expected = torch.empty((rows, n), dtype=torch.float64)
        prev = 0
        for e, end in enumerate(offs_list):
            expected[prev:end] = float(k * (e + 1))
            prev = end
        assert torch.equal(out.double().cpu(), expected)


def test_validation_errors():
    from kernels.grouped_mm import grouped_mm

    a = torch.zeros((8, 16), device="cuda", dtype=torch.bfloat16)
    b = torch.zeros((2, 16, 8), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        grouped_mm(a, b, torch.tensor([4, 8], device="cuda", dtype=torch.int64))
    with pytest.raises(ValueError):
        grouped_mm(a, b, torch.tensor([8], device="cuda", dtype=torch.int32))
    with pytest.raises(ValueError):
        grouped_mm(a, b[:, :8], torch.tensor([4, 8], device="cuda", dtype=torch.int32))
    with pytest.raises(ValueError):
        grouped_mm(a.t(), b, torch.tensor([4, 8], device="cuda", dtype=torch.int32))


def _lognormal_rows(seed: int, groups: int = 32, mean: int = 512, sigma: float = 0.6) -> list[int]:
    """Ragged routing: lognormal rows per expert around `mean`, with one empty and one single-row expert."""
    rng = np.random.default_rng(seed)
    sizes = [int(round(v)) for v in np.exp(rng.normal(math.log(mean) - sigma * sigma / 2, sigma, size=groups))]
    sizes[5], sizes[9] = 0, 1
    return sizes


@pytest.mark.parametrize("mean", [512, 64])
@pytest.mark.parametrize("schedule", ["static", "stealing"])
def test_dsv3_lognormal_routing_exact_and_oracle(schedule, mean):
    """DSV3 EP W13 shard (32 experts, K = 7168, N = 4096) with lognormal routing around `mean` rows:
    exact integers on every expert and oracle tail rows of the first and last non-empty experts,
    under each tile schedule with the autotuned config of that schedule."""
    from kernels.grouped_mm import grouped_mm

    sizes = _lognormal_rows(2024, mean=mean)
    offs_list = list(np.cumsum(sizes))
    rows, k, n, groups = offs_list[-1], 7168, 4096, len(sizes)
    print(f"offsets DSV3 lognormal mean={mean} schedule={schedule} rows={rows} sizes={sizes}", flush=True)
    offs = torch.tensor(offs_list, device="cuda", dtype=torch.int32)
    mat_a, mat_b = _operands(rows, k, n, groups, torch.bfloat16)
    out = torch.full((rows, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    grouped_mm(mat_a, mat_b, offs, out=out, tile_schedule=schedule)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    nonempty = [e for e, m in enumerate(sizes) if m]
    for e in (nonempty[0], nonempty[-1]):
        r1 = offs_list[e]
        tail = slice(max(r1 - 3, r1 - sizes[e]), r1)
        expected = from_oracle(oracle.gemm(to_oracle(mat_a[tail]), to_oracle(mat_b[e]), "bf16"), "bf16")
        assert normwise(out[tail].cpu(), expected) <= 1e-2, f"expert {e}"
    # Exact check of every row: small random integers in A and in each expert's B, so every fp32
    # sum is an exact integer (|sum| <= 4 K < 2^24) and the one rounding to bf16 is the reference's
    # own.  An fp32 torch product of integer operands is exact too, whatever its summation order.
    mat_a.copy_(_small_ints((rows, k)))
    mat_b.copy_(_small_ints((groups, k, n)))
    out.fill_(float("nan"))
    grouped_mm(mat_a, mat_b, offs, out=out, tile_schedule=schedule)
    torch.cuda.synchronize()
    for e in range(groups):
        r0, r1 = (offs_list[e - 1] if e else 0), offs_list[e]
        if r1 > r0:
            expected = (mat_a[r0:r1].float() @ mat_b[e].float()).to(torch.bfloat16)
            assert torch.equal(out[r0:r1], expected), f"expert {e}"


@pytest.mark.parametrize("schedule", ["static", "stealing"])
@pytest.mark.parametrize("k", [64, 136, 328])
def test_chained_tiles_on_ragged_offsets_small_grids(k, schedule):
    """Offsets launches whose groups fit one prefix chunk run the chained schedule: every chained
    tile (two-stage tiles up to 64 rows, the ping-pong tile), at grids that give each workgroup many
    ragged tiles, empty groups included, rows past the last offset left untouched, static and
    stealing.  A and every group's B hold small random integers, so each output is an exact integer
    sum rounded once to bf16: a stale or wrong K slice, N tile or M tile, even from the same group,
    changes some row, and every row is compared bit for bit with a float64 product per group."""
    from kernels import _native

    sizes = [70, 0, 3, 130, 257, 0, 1, 64, 200, 9]
    ends = list(np.cumsum(sizes))
    groups, rows, n = len(sizes), int(ends[-1]), 392
    spare = 5  # rows past the last offset: never written
    mat_a = _small_ints((rows + spare, k))
    mat_b = _small_ints((groups, k, n))
    offs = torch.tensor(ends, device="cuda", dtype=torch.int32)
    a64, b64 = mat_a.double().cpu(), mat_b.double().cpu()
    expected = torch.full((rows + spare, n), float("nan"), dtype=torch.float64)
    prev = 0
    for e, end in enumerate(ends):
        expected[prev:end] = a64[prev:end] @ b64[e]
        prev = end
    expected = expected.to(torch.bfloat16)
    chained = [t for t in _native.compiled_kernels(_native.DTYPE_BF16)
               if (t[4] == 2 and t[0] <= 64) or (t[:2] == (256, 256) and t[3] == 8 and t[4] >= 3)]
    assert chained
    for bm, bn, bk, warps, stages, *_ in chained:
        for grid in (1, 5, 8):
            print(f"offsets chained {schedule} k={k} tile={(bm, bn, bk, warps, stages)} grid={grid}", flush=True)
            out = torch.full((rows + spare, n), float("nan"), device="cuda", dtype=torch.bfloat16)
            args = (mat_a.data_ptr(), mat_b.data_ptr(), out.data_ptr(), offs.data_ptr(), groups, rows, n, k,
                    mat_a.stride(0), mat_b.stride(0), mat_b.stride(1), out.stride(0), _native.DTYPE_BF16, 0,
                    bm, bn, bk, 4, warps, stages, grid)
            stream = _native.current_stream_handle(mat_a.device)
            if schedule == "stealing":
                queue = torch.zeros(_native.QUEUE_BYTES // 4, dtype=torch.int32, device="cuda")
                status = _native.library().moegemm_grouped_mm_offs_stealing(*args, queue.data_ptr(), 0, stream)
            else:
                status = _native.library().moegemm_grouped_mm_offs(*args, 0, stream)
            _native.check(status)
            torch.cuda.synchronize()
            if schedule == "stealing":
                assert not queue.any(), f"queue not re-armed: {queue.tolist()}"
            label = f"{schedule} k {k} tile {(bm, bn, bk, warps, stages)} grid {grid}"
            got = out.cpu()
            bad = (got[:rows] != expected[:rows]).any(dim=1).nonzero().flatten().tolist()
            assert not bad, f"{label}: rows {bad[:8]} differ"
            assert torch.isnan(got[rows:]).all(), label
