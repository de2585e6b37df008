"""GPU parity tests of the non-temporal B copy policy (``b_stream`` = 1) through the C ABI and the
Python launchers.

The policy sets the cache hint of the LDS-DMA kernels' B copies and nothing else, so every output
must be bit-identical to the float64 product rounded to the operand dtype, as with ordinary copies.
Inputs are small random integers (every fp32 sum is exact).  Covered: every compiled 16-bit tile as
a single GEMM with M, N and K tails; homogeneous groups on the static and work-stealing schedules;
split-K and the stream-K tail; the expert-sorted layout; the fused SwiGLU epilogue; the autotuned
launchers, which time the policy on their finalists and record what ran; and argument checks.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


def _ints(shape, gen, dtype=torch.bfloat16):
    return torch.randint(-2, 3, shape, device="cuda", generator=gen).to(dtype)


def _exact(a, b, dtype):
    return (a.double() @ b.double()).to(dtype)


def _tiles16():
    from kernels import _native

    return [tuple(row[:5]) for row in _native.compiled_kernels(_native.DTYPE_BF16)]


@pytest.mark.parametrize("tile", _tiles16(), ids=lambda t: "x".join(map(str, t)))
def test_every_tile_single_gemm_exact_with_streamed_b(tile):
    from kernels.matmul import KernelConfig, last_matmul_b_stream, launch_matmul

    bm, bn, bk, warps, stages = tile
    gen = torch.Generator(device="cuda").manual_seed(bm * 7 + bn + bk)
    m, n, k = 2 * bm + 5, 3 * bn - 8, 5 * bk + 24
    a, b = _ints((m, k), gen), _ints((k, n), gen)
    c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    print(f"b_stream single tile={tile} m={m} n={n} k={k}", flush=True)
    launch_matmul(a, b, c, KernelConfig(bm, bn, bk, 8, warps, stages), autotune=False, split_k=1, b_stream=1)
    torch.cuda.synchronize()
    assert last_matmul_b_stream() == 1
    assert torch.equal(c, _exact(a, b, torch.bfloat16)), f"tile {tile}"


@pytest.mark.parametrize("schedule", ["static", "stealing", "streamk"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_grouped_schedules_exact_with_streamed_b(schedule, dtype):
    from kernels.grouped_gemm import launch_grouped, workspace_from_tensors
    from kernels.matmul import KernelConfig

    gen = torch.Generator(device="cuda").manual_seed(11)
    g, m, k, n = 9, 300, 1000, 520
    a = [_ints((m, k), gen, dtype) for _ in range(g)]
    b = [_ints((k, n), gen, dtype) for _ in range(g)]
    for cfg in (KernelConfig(256, 256, 32, 8, 8, 4), KernelConfig(64, 128, 64, 8, 4, 2),
                KernelConfig(16, 256, 128, 8, 4, 2)):
        c = [torch.full((m, n), float("nan"), device="cuda", dtype=dtype) for _ in range(g)]
        ws = workspace_from_tensors(a, b, c, cfg)
        print(f"b_stream grouped {schedule} {dtype} tile={cfg.tile_key}", flush=True)
        launch_grouped(ws, config=cfg, autotune=False, split_k=1, tile_schedule=schedule, b_stream=1)
        torch.cuda.synchronize()
        assert ws.b_stream == 1
        for e in range(g):
            assert torch.equal(c[e], _exact(a[e], b[e], dtype)), f"{cfg.tile_key} {schedule} problem {e}"


def test_split_k_exact_with_streamed_b():
    from kernels.matmul import KernelConfig, last_matmul_split, launch_matmul

    gen = torch.Generator(device="cuda").manual_seed(13)
    m, k, n = 40, 4096 + 64, 1032
    a, b = _ints((m, k), gen), _ints((k, n), gen)
    for cfg, splits in ((KernelConfig(16, 128, 64, 4, 4, 2), 8), (KernelConfig(256, 256, 32, 8, 8, 4), 4)):
        c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        print(f"b_stream split-K tile={cfg.tile_key} splits={splits}", flush=True)
        launch_matmul(a, b, c, cfg, autotune=False, split_k=splits, b_stream=1)
        torch.cuda.synchronize()
        assert last_matmul_split() == splits
        assert torch.equal(c, _exact(a, b, torch.bfloat16)), f"{cfg.tile_key} split {splits}"


@pytest.mark.parametrize("schedule", ["static", "stealing"])
def test_expert_sorted_exact_with_streamed_b(schedule):
    from kernels.grouped_mm import grouped_mm, last_grouped_mm_b_stream
    from kernels.matmul import KernelConfig

    gen = torch.Generator(device="cuda").manual_seed(17)
    sizes = [37, 0, 300, 1, 129, 64]
    rows, k, n = sum(sizes), 776, 392
    a = _ints((rows, k), gen)
    b = _ints((len(sizes), k, n), gen)
    ends = torch.tensor(sizes, device="cuda").cumsum(0).to(torch.int32)
    for cfg in (KernelConfig(256, 256, 32, 8, 8, 4), KernelConfig(32, 256, 64, 8, 4, 2)):
        out = torch.full((rows, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        print(f"b_stream offsets {schedule} tile={cfg.tile_key}", flush=True)
        grouped_mm(a, b, ends, out=out, config=cfg, autotune=False, tile_schedule=schedule, b_stream=1)
        torch.cuda.synchronize()
        assert last_grouped_mm_b_stream() == 1
        start = 0
        for e, size in enumerate(sizes):
            if size:
                assert torch.equal(out[start:start + size], _exact(a[start:start + size], b[e], torch.bfloat16)), e
            start += size


def test_swiglu_autotuned_and_pinned_policy_match_the_reference():
    from kernels.grouped_gemm import build_fused_gate_up_workspace, launch_gate_up_swiglu

    ws = build_fused_gate_up_workspace([(200, 512, 384)] * 4, torch.bfloat16, seed=3)
    outputs = launch_gate_up_swiglu(ws)
    torch.cuda.synchronize()
    assert ws.swiglu_b_stream in (0, 1)
    tuned = [h.clone() for h in outputs]
    f = ws.b[0].shape[1] // 2
    for a, b, h in zip(ws.a, ws.b, tuned):
        gate, up = a.float() @ b[:, :f].float(), a.float() @ b[:, f:].float()
        reference = torch.nn.functional.silu(gate) * up
        assert (h.float() - reference).abs().max() <= 2e-2 * reference.abs().max()
    # The same config with ordinary B copies gives the same bits, whichever policy the tuner chose.
    cfg = ws.swiglu_config
    other = [h.clone() for h in launch_gate_up_swiglu(ws, cfg, autotune=False)]
    torch.cuda.synchronize()
    assert ws.swiglu_b_stream == 0
    for x, y in zip(tuned, other):
        assert torch.equal(x, y)


def test_autotuned_launchers_time_the_policy_and_record_it():
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped
    from kernels.matmul import last_matmul_b_stream, launch_matmul

    ws = build_grouped_workspace([(8, 2048, 1024)] * 16, torch.bfloat16, seed=5)
    launch_grouped(ws)
    torch.cuda.synchronize()
    assert ws.b_stream in (0, 1)
    for a, b, c in zip(ws.a, ws.b, ws.c):
        assert (c.float() - a.float() @ b.float()).abs().max() <= 1e-2 * (a.float() @ b.float()).abs().max() + 1e-3
    gen = torch.Generator(device="cuda").manual_seed(19)
    a, b = _ints((64, 2048), gen), _ints((2048, 1024), gen)
    c = torch.empty((64, 1024), device="cuda", dtype=torch.bfloat16)
    launch_matmul(a, b, c)
    torch.cuda.synchronize()
    assert last_matmul_b_stream() in (0, 1)
    assert torch.equal(c, _exact(a, b, torch.bfloat16))


def test_launchers_reject_a_bad_policy():
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped
    from kernels.matmul import launch_matmul

    ws = build_grouped_workspace([(8, 64, 64)] * 2, torch.bfloat16, seed=1)
    with pytest.raises(ValueError, match="b_stream"):
        launch_grouped(ws, b_stream=2)
    with pytest.raises(ValueError, match="b_stream"):
        launch_matmul(ws.a[0], ws.b[0], ws.c[0], b_stream=True + 1)
