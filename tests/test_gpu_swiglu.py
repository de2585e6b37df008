"""GPU parity tests of the fused SwiGLU epilogue (packed Gate+Up) through the C ABI.

H_e = silu(A_e @ B_e[:, :F]) * (A_e @ B_e[:, F:]) is checked against ``oracle.swiglu_reference``
(exact sums, float64 activation, one rounding; pinned in tests/test_oracle.py) with the normwise
bound max|H - R| / max|R| (bf16 <= 1e-2, fp16 <= 2e-3), on every tile that can run the epilogue,
on ragged M tails, on a heterogeneous (generic-mode) group, and on the DeepSeek-V3 EP W13 shard at
full size (sampled rows against a float32 torch product).  Unsupported inputs raise ValueError.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import DTYPE_NAME, from_oracle, normwise, to_oracle
from oracle import oracle

pytestmark = pytest.mark.gpu

NORMWISE = {"bf16": 1e-2, "fp16": 2e-3}


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")
    torch.manual_seed(17)


def _reference(a, b):
    name = DTYPE_NAME[a.dtype]
    return from_oracle(oracle.swiglu_reference(np.ascontiguousarray(to_oracle(a)),
                                               np.ascontiguousarray(to_oracle(b)), name), name)


def _workspace(shapes, dtype):
    from kernels.grouped_gemm import workspace_from_tensors

    a = [torch.randn((m, k), device="cuda", dtype=dtype) / math.sqrt(k) for m, k, _ in shapes]
    b = [torch.randn((k, n), device="cuda", dtype=dtype) for _, k, n in shapes]
    c = [torch.empty((m, n), device="cuda", dtype=dtype) for m, _, n in shapes]
    return workspace_from_tensors(a, b, c)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16), ids=lambda d: DTYPE_NAME[d])
def test_every_swiglu_tile_ragged_m(dtype):
    from kernels import _native
    from kernels.grouped_gemm import launch_gate_up_swiglu
    from kernels.matmul import KernelConfig

    ws = _workspace([(37, 96, 512)] * 3, dtype)
    expected = [_reference(a, b) for a, b in zip(ws.a, ws.b)]
    tiles = sorted(_native.swiglu_tiles(_native.dtype_code(dtype)))
    assert len(tiles) >= 10
    for bm, bn, bk, warps, stages in tiles:
        cfg = KernelConfig(bm, bn, bk, 8, warps, stages, 1)
        print(f"swiglu tile={cfg.tile_key} dtype={DTYPE_NAME[dtype]}", flush=True)
        if ws.h is not None:
            for h in ws.h:
                h.fill_(float("nan"))
        outputs = launch_gate_up_swiglu(ws, cfg, autotune=False)
        torch.cuda.synchronize()
        for h, r in zip(outputs, expected):
            assert torch.isfinite(h).all(), f"tile {cfg.tile_key} left unwritten outputs"
            assert normwise(h.cpu(), r) <= NORMWISE[DTYPE_NAME[dtype]], f"tile {cfg.tile_key}"


def test_heterogeneous_group_runs_generic_mode():
    from kernels.grouped_gemm import launch_gate_up_swiglu

    ws = _workspace([(5, 64, 256), (70, 128, 256), (129, 64, 512)], torch.bfloat16)
    assert not ws.homogeneous
    print("swiglu generic group", flush=True)
    outputs = launch_gate_up_swiglu(ws)
    torch.cuda.synchronize()
    assert ws.swiglu_config is not None
    for a, b, h in zip(ws.a, ws.b, outputs):
        assert h.shape == (a.shape[0], b.shape[1] // 2)
        assert normwise(h.cpu(), _reference(a, b)) <= NORMWISE["bf16"]


def test_dsv3_ep_w13_shard_matches_float32_torch():
    from kernels.grouped_gemm import build_fused_gate_up_workspace, launch_gate_up_swiglu
    from utils.metrics import moe_shapes

    shapes = moe_shapes("W1", "EP", 512, 7168, 2048, 256, 8)
    print("swiglu DSV3 EP W13 M_e=512", flush=True)
    ws = build_fused_gate_up_workspace(shapes, torch.bfloat16, seed=1234)
    outputs = launch_gate_up_swiglu(ws)
    torch.cuda.synchronize()
    f = shapes[0][2] // 2
    for index in (0, 17, 31):
        rows = torch.tensor([0, 255, 256, 511], device="cuda")
        a, b = ws.a[index][rows].float(), ws.b[index].float()
        expected = torch.nn.functional.silu(a @ b[:, :f]) * (a @ b[:, f:])
        assert normwise(outputs[index][rows].float().cpu(), expected.cpu()) <= 1e-2


def test_unsupported_inputs_raise_value_error():
    from kernels import _native
    from kernels.grouped_gemm import launch_gate_up_swiglu
    from kernels.matmul import KernelConfig

    with pytest.raises(ValueError):
        launch_gate_up_swiglu(_workspace([(16, 64, 128)] * 2, torch.float32))
    with pytest.raises(ValueError):
        launch_gate_up_swiglu(_workspace([(16, 64, 72)] * 2, torch.bfloat16))  # F = 36 not a multiple of 8
    odd = [row[:5] for row in _native.compiled_kernels(_native.DTYPE_BF16)
           if tuple(row[:5]) not in _native.swiglu_tiles(_native.DTYPE_BF16)]
    assert odd, "expected some tiles without the epilogue (odd fragments per wave)"
    bm, bn, bk, warps, stages = odd[0]
    with pytest.raises(ValueError):
        launch_gate_up_swiglu(_workspace([(16, 64, 256)] * 2, torch.bfloat16),
                              KernelConfig(bm, bn, bk, 8, warps, stages, 1), autotune=False)
