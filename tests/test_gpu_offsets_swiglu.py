"""GPU parity tests of packed Gate+Up with the fused SwiGLU epilogue over the expert-sorted layout.

H[r0:r1] = silu(A[r0:r1] @ B[e][:, :F]) * (A[r0:r1] @ B[e][:, F:]) per group is checked against
``oracle.swiglu_reference`` applied to each group's rows (``oracle.offsets_groups``; both pinned in
tests/test_oracle.py) with the normwise bound max|H - R| / max|R| (bf16 <= 1e-2, fp16 <= 2e-3):
every tile that can pair gate and up fragments, ragged offsets with an empty group and rows past
offs[-1] (which must stay untouched), and a DeepSeek-V3 EP W13 shard with ragged routing on sampled
rows against a float32 torch product; and a whole expert FFN on sorted tokens in two launches
(grouped_mm_swiglu, then grouped_mm for W2 on the same offsets, with an expert that received no
tokens).  Unsupported inputs raise ValueError.
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
    torch.manual_seed(29)


def _operands(rows, k, n, groups, dtype):
    mat_a = torch.randn((rows, k), device="cuda", dtype=dtype) / math.sqrt(k)
    mat_b = torch.randn((groups, k, n), device="cuda", dtype=dtype)
    return mat_a, mat_b


def _reference(mat_a, mat_b, offs_list):
    name = DTYPE_NAME[mat_a.dtype]
    a = to_oracle(mat_a)
    rows, f = mat_a.shape[0], mat_b.shape[2] // 2
    out = np.zeros((rows, f), dtype=a.dtype)
    for e, (r0, m) in enumerate(oracle.offsets_groups(offs_list, rows)):
        if m:
            out[r0:r0 + m] = oracle.swiglu_reference(np.ascontiguousarray(a[r0:r0 + m]),
                                                      np.ascontiguousarray(to_oracle(mat_b[e])), name)
    return from_oracle(out, name)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16), ids=lambda d: DTYPE_NAME[d])
def test_every_swiglu_tile_ragged_offsets(dtype):
    from kernels import _native
    from kernels.grouped_mm import grouped_mm_swiglu
    from kernels.matmul import KernelConfig

    rows, k, n = 211, 96, 512
    offs_list = [40, 40, 41, 150, 190]  # empty group, one-row group, rows 190..210 past the end
    mat_a, mat_b = _operands(rows, k, n, len(offs_list), dtype)
    offs = torch.tensor(offs_list, device="cuda", dtype=torch.int32)
    covered = offs_list[-1]
    expected = _reference(mat_a, mat_b, offs_list)
    tiles = sorted(_native.swiglu_tiles(_native.dtype_code(dtype)))
    assert len(tiles) >= 10
    for bm, bn, bk, warps, stages in tiles:
        cfg = KernelConfig(bm, bn, bk, 8, warps, stages, 1)
        print(f"offsets swiglu tile={cfg.tile_key} dtype={DTYPE_NAME[dtype]} offs={offs_list}", flush=True)
        out = torch.full((rows, n // 2), float("nan"), device="cuda", dtype=dtype)
        grouped_mm_swiglu(mat_a, mat_b, offs, out=out, config=cfg)
        torch.cuda.synchronize()
        assert torch.isfinite(out[:covered]).all(), f"tile {cfg.tile_key} left rows unwritten"
        assert normwise(out[:covered].cpu(), expected[:covered]) <= NORMWISE[DTYPE_NAME[dtype]], f"tile {cfg.tile_key}"
        assert torch.isnan(out[covered:]).all(), f"tile {cfg.tile_key} wrote rows past offs[-1]"


def test_autotuned_dsv3_ep_w13_ragged_routing():
    from kernels.grouped_mm import grouped_mm_swiglu, last_grouped_mm_swiglu_config

    rng = np.random.default_rng(13)
    sizes = [int(v) for v in rng.integers(300, 700, size=32)]
    ends = np.cumsum(sizes).tolist()
    rows, k, n = ends[-1], 7168, 4096
    print(f"offsets swiglu DSV3 EP W13 rows={rows}", flush=True)
    mat_a = torch.randn((rows, k), device="cuda", dtype=torch.bfloat16) * 0.1
    mat_b = torch.randn((32, k, n), device="cuda", dtype=torch.bfloat16) * 0.1
    offs = torch.tensor(ends, device="cuda", dtype=torch.int32)
    h = grouped_mm_swiglu(mat_a, mat_b, offs)
    torch.cuda.synchronize()
    assert last_grouped_mm_swiglu_config() is not None
    f = n // 2
    for e in (0, 17, 31):
        r0 = 0 if e == 0 else ends[e - 1]
        rows_e = torch.tensor([r0, r0 + sizes[e] // 2, ends[e] - 1], device="cuda")
        a = mat_a[rows_e].float()
        b = mat_b[e].float()
        ref = torch.nn.functional.silu(a @ b[:, :f]) * (a @ b[:, f:])
        assert normwise(h[rows_e].float().cpu(), ref.cpu()) <= 1e-2, f"group {e}"


def test_unsupported_inputs_raise_value_error():
    from kernels import _native
    from kernels.grouped_mm import grouped_mm_swiglu
    from kernels.matmul import KernelConfig

    offs = torch.tensor([8, 16], device="cuda", dtype=torch.int32)
    with pytest.raises(ValueError):
        grouped_mm_swiglu(*_operands(16, 64, 128, 2, torch.float32), offs)
    with pytest.raises(ValueError):
        grouped_mm_swiglu(*_operands(16, 64, 72, 2, torch.bfloat16), offs)  # F = 36 is not a multiple of 8
    with pytest.raises(ValueError):
        grouped_mm_swiglu(*_operands(16, 64, 128, 2, torch.bfloat16), offs,
                          out=torch.empty((16, 128), device="cuda", dtype=torch.bfloat16))
    odd = [row[:5] for row in _native.compiled_kernels(_native.DTYPE_BF16)
           if tuple(row[:5]) not in _native.swiglu_tiles(_native.DTYPE_BF16)]
    bm, bn, bk, warps, stages = odd[0]
    with pytest.raises(ValueError):
        grouped_mm_swiglu(*_operands(16, 64, 256, 2, torch.bfloat16), offs,
                          config=KernelConfig(bm, bn, bk, 8, warps, stages, 1))


def test_expert_ffn_on_sorted_tokens_in_two_launches():
    """Y = W2(silu(X W1) * (X W3)) per expert: grouped_mm_swiglu then grouped_mm on the same offs,
    against float32 torch on sampled rows (H rounded to bf16 between the launches, as stored)."""
    from kernels.grouped_mm import grouped_mm, grouped_mm_swiglu

    rng = np.random.default_rng(3)
    experts, hidden, ffn = 16, 1024, 512
    sizes = [int(v) for v in rng.integers(0, 200, size=experts)]
    sizes[3] = 0  # an expert no token was routed to
    ends = np.cumsum(sizes).tolist()
    rows = ends[-1]
    print(f"expert FFN rows={rows} experts={experts} H={hidden} F={ffn}", flush=True)
    x = torch.randn((rows, hidden), device="cuda", dtype=torch.bfloat16)
    w13 = torch.randn((experts, hidden, 2 * ffn), device="cuda", dtype=torch.bfloat16) / math.sqrt(hidden)
    w2 = torch.randn((experts, ffn, hidden), device="cuda", dtype=torch.bfloat16) / math.sqrt(ffn)
    offs = torch.tensor(ends, device="cuda", dtype=torch.int32)
    h = grouped_mm_swiglu(x, w13, offs)
    y = grouped_mm(h, w2, offs)
    torch.cuda.synchronize()
    for e in range(experts):
        if sizes[e] == 0:
            continue
        r0 = ends[e] - sizes[e]
        sample = torch.tensor(sorted({r0, r0 + sizes[e] // 2, ends[e] - 1}), device="cuda")
        xs = x[sample].float()
        gate, up = xs @ w13[e, :, :ffn].float(), xs @ w13[e, :, ffn:].float()
        h_ref = (torch.nn.functional.silu(gate) * up).to(torch.bfloat16).float()
        y_ref = h_ref @ w2[e].float()
        assert normwise(h[sample].float().cpu(), h_ref.cpu()) <= 1e-2, f"expert {e}: H"
        assert normwise(y[sample].float().cpu(), y_ref.cpu()) <= 1e-2, f"expert {e}: Y"
