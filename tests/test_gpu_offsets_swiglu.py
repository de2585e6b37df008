"""GPU parity tests of packed Gate+Up with the fused SwiGLU epilogue over the expert-sorted layout.

H[r0:r1] = silu(A[r0:r1] @ B[e][:, :F]) * (A[r0:r1] @ B[e][:, F:]) per group is checked against
``oracle.swiglu_reference`` applied to each group's rows (``oracle.offsets_groups``; both pinned in
tests/test_oracle.py) with the normwise bound max|H - R| / max|R| (bf16 <= 1e-2, fp16 <= 2e-3):
every tile that can pair gate and up fragments, ragged offsets with an empty group and rows past
offs[-1] (which must stay untouched), and a DeepSeek-V3 EP W13 shard with ragged routing on sampled
rows against a float32 torch product.  Unsupported inputs raise ValueError.
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
