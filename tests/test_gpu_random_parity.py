"""Randomised exact-integer parity sweep over the launch modes, tiles, grids, schedules and splits.

Each case draws a dtype (bf16, fp16, or fp32 with IEEE or TF32 products), a compiled config with a
x1 or x2 grid, a launch mode (homogeneous grouped, heterogeneous grouped, expert-sorted offsets with
empty groups, or a single GEMM), a tile schedule (static, work stealing, or for homogeneous 16-bit
groups the stream-K tail) and, where the mode allows it, a K split (16-bit operands), then shapes: K and N sometimes off the 8-element vector layout, M from 1 row up.
Operands are small random integers in [-2, 2], so every fp32 sum is exact and the expected output
is the float64 product rounded once to the operand dtype (TF32 rounds such integers exactly): the
launch must match it bit for bit (NaN-filled outputs also catch unwritten tiles).  The seeds are
fixed; a failure names the seed and the drawn case.
"""

from __future__ import annotations

import itertools
import json
import random

import pytest
import torch

pytestmark = pytest.mark.gpu

SEEDS = (101, 202, 303, 404)
CASES_PER_SEED = 150


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


def _draw_and_run(rng: random.Random, gen: torch.Generator) -> tuple[dict, list]:
    from kernels.grouped_gemm import launch_grouped, workspace_from_tensors
    from kernels.grouped_mm import grouped_mm
    from kernels.matmul import KernelConfig, config_pool, launch_matmul

    def ints(shape, dtype):
        return torch.randint(-2, 3, shape, device="cuda", generator=gen).to(dtype)

    def expect(a, b, dtype):
        return (a.double() @ b.double()).to(dtype)

    def dim(lo, hi, mult):
        v = rng.randint(lo, hi)
        return max(mult, v // mult * mult)

    def nan(shape, dtype):
        return torch.full(shape, float("nan"), device="cuda", dtype=dtype)

    dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    wide = dtype == torch.float32
    precision = rng.choice(["ieee", "tf32"]) if wide else "ieee"
    base = rng.choice(config_pool(dtype))
    cfg = KernelConfig(base.block_m, base.block_n, base.block_k, base.group_size_m, base.num_warps, base.num_stages,
                       rng.choice([1, 1, 2]))
    mode = rng.choice(["homogeneous", "homogeneous", "generic", "offsets", "offsets", "single"])
    # Homogeneous 16-bit groups may also draw the stream-K tail (the launcher runs the static
    # schedule where the tile count leaves no partial last round or the layout does not qualify).
    streamk_ok = mode == "homogeneous" and not wide and cfg.cta_multiplier == 1
    schedule = rng.choice(["static", "stealing", "streamk"] if streamk_ok else ["static", "stealing"])
    k = dim(16, 2500, rng.choice([1, 8]))
    n = dim(8, 800, rng.choice([1, 8, 8]))
    case = {"mode": mode, "dtype": str(dtype).split(".")[-1], "precision": precision, "config": cfg.as_dict(),
            "schedule": schedule}
    if mode == "homogeneous":
        g, m = rng.randint(1, 24), rng.randint(1, 600)
        split = rng.choice([1, 1, None, 2, 3]) if schedule == "static" and not wide else 1
        case.update(groups=g, m=m, k=k, n=n, split_k=split)
        a = [ints((m, k), dtype) for _ in range(g)]
        b = [ints((k, n), dtype) for _ in range(g)]
        c = [nan((m, n), dtype) for _ in range(g)]
        launch_grouped(workspace_from_tensors(a, b, c, cfg), precision, config=cfg, autotune=False, split_k=split,
                       tile_schedule=schedule)
        torch.cuda.synchronize()
        return case, [e for e in range(g) if not torch.equal(c[e], expect(a[e], b[e], dtype))]
    if mode == "generic":
        shapes = [(rng.randint(1, 400), dim(16, 1500, 8), dim(8, 600, 8)) for _ in range(rng.randint(2, 20))]
        case.update(shapes=shapes)
        a = [ints((m, kk), dtype) for m, kk, _ in shapes]
        b = [ints((kk, nn), dtype) for _, kk, nn in shapes]
        c = [nan((m, nn), dtype) for m, _, nn in shapes]
        launch_grouped(workspace_from_tensors(a, b, c, cfg), precision, config=cfg, autotune=False, split_k=1,
                       tile_schedule=schedule)
        torch.cuda.synchronize()
        return case, [e for e in range(len(shapes)) if not torch.equal(c[e], expect(a[e], b[e], dtype))]
    if mode == "offsets":
        g = rng.randint(1, 40)
        sizes = [rng.choice([0, rng.randint(1, 40), rng.randint(1, 600)]) for _ in range(g)]
        sizes[0] = sizes[0] or 5
        rows = sum(sizes)
        case.update(groups=g, sizes=sizes, k=k, n=n)
        a, b = ints((rows, k), dtype), ints((g, k, n), dtype)
        offs = torch.tensor(list(itertools.accumulate(sizes)), device="cuda", dtype=torch.int32)
        out = nan((rows, n), dtype)
        grouped_mm(a, b, offs, out=out, config=cfg, input_precision=precision, autotune=False, tile_schedule=schedule)
        torch.cuda.synchronize()
        bad, start = [], 0
        for e, s in enumerate(sizes):
            if s and not torch.equal(out[start:start + s], expect(a[start:start + s], b[e], dtype)):
                bad.append(e)
            start += s
        return case, bad
    m = rng.randint(1, 1500)
    split = rng.choice([1, None, 2, 4, 8]) if not wide else 1
    case.update(m=m, k=k, n=n, split_k=split)
    a, b = ints((m, k), dtype), ints((k, n), dtype)
    c = nan((m, n), dtype)
    launch_matmul(a, b, c, cfg, precision, autotune=False, split_k=split)
    torch.cuda.synchronize()
    return case, [] if torch.equal(c, expect(a, b, dtype)) else [0]


@pytest.mark.parametrize("seed", SEEDS)
def test_random_cases_match_exact_integer_products(seed):
    rng = random.Random(seed)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    failures = []
    for index in range(CASES_PER_SEED):
        case, bad = _draw_and_run(rng, gen)
        if bad:
            failures.append(json.dumps({"seed": seed, "case": index, **case, "wrong_problems": bad[:8]}))
    assert not failures, "\n".join(failures[:5])
