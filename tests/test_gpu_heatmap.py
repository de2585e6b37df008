"""GPU parity over the heatmap family of single grouped GEMMs (bf16, seeded N(0,1)/sqrt(K) inputs).

The grid extends the reference's single-GEMM heatmap (benchmark_shapes.py:321-335, G = 1) to
G in {1, 8, 64, 256} groups of equal problems, with extents that are not tile multiples
(2880 = 22.5 x 128, from gpt-oss-120b): all 500 points, M_e in {8, 32, 128, 512, 2048} x N, K in
{256, 1024, 2880, 4096, 7168} at every G, from 256 x [8,256]@[256,256] up to
256 x [2048,7168]@[7168,7168].  Every point is launched through ``launch_grouped`` with the
heuristic config (G = 1 dispatches to the single GEMM, whose heuristic may split K), and checked
three ways, in the pattern of the reference's tests/test_gpu.py:127-154:
  * seeded random inputs drawn N(0,1)/sqrt(K), as the configuration states: the first and last
    problem against a float32 torch product on the GPU (normwise max|C - R| / max|R| <= 1e-2),
    and tail rows of both against the CPU oracle;
  * exact integers on every problem: A = 1, B_e = e % 31 + 1, so C_e = K (e % 31 + 1) exactly in
    the fp32 accumulator, rounded to bf16 the same way as the expected value - a wrong problem
    index, a skipped or duplicated tile, or a missed tail shows on whichever problem it hits;
  * C is NaN-filled before each launch, so an unwritten element fails both checks.
"""

from __future__ import annotations

import pytest
import torch

from helpers import normwise, oracle_product

pytestmark = pytest.mark.gpu

EXTENTS = (256, 1024, 2880, 4096, 7168)
SMALL_GROUPS = [(g, m, n, k) for g in (1, 8) for m in (8, 32, 128, 512, 2048) for n in EXTENTS for k in EXTENTS]
LARGE_GROUPS = [(g, m, n, k) for g in (64, 256) for m in (8, 32, 128, 512, 2048) for n in EXTENTS for k in EXTENTS]


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


def _check_point(g: int, m: int, n: int, k: int) -> None:
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped

    print(f"heatmap G={g} M={m} N={n} K={k}", flush=True)
    workspace = build_grouped_workspace([(m, k, n)] * g, torch.bfloat16, seed=m * 7 + n * 3 + k + g)
    generator = torch.Generator(device="cuda").manual_seed(m * 7 + n * 3 + k + g)
    for a, b, c in workspace.problem_tensors():
        a.normal_(generator=generator).div_(k ** 0.5)
        b.normal_(generator=generator).div_(k ** 0.5)
        c.fill_(float("nan"))
    launch_grouped(workspace, autotune=False)
    torch.cuda.synchronize()
    label = f"G={g} M={m} N={n} K={k} config={workspace.config} split={workspace.split_k}"
    for index in sorted({0, g - 1}):
        a, b, c = workspace.a[index], workspace.b[index], workspace.c[index]
        assert torch.isfinite(c).all(), f"problem {index} left unwritten: {label}"
        assert normwise(c, a.float() @ b.float()) <= 1e-2, f"problem {index}: {label}"
        rows = slice(max(0, m - 3), m)
        assert normwise(c[rows], oracle_product(a[rows], b)) <= 1e-2, f"oracle rows, problem {index}: {label}"
    for index, (a, b, c) in enumerate(workspace.problem_tensors()):
        a.fill_(1)
        b.fill_(index % 31 + 1)
        c.fill_(float("nan"))
    launch_grouped(workspace, autotune=False)
    torch.cuda.synchronize()
    for index, c in enumerate(workspace.c):
        expected = torch.full_like(c, float(k * (index % 31 + 1)))
        assert torch.equal(c, expected), f"exact integers, problem {index}: {label}"
    del workspace
    if g * m * k >= (1 << 28):
        torch.cuda.empty_cache()


@pytest.mark.parametrize("point", SMALL_GROUPS, ids=lambda p: "g{}_m{}_n{}_k{}".format(*p))
def test_heatmap_small_groups(point):
    _check_point(*point)


@pytest.mark.parametrize("point", LARGE_GROUPS, ids=lambda p: "g{}_m{}_n{}_k{}".format(*p))
def test_heatmap_large_groups(point):
    _check_point(*point)
