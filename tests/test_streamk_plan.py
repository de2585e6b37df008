"""CPU checks of the stream-K tail bookkeeping and its host-side plan.

The kernel (csrc/gemm_kernel.h, streamk_units) assigns tail slices to runs with closed-form integer
expressions; here those expressions are restated and compared, for many (tail tiles, K slices,
grid) triples, with a brute-force enumeration of the runs' slice ranges.  A mistake in an index
(an off-by-one in a tile's first or last owner, a slot that two pieces share) fails one of them.
"""

from __future__ import annotations

import itertools

import pytest
import torch

from kernels import _native
from kernels.grouped_gemm import build_grouped_workspace, launch_grouped, with_schedule_options
from kernels.matmul import KernelConfig


def kernel_pieces(tail: int, kt: int, grid: int):
    """The kernel's bookkeeping, restated: for every run v, its pieces as (tile j, first slice k0,
    end slice k1, pieces of tile j = ProblemDesc::splits, piece index = ::split, ::slot0).  The
    piece's partial goes to slot slot0 + split."""
    iters = tail * kt
    out = {}
    for v in range(grid):
        it, end = v * iters // grid, (v + 1) * iters // grid
        pieces = []
        while it < end:
            j = it // kt
            k0 = it - j * kt
            k1 = min(kt, k0 + (end - it))
            first = ((j * kt + 1) * grid - 1) // iters
            last = ((j + 1) * kt * grid - 1) // iters
            pieces.append((j, k0, k1, last - first + 1, v - first, first + j))
            it += k1 - k0
        out[v] = pieces
    return out


def brute_force(tail: int, kt: int, grid: int):
    """Owner of every tail slice from the runs' ranges, enumerated one slice at a time."""
    iters = tail * kt
    owner = [None] * iters
    for v in range(grid):
        for i in range(v * iters // grid, (v + 1) * iters // grid):
            assert owner[i] is None
            owner[i] = v
    return owner


CASES = [(t, kt, g) for t, kt, g in itertools.product((1, 2, 3, 5, 64, 80, 128, 192), (1, 3, 7, 64, 224), (8, 24, 256))
         if t * kt >= g]


@pytest.mark.parametrize("tail,kt,grid", CASES)
def test_kernel_piece_bookkeeping_matches_brute_force(tail, kt, grid):
    owner = brute_force(tail, kt, grid)
    pieces = kernel_pieces(tail, kt, grid)
    covered = [0] * (tail * kt)
    by_tile: dict[int, list] = {}
    slots = set()
    for v, plist in pieces.items():
        for j, k0, k1, count, index, slot0 in plist:
            slot = slot0 + index
            assert 0 <= k0 < k1 <= kt
            for i in range(j * kt + k0, j * kt + k1):
                covered[i] += 1
                assert owner[i] == v
            # The tile's owners are exactly the runs that hold one of its slices.
            runs = sorted({owner[i] for i in range(j * kt, (j + 1) * kt)})
            assert runs == list(range(runs[0], runs[-1] + 1))
            assert count == len(runs) and index == v - runs[0]
            assert slot not in slots
            slots.add(slot)
            by_tile.setdefault(j, []).append((index, slot, k0))
    assert covered == [1] * (tail * kt)
    assert max(slots) < grid + tail  # the workspace's grid + tail slots
    for j, plist in by_tile.items():
        plist.sort()
        # Pieces of a tile: indices 0..n-1 in K order, in consecutive slots.
        assert [p[0] for p in plist] == list(range(len(plist)))
        assert [p[1] for p in plist] == list(range(plist[0][1], plist[0][1] + len(plist)))
        assert [p[2] for p in plist] == sorted(p[2] for p in plist)


def test_piece_bound_of_the_host_check():
    # The library rejects plans that would cut a tile into more than 64 pieces, using the bound
    # ceil(KT / floor(I / W)) + 1; check the bound holds (it is what sizes the arrival field).
    for tail, kt, grid in CASES:
        per_run = tail * kt // grid
        bound = -(-kt // per_run) + 1
        worst = max(count for plist in kernel_pieces(tail, kt, grid).values() for _, _, _, count, _, _ in plist)
        assert worst <= bound


def test_streamk_tail_is_the_partial_last_round():
    assert _native.streamk_tail(448, 256, 4096, 32) == 192
    assert _native.streamk_tail(1104, 256, 2880, 32) == 80
    assert _native.streamk_tail(1024, 256, 7168, 32) == 0      # exact rounds: nothing to spread
    assert _native.streamk_tail(192, 256, 2048, 32) == 192     # one partial round
    assert _native.streamk_tail(1, 256, 4096, 64) == 0         # 64 slices over 256 runs: too thin
    assert _native.streamk_tail(0, 256, 4096, 64) == 0


def test_schedule_options_add_streamk_where_it_applies():
    a, b = KernelConfig(256, 256, 32, 8, 8, 4, 1), KernelConfig(64, 128, 64, 8, 4, 4, 1)
    options = [(a, 1), (a, 4), (b, 1)]
    applies = lambda cfg: cfg is a  # noqa: E731
    assert with_schedule_options(options, None, applies) == [
        (a, 1, "static"), (a, 1, "stealing"), (a, 1, "streamk"), (a, 4, "static"),
        (b, 1, "static"), (b, 1, "stealing")]
    assert with_schedule_options(options, "streamk", applies) == [(a, 1, "streamk")]
    assert with_schedule_options(options, "static", applies) == [(a, 1, "static"), (a, 4, "static"),
                                                                (b, 1, "static")]


def test_streamk_schedule_is_validated_before_touching_a_gpu():
    workspace = build_grouped_workspace([(8, 16, 32)] * 2, torch.bfloat16, device="cpu")
    with pytest.raises(ValueError, match="unsplit"):
        launch_grouped(workspace, tile_schedule="streamk", split_k=2)
