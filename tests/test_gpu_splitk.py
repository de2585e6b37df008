"""GPU parity tests of split-K inside one launch (low-tile-count shapes) through the C ABI.

Known answers whose K chunks differ (A = 1, B[k, n] = ((k // 64) % 5 - 2) + n % 2), so a unit that
summed the wrong K range, a lost partial or a double-counted split changes the exact integer
result; seeded random inputs against the oracle (normwise bf16 <= 1e-2); M, N and K tails; forced
and heuristic split counts; grouped homogeneous split-K; and a captured graph replayed several
times with eager work in between (the per-tile counters must re-arm themselves); and launches of
different tile counts sharing one stream's workspace in an order where a counter layout sized per
launch put one launch's partials on the next launch's counters.
"""

from __future__ import annotations

import math

import pytest
import torch

from helpers import normwise, oracle_product

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")
    torch.manual_seed(23)


def _known(m, k, n, dtype):
    """A = 1, B[k, n] = ((k // 64) % 5 - 2) + n % 2: every K chunk (whole 64-element slices) has its
    own sum, all sums are multiples of 64, and the exact results stay representable in bf16, so a
    missing, doubled or shifted K range changes the stored value."""
    a = torch.ones((m, k), device="cuda", dtype=dtype)
    kk = torch.arange(k, device="cuda").div(64, rounding_mode="floor").remainder(5).sub(2).view(k, 1)
    nn = torch.arange(n, device="cuda").remainder(2).view(1, n)
    b = (kk + nn).to(dtype)
    exact = (kk.double().sum() + k * nn.double()).expand(m, n).cpu()
    assert torch.equal(exact.to(dtype).double(), exact), "known answer must be exact in the dtype"
    return a, b, exact


@pytest.mark.parametrize("splits", [2, 7, 16])
def test_mixtral_ep_w2_known_answer_forced_splits(splits):
    from kernels.matmul import KernelConfig, last_matmul_split, launch_matmul

    m, k, n = 16, 14336, 4096  # Mixtral-8x7B EP rank, W2 at M_e = 16: 16 tiles of 16 x 256
    a, b, exact = _known(m, k, n, torch.bfloat16)
    for cfg in (KernelConfig(16, 256, 128, 8, 4, 2, 1), KernelConfig(16, 256, 64, 8, 4, 4, 1),
                KernelConfig(32, 128, 64, 8, 4, 4, 1)):
        print(f"splitk known answer splits={splits} tile={cfg.tile_key}", flush=True)
        c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        launch_matmul(a, b, c, cfg, autotune=False, split_k=splits)
        torch.cuda.synchronize()
        assert last_matmul_split() == splits
        assert torch.equal(c.double().cpu(), exact), f"tile {cfg.tile_key} splits {splits}"


def test_heuristic_split_random_inputs_with_tails():
    from kernels.matmul import KernelConfig, last_matmul_split, launch_matmul

    m, k, n = 37, 14400, 4104  # M tail, N tail (8 valid columns in the last tile), K not a split multiple
    a = torch.randn((m, k), device="cuda", dtype=torch.bfloat16) / math.sqrt(k)
    b = torch.randn((k, n), device="cuda", dtype=torch.bfloat16)
    c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    print("splitk heuristic random m=37 k=14400 n=4104", flush=True)
    launch_matmul(a, b, c, KernelConfig(64, 256, 64, 8, 4, 3, 1), autotune=False)
    torch.cuda.synchronize()
    assert last_matmul_split() > 1
    assert torch.isfinite(c).all()
    rows = [0, 18, 36]
    expected = oracle_product(a[rows], b)
    assert normwise(c[rows].cpu(), expected) <= 1e-2


def test_autotuned_mixtral_ep_w2_matches_oracle_split_or_not():
    from kernels.matmul import last_matmul_split, launch_matmul

    m, k, n = 16, 14336, 4096
    a = torch.randn((m, k), device="cuda", dtype=torch.bfloat16) / math.sqrt(k)
    b = torch.randn((k, n), device="cuda", dtype=torch.bfloat16)
    c = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
    c1 = torch.empty_like(c)
    print("splitk autotuned Mixtral EP W2", flush=True)
    launch_matmul(a, b, c)  # the tuner measures each tile unsplit and split and keeps the faster
    split = last_matmul_split()
    launch_matmul(a, b, c1, split_k=1)
    torch.cuda.synchronize()
    assert split >= 1
    expected = oracle_product(a, b)
    assert normwise(c.cpu(), expected) <= 1e-2
    assert normwise(c1.cpu(), expected) <= 1e-2


def test_grouped_homogeneous_split_k_known_answer():
    from kernels.grouped_gemm import launch_grouped, workspace_from_tensors
    from kernels.matmul import KernelConfig

    g, m, k, n = 4, 16, 7168, 512
    a, b, c = [], [], []
    exacts = []
    for e in range(g):
        ae, be, ex = _known(m, k, n, torch.bfloat16)
        a.append(ae)
        b.append(be)
        exacts.append(ex)
        c.append(torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16))
    ws = workspace_from_tensors(a, b, c)
    for splits in (None, 3):
        print(f"splitk grouped splits={splits}", flush=True)
        for ce in ws.c:
            ce.fill_(float("nan"))
        launch_grouped(ws, config=KernelConfig(16, 256, 128, 8, 4, 2, 1), autotune=False, split_k=splits)
        torch.cuda.synchronize()
        assert ws.split_k > 1
        for ce, ex in zip(ws.c, exacts):
            assert torch.equal(ce.double().cpu(), ex)


def test_graph_replays_rearm_the_counters():
    from kernels.matmul import KernelConfig, launch_matmul

    m, k, n = 16, 8192, 2048
    a, b, exact = _known(m, k, n, torch.bfloat16)
    c = torch.zeros((m, n), device="cuda", dtype=torch.bfloat16)
    cfg = KernelConfig(16, 256, 128, 8, 4, 2, 1)
    launch_matmul(a, b, c, cfg, autotune=False, split_k=8)  # allocates the workspace outside capture
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        launch_matmul(a, b, c, cfg, autotune=False, split_k=8)  # this stream's workspace, before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            launch_matmul(a, b, c, cfg, autotune=False, split_k=8)
    torch.cuda.synchronize()
    for replay in range(4):
        print(f"splitk graph replay {replay}", flush=True)
        c.zero_()
        launch_matmul(a, b, torch.empty_like(c), cfg, autotune=False, split_k=8)  # eager work in between
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c.double().cpu(), exact)


def test_launches_of_different_tile_counts_share_one_workspace():
    from kernels.matmul import KernelConfig, launch_matmul

    m, k, n = 128, 14336, 4096  # Mixtral-8x7B EP rank, W2 at M_e = 128
    a, b, exact = _known(m, k, n, torch.bfloat16)
    # 16 tiles, then 128, 128 and 512 tiles: each launch has more tile counters than the one before.
    sequence = ((KernelConfig(128, 256, 64, 8, 8, 3, 1), 16), (KernelConfig(16, 256, 128, 8, 4, 2, 1), 2),
                (KernelConfig(64, 64, 64, 8, 4, 4, 1), 4), (KernelConfig(16, 64, 128, 8, 4, 7, 1), 3),
                (KernelConfig(128, 256, 64, 8, 8, 3, 1), 16), (KernelConfig(16, 64, 128, 8, 4, 7, 1), 8))
    for cfg, splits in sequence:
        print(f"splitk shared workspace tile={cfg.tile_key} splits={splits}", flush=True)
        c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        launch_matmul(a, b, c, cfg, autotune=False, split_k=splits)
        torch.cuda.synchronize()
        assert torch.equal(c.double().cpu(), exact), f"tile {cfg.tile_key} splits {splits}"


@pytest.mark.parametrize("splits", [3, 9, 16])
def test_every_tile_split_known_answer_with_tails(splits):
    """Every compiled 16-bit tile, forced splits (not multiples of how many partials the last unit
    stages at once), M and N tails: the reduction's grouping, its own-partial shortcut and the
    register fallback of the largest tiles all give the exact result."""
    from kernels import _native
    from kernels.matmul import KernelConfig, last_matmul_split, launch_matmul

    for bm, bn, bk, warps, stages, _lds, _wm in _native.compiled_kernels(_native.DTYPE_BF16):
        m, n, k = 2 * bm - 5, 2 * bn + 8, 1280
        a, b, exact = _known(m, k, n, torch.bfloat16)
        cfg = KernelConfig(bm, bn, bk, 8, warps, stages, 1)
        print(f"splitk every tile {cfg.tile_key} splits={splits}", flush=True)
        c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        launch_matmul(a, b, c, cfg, autotune=False, split_k=splits)
        torch.cuda.synchronize()
        assert last_matmul_split() == splits
        assert torch.equal(c.double().cpu(), exact), f"tile {cfg.tile_key} splits {splits}"


@pytest.mark.parametrize("polls", [None, "1", "0"], ids=["polls_default", "polls_1", "polls_0"])
@pytest.mark.parametrize("tile", [(256, 256, 32, 8, 4), (128, 256, 64, 8, 3), (64, 128, 64, 4, 4),
                                  (16, 64, 128, 4, 4)], ids=lambda t: "x".join(map(str, t)))
def test_split_reduction_same_bits_whoever_reduces(tile, polls, monkeypatch):
    """The units of a tile share its reduction when every unit has a workgroup of its own (grid >=
    units) and the partials are large; on smaller grids a workgroup runs several units and the last
    unit of each tile reduces it alone.  A unit waits for its partners only a bounded number of
    polls (MOEGEMM_SPLIT_POLLS; 1 makes units stop waiting often, so the last unit to arrive takes
    over their slices; 0 never waits).  Every element sums the partials in split order whoever
    reduces it, so all grids and poll limits give the same bits, close to the oracle, and every
    launch leaves the workspace counters at zero."""
    from kernels import _native

    if polls is None:
        monkeypatch.delenv("MOEGEMM_SPLIT_POLLS", raising=False)
    else:
        monkeypatch.setenv("MOEGEMM_SPLIT_POLLS", polls)

    bm, bn, bk, warps, stages = tile
    m, k, n = 2 * bm + 44, 4096, 2 * bn + 8
    a = (torch.randn((m, k), device="cuda") / math.sqrt(k)).to(torch.bfloat16)
    b = torch.randn((k, n), device="cuda").to(torch.bfloat16)
    tiles = -(-m // bm) * -(-n // bn)
    lib = _native.library()
    stream = _native.current_stream_handle(a.device)
    for splits in (3, 4):
        nbytes = _native.splitk_workspace_bytes(tiles, splits, bm, bn)
        workspace = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        outputs = []
        for grid in (0, 1, 5, tiles * splits - 1):
            print(f"splitk whoever reduces tile={tile} polls={polls} splits={splits} grid={grid}", flush=True)
            c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
            _native.check(lib.moegemm_matmul_splitk(
                a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, a.stride(0), a.stride(1), b.stride(0),
                b.stride(1), c.stride(0), c.stride(1), _native.DTYPE_BF16, bm, bn, bk, 8, warps, stages, splits,
                grid, workspace.data_ptr(), workspace.numel(), 0, stream))
            torch.cuda.synchronize()
            assert not workspace[:256 * 1024].any(), f"counters not re-armed (grid {grid})"
            outputs.append(c)
        for grid, c in zip((1, 5, tiles * splits - 1), outputs[1:]):
            assert torch.equal(c, outputs[0]), f"splits {splits} grid {grid} differs from grid = units"
        assert normwise(outputs[0], a.float() @ b.float()) <= 1e-2
        rows = slice(m - 3, m)
        assert normwise(outputs[0][rows], oracle_product(a[rows], b)) <= 1e-2
