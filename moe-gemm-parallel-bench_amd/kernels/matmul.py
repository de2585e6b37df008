"""Masked single GEMM on gfx950: config record, compiled tile menu, candidates and launcher.

Public surface and behaviour follow the reference's kernels/matmul.py:
  * ``KernelConfig`` (reference :19-32) with the same fields.  On this backend ``num_warps`` is the
    number of wave64 wavefronts per workgroup and ``num_stages`` the number of LDS stages of the
    K pipeline; ``group_size_m`` is the GROUP_M traversal width and ``cta_multiplier`` the
    persistent-grid multiplier of grouped launches.
  * ``select_config`` (:35-45) is the heuristic fallback; ``matmul_candidate_configs`` (:146-170)
    returns a bounded shape-family candidate set; ``diverse_configs`` (:101-120) keeps coverage of
    tile/traversal choices when truncating a ranked list.
  * ``launch_matmul`` (:332-392) validates like ``_validate_matrices`` (:318-329): ValueError for
    bad shapes/dtypes/devices, RuntimeError when the native library or a GPU is missing.  With
    ``autotune=True`` the first call for a shape key measures the candidates (hot graph timing)
    and later calls are a cache lookup plus exactly one kernel launch (capturable).
The kernel itself is ``csrc/gemm_kernel.h`` behind ``moegemm_matmul`` (include/moegemm.h).
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass

from utils.benchmark import hot_autotune_bench

from . import _native


@dataclass(frozen=True)
class KernelConfig:
    block_m: int
    block_n: int
    block_k: int
    group_size_m: int
    num_warps: int
    num_stages: int
    # Persistent-grid multiplier; only grouped launches use it.
    cta_multiplier: int = 1

    def as_dict(self) -> dict[str, int]:
        return asdict(self)

    @property
    def tile_key(self) -> tuple[int, int, int, int, int]:
        return (self.block_m, self.block_n, self.block_k, self.num_warps, self.num_stages)


# Compiled tile menus: (block_m, block_n, block_k, num_warps, num_stages).  They must equal the
# X-macro menus of csrc/registry.h; tests/test_native_abi.py compares them with the library.
_MENU_16BIT: tuple[tuple[int, int, int, int, int], ...] = (
    (256, 256, 64, 8, 2), (256, 256, 64, 4, 2), (256, 256, 32, 4, 4), (256, 256, 32, 8, 4),
    (256, 128, 64, 4, 3), (128, 256, 64, 8, 3), (128, 256, 64, 4, 3), (128, 128, 64, 4, 4), (128, 64, 64, 4, 4),
    (64, 256, 64, 4, 3), (64, 128, 64, 4, 4), (64, 64, 64, 4, 4),
    (32, 256, 64, 4, 4), (32, 128, 64, 4, 4), (32, 128, 128, 4, 3),
    (16, 256, 64, 4, 4), (16, 256, 128, 4, 2), (16, 128, 128, 4, 4),
    (16, 64, 128, 4, 4), (16, 64, 128, 4, 7),
    (16, 256, 64, 4, 2), (32, 256, 64, 4, 2), (64, 128, 64, 4, 2), (16, 128, 64, 4, 2),
    (16, 512, 64, 4, 2), (64, 512, 64, 4, 2),
    (32, 512, 32, 4, 4),
)
_MENU_F32: tuple[tuple[int, int, int, int, int], ...] = (
    (128, 128, 32, 4, 2), (64, 64, 32, 4, 2), (32, 64, 32, 4, 2),
    (16, 64, 32, 4, 2), (32, 32, 32, 2, 2),
)
_GROUP_SIZES = (1, 4, 8)


def _menu(dtype=None) -> tuple[tuple[int, int, int, int, int], ...]:
    return _MENU_F32 if _is_f32(dtype) else _MENU_16BIT


def _is_f32(dtype) -> bool:
    if dtype is None:
        return False
    if isinstance(dtype, str):
        return dtype == "fp32"
    return str(dtype) == "torch.float32"


def config_pool(dtype=None) -> tuple[KernelConfig, ...]:
    """Every launchable single-GEMM config for a dtype: compiled tiles x GROUP_M widths."""
    return tuple(
        KernelConfig(bm, bn, bk, group, warps, stages)
        for bm, bn, bk, warps, stages in _menu(dtype)
        for group in _GROUP_SIZES
    )


_MATMUL_CONFIG_POOL: tuple[KernelConfig, ...] = config_pool()
_MATMUL_CONFIG_POOL_F32: tuple[KernelConfig, ...] = config_pool("fp32")


def _snap(block_m: int, block_n: int, block_k: int, dtype=None, group: int = 8) -> KernelConfig:
    """The compiled tile nearest to a wanted (block_m, block_n, block_k), in log2 distance."""
    def distance(entry):
        bm, bn, bk, _, _ = entry
        return (abs(math.log2(bm / block_m)) + abs(math.log2(bn / block_n)), abs(math.log2(bk / block_k)))

    bm, bn, bk, warps, stages = min(_menu(dtype), key=distance)
    return KernelConfig(bm, bn, bk, group, warps, stages)


def select_config(m: int, n: int, k: int, dtype=None) -> KernelConfig:
    """Heuristic compiled config used before (or instead of) measurement."""
    if _is_f32(dtype):
        if m <= 16:
            return _snap(16, 64, 32, dtype)
        if m <= 32:
            return _snap(32, 64, 32, dtype)
        if m <= 64 or n <= 64:
            return _snap(64, 64, 32, dtype)
        return _snap(128, 128, 32, dtype)
    wide = 256 if n > 128 else 128 if n > 64 else 64
    if m <= 16:
        return _snap(16, wide, 128 if k >= 128 and wide < 256 else 64, dtype)
    if m <= 32:
        return _snap(32, 256 if n > 128 else 128, 64, dtype)
    if m <= 64:
        return _snap(64, wide, 64, dtype)
    if m <= 128:
        return _snap(128, 128 if n > 64 else 64, 64, dtype)
    if n <= 64:
        return _snap(128, 64, 64, dtype)
    return _snap(256, 256 if n > 128 else 128, 64, dtype)


def diverse_configs(ordered: list[KernelConfig], limit: int) -> list[KernelConfig]:
    """Truncate a best-first list to ``limit`` while covering distinct tile/traversal choices.

    Each pick is the remaining config that adds the most not-yet-covered choices, where a new
    (block_m, block_n) tile counts twice and a new block_k, GROUP_M, wave count or stage count
    once each; ties go to the better-ranked config.
    """
    def novelty(cfg: KernelConfig, seen: set) -> int:
        score = 2 if ("tile", (cfg.block_m, cfg.block_n)) not in seen else 0
        for key in (("bk", cfg.block_k), ("group", cfg.group_size_m), ("warps", cfg.num_warps),
                    ("stages", cfg.num_stages)):
            score += key not in seen
        return score

    remaining = list(dict.fromkeys(ordered))
    chosen: list[KernelConfig] = []
    seen: set = set()
    while remaining and len(chosen) < max(1, limit):
        best = max(range(len(remaining)), key=lambda i: (novelty(remaining[i], seen), -i))
        cfg = remaining.pop(best)
        chosen.append(cfg)
        seen |= {("tile", (cfg.block_m, cfg.block_n)), ("bk", cfg.block_k), ("group", cfg.group_size_m),
                 ("warps", cfg.num_warps), ("stages", cfg.num_stages)}
    return chosen


# MI355X figures used only to rank candidates before measurement.
_PEAK_FLOPS_16BIT = 2.5166e15
_PEAK_FLOPS_F32 = 1.573e14
_HBM_BYTES_PER_S = 8.0e12


def _mfma_fraction(cfg: KernelConfig) -> float:
    """Sustained fraction of MFMA peak the model assumes for a tile config (measured ordering on
    gfx950: the 8-wave 256 x 256 schedules lead; a wave tile past 128 x 64 accumulators spills)."""
    wave_tile = (cfg.block_m * cfg.block_n) / max(1, cfg.num_warps)
    if wave_tile > 8192:
        return 0.3
    if cfg.block_m == cfg.block_n == 256 and cfg.num_warps == 8:
        return 0.85 if cfg.num_stages >= 3 else 0.8
    return min(0.7, 0.25 + wave_tile / 16384.0)


def estimate_seconds(
    shapes, cfg: KernelConfig, element_size: int, sm_count: int, f32: bool = False
) -> float:
    """Rough roofline time of a tile config on a group of (M, K, N) problems.

    Compute: padded MFMA work at a tile-size-dependent fraction of peak, inflated by wave
    quantisation of the output tiles over the compute units.  Memory: A is re-read once per
    N tile and B once per M tile (L2 reuse ignored), plus one C write.
    """
    shapes = list(shapes)
    tiles = 0
    padded = 0
    traffic = 0
    for m, k, n in shapes:
        mt, nt, kt = math.ceil(m / cfg.block_m), math.ceil(n / cfg.block_n), math.ceil(k / cfg.block_k)
        tiles += mt * nt
        padded += 2 * mt * nt * kt * cfg.block_m * cfg.block_n * cfg.block_k
        traffic += element_size * (m * k * nt + k * n * mt + m * n)
    if not tiles:
        return 0.0
    units = max(1, sm_count or 256)
    waves = math.ceil(tiles / units)
    quantisation = waves * units / tiles
    mfma_fraction = _mfma_fraction(cfg)
    peak = _PEAK_FLOPS_F32 if f32 else _PEAK_FLOPS_16BIT
    compute = padded / (peak * mfma_fraction) * quantisation
    # A tile's K loop streams at most ~1/units of HBM bandwidth; few tiles cannot use it all.
    busy = min(1.0, tiles / units)
    memory = traffic / (_HBM_BYTES_PER_S * max(busy, 1.0 / units))
    return max(compute, memory)


def matmul_candidate_configs(m: int, n: int, k: int, limit: int = 10, *, dtype=None,
                             sm_count: int = 256) -> tuple[KernelConfig, ...]:
    """Bounded candidate set for one [m, k] @ [k, n] shape, best predicted first."""
    f32 = _is_f32(dtype)
    element_size = 4 if f32 else 2
    pool = config_pool(dtype)
    # Shape family: drop tiles whose M or N edge is more than twice the (rounded-up) extent.
    family = [
        cfg for cfg in pool
        if cfg.block_m <= max(16, 2 ** math.ceil(math.log2(max(m, 1))))
        and cfg.block_n <= max(64, 2 ** math.ceil(math.log2(max(n, 1))))
    ] or list(pool)
    fallback = select_config(m, n, k, dtype)
    if fallback not in family:
        family.append(fallback)
    # The model ignores L2 reuse, so GROUP_M only breaks ties: with several M tiles the widest group
    # goes first (the M tiles that share a B panel run together; measured 10 % faster on
    # [1024,14336]@[14336,4096] with the 128x128 tile), with one M tile the narrowest.
    ranked = sorted(
        family,
        key=lambda cfg: (estimate_seconds([(m, k, n)], cfg, element_size, sm_count, f32),
                         -_mfma_fraction(cfg), -cfg.block_m * cfg.block_n, cfg.block_k,
                         -cfg.group_size_m if m > cfg.block_m else cfg.group_size_m),
    )
    return tuple(diverse_configs(ranked, limit))


# -------------------------------------------------------------------------------------------------
# Launch

_AUTOTUNE_CACHE: dict[tuple, KernelConfig] = {}
_LAST_AUTOTUNED: list[KernelConfig | None] = [None]


def _device_signature(device) -> int:
    import torch

    props = torch.cuda.get_device_properties(device)
    return (int(props.major) * 10 + int(props.minor)) * 1000 + int(props.multi_processor_count)


def last_matmul_config(fallback: KernelConfig) -> KernelConfig:
    """Config selected by the most recent autotuned ``launch_matmul`` (else ``fallback``)."""
    return _LAST_AUTOTUNED[0] or fallback


def _validate_matrices(a, b, c) -> tuple[int, int, int]:
    if a.ndim != 2 or b.ndim != 2 or c.ndim != 2:
        raise ValueError("A, B, and C must be matrices")
    m, k = a.shape
    kb, n = b.shape
    if k != kb or tuple(c.shape) != (m, n):
        raise ValueError(f"shape mismatch: A={tuple(a.shape)}, B={tuple(b.shape)}, C={tuple(c.shape)}")
    if a.device != b.device or a.device != c.device or a.device.type != "cuda":
        raise ValueError("A, B, and C must be on the same GPU device")
    if a.dtype != b.dtype or a.dtype != c.dtype:
        raise ValueError("A, B, and C must have the same dtype")
    return int(m), int(n), int(k)


def _require_runtime() -> None:
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required to launch the native GEMM kernels")
    try:
        _native.library()
    except _native.NativeUnavailable as exc:
        raise RuntimeError(str(exc)) from exc


def _vector_ok(a, b, c) -> bool:
    """Preconditions of the LDS-DMA kernels for one 16-bit problem (see include/moegemm.h)."""
    import torch

    if a.dtype not in (torch.float16, torch.bfloat16):
        return False
    k = a.shape[1]
    n = b.shape[1]
    sam, sak = a.stride()
    sbk, sbn = b.stride()
    scm, scn = c.stride()
    return (
        sak == 1 and sbn == 1 and scn == 1
        and k % 8 == 0 and n % 8 == 0 and sam % 8 == 0 and sbk % 8 == 0 and scm % 4 == 0
        and sam >= k and sbk >= n and scm >= n
        and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0 and c.data_ptr() % 8 == 0
        and _native.panels_fit(k, sam, sbk, scm)
    )


def splitk_count(tiles: int, k: int, block_k: int, sm_count: int) -> int:
    """K splits for a launch with ``tiles`` output tiles: 1 unless the tiles leave over half the CUs
    idle; otherwise enough splits to give every CU a unit, each at least 4 K slices, at most 16."""
    if tiles <= 0 or 2 * tiles > sm_count:
        return 1
    splits = min(sm_count // tiles, k // (4 * block_k), 16)
    return splits if splits >= 2 else 1


def with_split_options(configs, tiles_of, k: int, sm_count: int, split_k, splittable: bool) -> list:
    """(config, split) tuning candidates: each config unsplit and, where ``splitk_count`` would
    split it, also split — so measurement, not the heuristic alone, decides.  An explicit
    ``split_k`` pins the split of every candidate."""
    out = []
    for cfg in configs:
        if split_k is not None:
            out.append((cfg, split_k))
            continue
        out.append((cfg, 1))
        splits = splitk_count(tiles_of(cfg), k, cfg.block_k, sm_count) if splittable else 1
        if splits > 1:
            out.append((cfg, splits))
    return out


_LAST_SPLIT: list[int] = [1]
_LAST_SCHEDULE: list[str] = ["static"]
_LAST_B_STREAM: list[int] = [0]
STREAMK = "streamk"  # split option of a tuning candidate: whole tiles in exact rounds, then a stream-K tail


def last_matmul_split() -> int:
    """K splits used by the most recent ``launch_matmul`` call (1 = no split-K)."""
    return _LAST_SPLIT[0]


def last_matmul_schedule() -> str:
    """Tile schedule of the most recent ``launch_matmul`` call: "static" or "streamk"."""
    return _LAST_SCHEDULE[0]


def last_matmul_b_stream() -> int:
    """B copy policy of the most recent ``launch_matmul`` call: 1 = non-temporal B copies."""
    return _LAST_B_STREAM[0]


def _streamk_tail(a, b, c, m, n, k, cfg: KernelConfig) -> int:
    """Tail tiles of a stream-K launch of this GEMM on one workgroup per CU (0: not applicable)."""
    if not _vector_ok(a, b, c):
        return 0
    tiles = -(-m // cfg.block_m) * -(-n // cfg.block_n)
    return _native.streamk_tail(tiles, _device_signature(a.device) % 1000, k, cfg.block_k)


def _launch_fixed_streamk(a, b, c, m, n, k, cfg: KernelConfig, dtype_code: int, tail: int, b_stream: int = 0) -> None:
    grid = _device_signature(a.device) % 1000
    stream = _native.current_stream_handle(a.device)
    workspace = _native.splitk_workspace(a.device, stream,
                                         _native.streamk_workspace_bytes(tail, grid, cfg.block_m, cfg.block_n))
    status = _native.library().moegemm_matmul_streamk(
        a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k,
        a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1), dtype_code,
        cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages, tail, grid,
        workspace.data_ptr(), workspace.numel(), b_stream, stream,
    )
    _native.check(status)


def _launch_fixed_splitk(a, b, c, m, n, k, cfg: KernelConfig, dtype_code: int, splits: int, b_stream: int = 0) -> None:
    tiles = -(-m // cfg.block_m) * -(-n // cfg.block_n)
    nbytes = _native.splitk_workspace_bytes(tiles, splits, cfg.block_m, cfg.block_n)
    stream = _native.current_stream_handle(a.device)
    workspace = _native.splitk_workspace(a.device, stream, nbytes)
    status = _native.library().moegemm_matmul_splitk(
        a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k,
        a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1), dtype_code,
        cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages, splits,
        0, workspace.data_ptr(), workspace.numel(), b_stream, stream,
    )
    _native.check(status)


def _launch_fixed(a, b, c, m, n, k, cfg: KernelConfig, dtype_code: int, precision: int, split_k=None,
                  b_stream: int = 0) -> int:
    """One launch; returns the K splits used (``split_k`` None = ``splitk_count``'s choice,
    ``STREAMK`` = a stream-K tail where one applies, else the unsplit launch).  ``b_stream`` 1 issues
    the LDS-DMA kernels' B copies non-temporal."""
    _LAST_SCHEDULE[0] = "static"
    _LAST_B_STREAM[0] = b_stream
    if split_k == STREAMK:
        tail = _streamk_tail(a, b, c, m, n, k, cfg) if precision == _native.PRECISION_IEEE else 0
        if tail:
            _launch_fixed_streamk(a, b, c, m, n, k, cfg, dtype_code, tail, b_stream)
            _LAST_SCHEDULE[0] = STREAMK
            return 1
        split_k = 1
    splits = 1
    if _vector_ok(a, b, c):
        tiles = -(-m // cfg.block_m) * -(-n // cfg.block_n)
        splits = split_k if split_k is not None else splitk_count(tiles, k, cfg.block_k,
                                                                  _device_signature(a.device) % 1000)
    if splits > 1:
        _launch_fixed_splitk(a, b, c, m, n, k, cfg, dtype_code, splits, b_stream)
        return splits
    lib = _native.library()
    status = lib.moegemm_matmul(
        a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k,
        a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1),
        dtype_code, precision,
        cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages,
        0, b_stream, _native.current_stream_handle(a.device),
    )
    _native.check(status)
    return 1


def launch_matmul(
    a,
    b,
    c,
    config: KernelConfig | None = None,
    input_precision: str = "ieee",
    *,
    autotune: bool = True,
    split_k: int | None = None,
    b_stream: int | None = None,
) -> None:
    """Launch C = A @ B: autotuned per shape key, or with an explicit config when autotune is false.

    ``split_k`` (keyword-only, not in the reference's signature): None lets ``splitk_count`` split
    K when the output tiles leave most CUs idle (fp16/bf16 vector layouts, one launch with a
    deterministic in-kernel reduction); 1 disables it; n > 1 forces n splits.
    ``b_stream`` (keyword-only, not in the reference's signature): 1 issues the LDS-DMA kernels' B
    copies non-temporal, 0 as ordinary loads; None lets the tuner measure both (0 without
    autotuning).  ``last_matmul_b_stream()`` reports what ran.
    """
    m, n, k = _validate_matrices(a, b, c)
    _require_runtime()
    dtype_code = _native.dtype_code(a.dtype)
    precision = _native.precision_code(input_precision, dtype_code)
    if split_k is not None and split_k < 1:
        raise ValueError("split_k must be None or a positive integer")
    if b_stream not in (None, 0, 1):
        raise ValueError(f"b_stream must be None, 0 or 1, got {b_stream!r}")
    if not autotune:
        cfg = config or select_config(m, n, k, a.dtype)
        _LAST_SPLIT[0] = _launch_fixed(a, b, c, m, n, k, cfg, dtype_code, precision, split_k, b_stream or 0)
        return
    key = (
        m, n, k, tuple(a.stride()), tuple(b.stride()), tuple(c.stride()), dtype_code, precision,
        _device_signature(a.device), split_k, b_stream,
    )
    best = _AUTOTUNE_CACHE.get(key)
    if best is None:
        sm_count = _device_signature(a.device) % 1000
        configs = matmul_candidate_configs(m, n, k, dtype=a.dtype, sm_count=sm_count)
        options = with_split_options(configs, lambda cfg: -(-m // cfg.block_m) * -(-n // cfg.block_n), k,
                                     sm_count, split_k, _vector_ok(a, b, c))
        if split_k is None:  # a stream-K tail where the tiles leave a partial last round
            options += [(cfg, STREAMK) for cfg in configs if _streamk_tail(a, b, c, m, n, k, cfg)]
        options = [(cfg, split, b_stream or 0) for cfg, split in options]
        # The B copy policy is timed on the finalists where it is not pinned and the LDS-DMA kernels run.
        twin = (lambda o: (o[0], o[1], 1)) if b_stream is None and _vector_ok(a, b, c) else None
        best = _tune(options, lambda o: _launch_fixed(a, b, c, m, n, k, o[0], dtype_code, precision, o[1], o[2]),
                     twin=twin)
        _AUTOTUNE_CACHE[key] = best
    _LAST_AUTOTUNED[0] = best[0]
    _LAST_SPLIT[0] = _launch_fixed(a, b, c, m, n, k, best[0], dtype_code, precision, best[1], best[2])


def _warm_clocks(launch, budget_ms: float = 100.0) -> None:
    """Run ``launch`` back to back for ~budget_ms so the GPU is at its working clock before timing."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    launch()
    end.record()
    end.synchronize()
    per_call = max(start.elapsed_time(end), 0.01)
    for _ in range(min(2000, int(budget_ms / per_call))):
        launch()
    torch.cuda.synchronize()


_FINALISTS = 5
# Rounds of the interleaved finalist timing.  One ~25 ms sample of a ~40 us launch spreads about
# +-6 % on the MI355X (clock and power drift), against gaps of 2-5 % between the finalists of
# mid-size launches (Mixtral W13 at M_e = 128); the median of seven rounds narrows the spread at
# about 0.2 s per finalist.
_FINAL_ROUNDS = 7


def _tune(candidates, launch, prefer=None, prefer_margin: float = 0.03, twin=None):
    """Hot-time every candidate (graph replays, bounded) after a clock warm-up, twice (a forward and a
    reverse sweep), then re-time the best five interleaved (seven rounds of A, B, C, D, E) and keep
    the lowest median, so a clock drift during tuning shifts every finalist alike instead of
    favouring whichever ran at the better moment, and a candidate that a noisy first pass ranked
    fourth or fifth still competes.

    ``prefer`` (one of the candidates) always joins the finalists and is kept unless another
    finalist is faster by more than ``prefer_margin``: a choice already measured on the same
    workload is not overturned by timing noise.  ``twin(option)`` (or None) names a variant of a
    finalist that only the interleaved rounds time, next to it: the non-temporal B copies, whose
    effect depends on the workload but hardly on which of the leading tiles runs."""
    candidates = list(candidates)
    first: dict[int, float] = {}
    failed: set[int] = set()
    warmed = False
    # Two sweeps, forward then reverse, keeping each candidate's lower median: a candidate timed
    # while the clock was still settling (the first ones after the warm-up) gets a second sample
    # at the other end of the pass before the finalists are cut.
    for order in (range(len(candidates)), reversed(range(len(candidates)))):
        for index in order:
            if index in failed:
                continue
            cfg = candidates[index]
            try:
                if not warmed:
                    _warm_clocks(lambda cfg=cfg: launch(cfg))
                    warmed = True
                median_ms = hot_autotune_bench(lambda cfg=cfg: launch(cfg), (0.5,))[0]
            except (RuntimeError, ValueError):
                failed.add(index)
                first.pop(index, None)
                continue
            first[index] = min(median_ms, first.get(index, math.inf))
    measured = [(first[index], candidates[index]) for index in sorted(first)]
    if not measured:
        raise RuntimeError("every autotune candidate failed to launch")
    measured.sort(key=lambda item: item[0])
    finalists = [cfg for _, cfg in measured[:_FINALISTS]]
    if prefer is not None and prefer not in finalists and any(cfg == prefer for _, cfg in measured):
        finalists.append(prefer)
    if twin is not None:
        finalists += [t for t in dict.fromkeys(twin(cfg) for cfg in finalists) if t is not None and t not in finalists]
    rounds: list[list[float]] = [[] for _ in finalists]
    for _ in range(_FINAL_ROUNDS):
        for index, cfg in enumerate(finalists):
            rounds[index].append(hot_autotune_bench(lambda cfg=cfg: launch(cfg), (0.5,))[0])
    medians = [sorted(times)[_FINAL_ROUNDS // 2] for times in rounds]
    best = finalists[medians.index(min(medians))]
    if prefer in finalists and medians[finalists.index(prefer)] <= min(medians) * (1.0 + prefer_margin):
        return prefer
    return best
