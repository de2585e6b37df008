"""Persistent grouped GEMM over distinct expert A/B/C pointers, on gfx950.

Same public surface as the reference's kernels/grouped_gemm.py:
  * ``GroupedWorkspace`` (reference :67-111): per-problem tensors, int64 pointer tables, int32
    ``dims`` [G,3] = (m, n, k), int64 ``strides`` [G,6] = (am, ak, bk, bn, cm, cn), provenance.
  * ``build_grouped_workspace`` / ``build_fused_gate_up_workspace`` (:507-594): seeded device RNG
    ``normal_() * 0.1`` inputs; W13 packs [gate | up] along N in one B and one C per expert.
  * ``grouped_candidate_configs`` (:114-224): bounded workload-aware candidates including
    persistent-grid multipliers.
  * ``launch_grouped`` (:618-760): G == 1 dispatches to ``launch_matmul`` ("single_problem_matmul");
    equal contiguous problems use the homogeneous mode ("homogeneous_persistent"); anything else
    the generic mode with device dims/strides ("generic_persistent").  Exactly one kernel launch
    per call; ``workspace.config`` / ``workspace.scheduler`` record what ran.
The device code is one templated HIP kernel (csrc/gemm_kernel.h) behind ``moegemm_grouped_gemm``.
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from dataclasses import dataclass

from . import _native
from .matmul import (
    KernelConfig,
    last_matmul_b_stream,
    last_matmul_schedule,
    last_matmul_split,
    splitk_count,
    with_split_options,
    _is_f32,
    _require_runtime,
    _tune,
    config_pool,
    diverse_configs,  # importable from here as in the reference's kernels/grouped_gemm.py
    estimate_seconds,
    last_matmul_config,
    launch_matmul,
    matmul_candidate_configs,
    select_config,
)

_CTA_MULTIPLIERS = (1, 2, 4)

# Base configs (cta_multiplier == 1) from which grouped candidates are drawn.
_GROUPED_BASE_CONFIG_POOL: tuple[KernelConfig, ...] = config_pool()
_GROUPED_BASE_CONFIG_POOL_F32: tuple[KernelConfig, ...] = config_pool("fp32")


@dataclass
class GroupedWorkspace:
    a: list
    b: list
    c: list
    a_ptrs: object
    b_ptrs: object
    c_ptrs: object
    dims: object
    strides: object
    shapes: tuple[tuple[int, int, int], ...]
    config: KernelConfig
    shape_signature: int
    device_signature: int
    sm_count: int
    storage_bytes: int
    homogeneous: bool
    operation: str = "gemm"
    scheduler: str = "not_launched"
    # Fused SwiGLU outputs H_e [M_e, N_e / 2] and their tables (allocated by launch_gate_up_swiglu).
    h: list | None = None
    h_ptrs: object = None
    h_strides: object = None
    swiglu_config: KernelConfig | None = None
    split_k: int = 1  # K splits of the most recent launch (1 = no split-K)
    # Tile schedule of the last launch: "static", "stealing" (work-stealing tile queues) or "streamk"
    # (whole tiles in exact rounds, then a stream-K tail).
    tile_schedule: str = "static"
    b_stream: int = 0  # 1: the last launch issued its B copies non-temporal
    swiglu_b_stream: int = 0  # the same for the last launch_gate_up_swiglu call

    @property
    def problem_count(self) -> int:
        return len(self.a)

    def _shape_stats(self) -> tuple:
        """(shapes, (max M, max N, max K), tile counts by (BM, BN)), kept while ``shapes`` is the same
        tuple object: every launch reads them, and over hundreds of problems recomputing them costs
        as much host time as a decode-sized kernel runs."""
        cached = self.__dict__.get("_shape_stats_cache")
        if cached is None or cached[0] is not self.shapes:
            shapes = self.shapes
            maxima = (max(m for m, _, _ in shapes), max(n for _, _, n in shapes), max(k for _, k, _ in shapes))
            cached = (shapes, maxima, {})
            self.__dict__["_shape_stats_cache"] = cached
        return cached

    @property
    def max_m(self) -> int:
        return self._shape_stats()[1][0]

    @property
    def max_n(self) -> int:
        return self._shape_stats()[1][1]

    @property
    def max_k(self) -> int:
        return self._shape_stats()[1][2]

    def tile_count_for(self, config: KernelConfig) -> int:
        shapes, _, counts = self._shape_stats()
        key = (config.block_m, config.block_n)
        count = counts.get(key)
        if count is None:
            count = counts[key] = sum(math.ceil(m / config.block_m) * math.ceil(n / config.block_n)
                                      for m, _, n in shapes)
        return count

    @property
    def tile_count(self) -> int:
        return self.tile_count_for(self.config)

    def problem_tensors(self):
        return zip(self.a, self.b, self.c)


def grouped_candidate_configs(
    max_m: int,
    max_n: int,
    max_k: int,
    base_limit: int = 12,
    *,
    problem_count: int = 1,
    sm_count: int = 0,
    dtype=None,
) -> tuple[KernelConfig, ...]:
    """Workload-aware tile and persistent-grid candidates (at most 36).

    Tile shapes (block_m, block_n) are ranked by ``estimate_seconds`` on the whole group, so a narrow
    N tile that exposes enough expert tiles to fill the device can outrank a better-padded wide one.
    The best-ranked shapes keep every compiled variant (block_k, waves, LDS stages), because the
    cost model cannot tell those apart and measurement can; GROUP_M variants are added only when a
    problem spans several M tiles (otherwise traversal order is the same).  Each kept config gets
    cta_multiplier 1, plus 2 (and 4 for skinny tiles) only when the group has more tiles than one
    grid's worth, so no two candidates launch the same grid.  A single problem dispatches to the
    single-GEMM path, whose candidates carry cta_multiplier 1 only.
    """
    if min(max_m, max_n, max_k, problem_count) <= 0:
        raise ValueError("grouped candidate dimensions and problem_count must be positive")
    if sm_count < 0:
        raise ValueError("sm_count must be non-negative")
    if problem_count == 1:
        return tuple(
            KernelConfig(c.block_m, c.block_n, c.block_k, c.group_size_m, c.num_warps, c.num_stages, 1)
            for c in matmul_candidate_configs(max_m, max_n, max_k, limit=base_limit, dtype=dtype,
                                              sm_count=sm_count or 256)
        )
    f32 = _is_f32(dtype)
    element_size = 4 if f32 else 2
    shapes = [(max_m, max_k, max_n)] * problem_count
    units = sm_count or 256
    # Decode groups (max_m <= 16) also try 32-row tiles: a 32x512x32 four-stage tile measured 2.8 %
    # faster than the best 16-row tile on DSV3 EP W2 at M_e = 8, though it pads more rows.
    decode = max_m <= 16
    m_cap = max(32 if decode else 16, 2 ** math.ceil(math.log2(max_m)))
    pool = [cfg for cfg in config_pool(dtype) if cfg.block_m <= m_cap] or list(config_pool(dtype))
    by_tile: dict[tuple[int, int], list[KernelConfig]] = {}
    for cfg in pool:
        by_tile.setdefault((cfg.block_m, cfg.block_n), []).append(cfg)
    score = {tile: min(estimate_seconds(shapes, cfg, element_size, units, f32) for cfg in cfgs)
             for tile, cfgs in by_tile.items()}
    tiles = sorted(by_tile, key=lambda t: (score[t], -t[0] * t[1]))
    candidates: list[KernelConfig] = []
    limit = 36
    for tile in tiles:
        several_m_tiles = math.ceil(max_m / tile[0]) > 1
        variants = [cfg for cfg in by_tile[tile] if cfg.group_size_m in ((1, 8) if several_m_tiles else (8,))]
        tile_count = problem_count * math.ceil(max_m / tile[0]) * math.ceil(max_n / tile[1])
        multipliers = [1]
        if not sm_count or tile_count > sm_count:
            multipliers.append(2)
        if tile[0] <= 32 and (not sm_count or tile_count > 2 * sm_count):
            multipliers.append(4)
        expanded = [KernelConfig(c.block_m, c.block_n, c.block_k, c.group_size_m, c.num_warps, c.num_stages, mult)
                    for c in variants for mult in multipliers]
        if candidates and len(candidates) + len(expanded) > limit:
            break
        candidates.extend(expanded[: limit - len(candidates)])
        if len({(c.block_m, c.block_n) for c in candidates}) >= max(1, base_limit // 3) + (2 if decode else 0):
            break
    fallback = select_config(max_m, max_n, max_k, dtype)
    if not any(c.tile_key == fallback.tile_key for c in candidates) and len(candidates) < limit:
        candidates.append(fallback)
    return tuple(dict.fromkeys(candidates))


def _shape_signature(shapes: Sequence[tuple[int, int, int]]) -> int:
    """31-bit FNV-1a-style fold of every dimension; an autotune-cache discriminator only.

    Same fold as the reference's kernels/grouped_gemm.py:227-233, so cache keys agree.
    """
    value = 2166136261
    for shape in shapes:
        for dimension in shape:
            value = ((value ^ int(dimension)) * 16777619) & 0x7FFFFFFF
    return value


def _normalize(shapes) -> tuple[tuple[int, int, int], ...]:
    if not shapes:
        raise ValueError("grouped GEMM requires at least one problem")
    normalized = tuple(tuple(int(v) for v in shape) for shape in shapes)
    if any(len(s) != 3 or any(v <= 0 for v in s) for s in normalized):
        raise ValueError("every grouped shape must be a positive (M, K, N) triple")
    return normalized


def workspace_from_tensors(arrays_a, arrays_b, arrays_c, config: KernelConfig | None = None) -> GroupedWorkspace:
    """Wrap caller-owned per-problem tensors (any strides) in a GroupedWorkspace."""
    import torch

    if not (len(arrays_a) == len(arrays_b) == len(arrays_c)) or not arrays_a:
        raise ValueError("A, B and C lists must be non-empty and of equal length")
    shapes = []
    for a, b, c in zip(arrays_a, arrays_b, arrays_c):
        if a.ndim != 2 or b.ndim != 2 or c.ndim != 2 or a.shape[1] != b.shape[0] or tuple(c.shape) != (a.shape[0], b.shape[1]):
            raise ValueError(f"shape mismatch: A={tuple(a.shape)}, B={tuple(b.shape)}, C={tuple(c.shape)}")
        shapes.append((int(a.shape[0]), int(a.shape[1]), int(b.shape[1])))
    normalized = _normalize(shapes)
    device = arrays_a[0].device
    dtype = arrays_a[0].dtype
    for tensor in (*arrays_a, *arrays_b, *arrays_c):
        if tensor.device != device or tensor.dtype != dtype:
            raise ValueError("every grouped tensor must share one device and dtype")
    first_m, first_k, first_n = normalized[0]
    config = config or select_config(first_m, first_n, first_k, dtype)

    def pointer_table(arrays):
        return torch.tensor([t.data_ptr() for t in arrays], device=device, dtype=torch.int64)

    a_ptrs, b_ptrs, c_ptrs = pointer_table(arrays_a), pointer_table(arrays_b), pointer_table(arrays_c)
    dims = torch.tensor([[m, n, k] for m, k, n in normalized], device=device, dtype=torch.int32)
    strides = torch.tensor(
        [[a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1)]
         for a, b, c in zip(arrays_a, arrays_b, arrays_c)],
        device=device, dtype=torch.int64,
    )
    tables = [a_ptrs, b_ptrs, c_ptrs, dims, strides]
    storage_bytes = sum(t.numel() * t.element_size() for t in (*arrays_a, *arrays_b, *arrays_c, *tables))
    if device.type == "cuda":
        props = torch.cuda.get_device_properties(device)
        sm_count = int(props.multi_processor_count)
        device_signature = (int(props.major) * 10 + int(props.minor)) * 1000 + sm_count
    else:
        sm_count, device_signature = 0, 0
    homogeneous = all(s == normalized[0] for s in normalized) and all(
        t.is_contiguous() for t in (*arrays_a, *arrays_b, *arrays_c)
    )
    return GroupedWorkspace(
        list(arrays_a), list(arrays_b), list(arrays_c), a_ptrs, b_ptrs, c_ptrs, dims, strides,
        normalized, config, _shape_signature(normalized), device_signature, sm_count, storage_bytes,
        homogeneous,
    )


def build_grouped_workspace(
    shapes: Sequence[tuple[int, int, int]],
    dtype,
    seed: int = 0,
    config: KernelConfig | None = None,
    *,
    device: str = "cuda",
) -> GroupedWorkspace:
    """Allocate G independent (A, B, C) triples with seeded ``normal_() * 0.1`` inputs.

    ``device="cpu"`` builds the same layout on the host (for the CPU oracle and plumbing checks);
    launching still requires a GPU.
    """
    import torch

    normalized = _normalize(shapes)
    if device != "cpu" and not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required to build device workspaces")
    generator = torch.Generator(device=device).manual_seed(seed)
    arrays_a, arrays_b, arrays_c = [], [], []
    for m, k, n in normalized:
        arrays_a.append(torch.empty((m, k), device=device, dtype=dtype).normal_(generator=generator).mul_(0.1))
        arrays_b.append(torch.empty((k, n), device=device, dtype=dtype).normal_(generator=generator).mul_(0.1))
        arrays_c.append(torch.empty((m, n), device=device, dtype=dtype))
    return workspace_from_tensors(arrays_a, arrays_b, arrays_c, config)


def build_fused_gate_up_workspace(
    shapes: Sequence[tuple[int, int, int]],
    dtype,
    seed: int = 0,
    config: KernelConfig | None = None,
    *,
    device: str = "cuda",
) -> GroupedWorkspace:
    """Packed W13 problems: each B_e is [H, 2F] = [gate | up], each C_e is [M_e, 2F] = [gate | up]."""
    normalized = tuple(tuple(int(v) for v in shape) for shape in shapes)
    if any(len(s) != 3 or s[2] % 2 for s in normalized):
        raise ValueError("fused Gate+Up shapes require an even packed output dimension")
    workspace = build_grouped_workspace(normalized, dtype, seed, config, device=device)
    workspace.operation = "gate_up"
    return workspace


def _grid_size(workspace: GroupedWorkspace, config: KernelConfig) -> int:
    tiles = workspace.tile_count_for(config)
    return max(1, min(tiles, workspace.sm_count * config.cta_multiplier))


def _problem_vector_ok(a, b, c) -> bool:
    """Preconditions of the LDS-DMA kernel for one problem (see include/moegemm.h)."""
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


def _vector_layout(workspace: GroupedWorkspace, dtype_code: int) -> bool:
    """True when every problem meets the fast kernel's layout; cached per set of tensor objects."""
    if dtype_code == _native.DTYPE_F32:
        return False
    key = (tuple(map(id, workspace.a)), tuple(map(id, workspace.b)), tuple(map(id, workspace.c)))
    cached = getattr(workspace, "_layout_cache", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    value = all(_problem_vector_ok(a, b, c) for a, b, c in zip(workspace.a, workspace.b, workspace.c))
    workspace._layout_cache = (key, value)
    return value


def _check_workspace(workspace: GroupedWorkspace) -> int:
    a0, b0, c0 = workspace.a[0], workspace.b[0], workspace.c[0]
    if a0.device.type != "cuda":
        raise RuntimeError("grouped launches need the workspace on a ROCm GPU")
    if a0.dtype != b0.dtype or a0.dtype != c0.dtype:
        raise ValueError("A, B, and C must have the same dtype")
    return _native.dtype_code(a0.dtype)


def _grouped_splits(workspace: GroupedWorkspace, cfg: KernelConfig, dtype_code: int, split_k, vector=None) -> int:
    if vector is None:
        vector = _vector_layout(workspace, dtype_code)
    if not workspace.homogeneous or not vector:
        return 1
    if split_k is not None:
        return split_k
    return splitk_count(workspace.tile_count_for(cfg), workspace.max_k, cfg.block_k, workspace.sm_count)


def with_schedule_options(options, tile_schedule: str | None, streamk_ok=None) -> list:
    """(config, split, schedule) tuning candidates: unsplit options run under the static and the
    stealing schedule, and under "streamk" where ``streamk_ok(config)`` says a stream-K tail
    applies, unless ``tile_schedule`` pins one; split options stay static."""
    out = []
    for cfg, split in options:
        streamk = split == 1 and streamk_ok is not None and streamk_ok(cfg)
        if split == 1 and tile_schedule is None:
            out += [(cfg, 1, "static"), (cfg, 1, "stealing")]
            if streamk:
                out.append((cfg, 1, "streamk"))
        elif tile_schedule == "streamk":
            if streamk:
                out.append((cfg, 1, "streamk"))
        elif split == 1 or tile_schedule != "stealing":
            out.append((cfg, split, tile_schedule or "static"))
    return out


def streamk_tail_for(workspace: GroupedWorkspace, cfg: KernelConfig, dtype_code: int) -> int:
    """Tail tiles of a stream-K launch of this workspace with ``cfg`` (0: stream-K does not apply).
    Homogeneous fp16/bf16 vector-layout groups only, on a grid of one workgroup per CU."""
    if not workspace.homogeneous or cfg.cta_multiplier != 1 or not _vector_layout(workspace, dtype_code):
        return 0
    return _native.streamk_tail(workspace.tile_count_for(cfg), workspace.sm_count, workspace.max_k, cfg.block_k)


def _launch_grouped_fixed(workspace: GroupedWorkspace, cfg: KernelConfig, dtype_code: int, precision: int,
                          split_k=None, schedule: str = "static", b_stream: int = 0) -> int:
    """One launch; returns the K splits used.  ``schedule`` "stealing" draws the tiles from the
    work-stealing queues (unsplit launches only); ``b_stream`` 1 issues the LDS-DMA kernels' B copies
    non-temporal."""
    if schedule == "streamk":
        tail = streamk_tail_for(workspace, cfg, dtype_code)
        if tail:
            m, k, n = workspace.shapes[0]
            grid = workspace.sm_count
            stream = _native.current_stream_handle(workspace.a[0].device)
            scratch = _native.splitk_workspace(workspace.a[0].device, stream,
                                               _native.streamk_workspace_bytes(tail, grid, cfg.block_m, cfg.block_n))
            status = _native.library().moegemm_grouped_gemm_streamk(
                workspace.a_ptrs.data_ptr(), workspace.b_ptrs.data_ptr(), workspace.c_ptrs.data_ptr(),
                workspace.problem_count, m, n, k, dtype_code,
                cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages, tail, grid,
                1, scratch.data_ptr(), scratch.numel(), b_stream, stream,
            )
            _native.check(status)
            return 1
        schedule = "static"  # no partial last round: the static launch is the same work
    vector = _vector_layout(workspace, dtype_code)
    splits = _grouped_splits(workspace, cfg, dtype_code, split_k, vector)
    if schedule == "stealing" and splits > 1:
        raise ValueError("the work-stealing schedule runs unsplit launches only (split_k must be 1)")
    if splits > 1:
        m, k, n = workspace.shapes[0]
        tiles = workspace.tile_count_for(cfg)
        stream = _native.current_stream_handle(workspace.a[0].device)
        scratch = _native.splitk_workspace(workspace.a[0].device, stream,
                                           _native.splitk_workspace_bytes(tiles, splits, cfg.block_m, cfg.block_n))
        status = _native.library().moegemm_grouped_gemm_splitk(
            workspace.a_ptrs.data_ptr(), workspace.b_ptrs.data_ptr(), workspace.c_ptrs.data_ptr(),
            workspace.problem_count, m, n, k, dtype_code,
            cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages, splits,
            max(1, min(tiles * splits, workspace.sm_count * cfg.cta_multiplier)), 1,
            scratch.data_ptr(), scratch.numel(), b_stream, stream,
        )
        _native.check(status)
        return splits
    lib = _native.library()
    m, k, n = workspace.shapes[0]
    stream = _native.current_stream_handle(workspace.a[0].device)
    args = (
        workspace.a_ptrs.data_ptr(), workspace.b_ptrs.data_ptr(), workspace.c_ptrs.data_ptr(),
        workspace.dims.data_ptr(), workspace.strides.data_ptr(),
        workspace.problem_count, m, n, k, 1 if workspace.homogeneous else 0,
        workspace.tile_count_for(cfg), dtype_code, precision,
        cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages,
        _grid_size(workspace, cfg), 1 if vector else 0,
    )
    if schedule == "stealing":
        queue = _native.tile_queue(workspace.a[0].device, stream)
        status = lib.moegemm_grouped_gemm_stealing(*args, queue.data_ptr(), b_stream, stream)
    elif schedule == "static":
        status = lib.moegemm_grouped_gemm(*args, b_stream, stream)
    else:
        raise ValueError(f"tile_schedule must be one of {_native.TILE_SCHEDULES}, got {schedule!r}")
    _native.check(status)
    return 1


_GROUPED_AUTOTUNE_CACHE: dict[tuple, tuple] = {}


def _grouped_tuning_key(workspace: GroupedWorkspace, scheduler: str, dtype_code: int, precision: int, split_k,
                        tile_schedule, b_stream=None) -> tuple:
    return (scheduler, workspace.problem_count, workspace.max_m, workspace.max_n, workspace.max_k,
            workspace.shape_signature, workspace.device_signature, workspace.sm_count, dtype_code, precision,
            split_k, tile_schedule, b_stream)


def launch_grouped(
    workspace: GroupedWorkspace,
    input_precision: str = "ieee",
    config: KernelConfig | None = None,
    *,
    autotune: bool = True,
    split_k: int | None = None,
    tile_schedule: str | None = None,
    b_stream: int | None = None,
) -> None:
    """Launch the persistent grouped kernel (autotuned per workload key, or a fixed config).

    ``split_k`` (keyword-only, not in the reference's signature) as for ``launch_matmul``: None
    splits K inside the one launch when a homogeneous 16-bit group has too few tiles to fill the
    CUs; 1 disables it; n forces n.  ``workspace.split_k`` records what ran.
    ``tile_schedule`` (keyword-only, not in the reference's signature): "static" (tiles pid,
    pid + grid, ... as the reference's programs take them), "stealing" (per-XCD tile queues
    with stealing) or "streamk" (whole tiles in exact rounds of one workgroup per CU, then the
    remaining tiles' K slices spread over every workgroup; homogeneous 16-bit groups whose tile
    count leaves a partial last round, static otherwise); None lets the tuner measure them
    (static without autotuning).  ``workspace.tile_schedule`` records what ran.  ``b_stream``
    (keyword-only, not in the reference's signature): 1 issues the LDS-DMA kernels' B copies
    non-temporal, 0 as ordinary loads, None lets the tuner measure both on its finalists (0 without
    autotuning); ``workspace.b_stream`` records what ran.  G == 1 always runs the single GEMM.
    """
    if split_k is not None and split_k < 1:
        raise ValueError("split_k must be None or a positive integer")
    if tile_schedule is not None and tile_schedule not in _native.GROUPED_SCHEDULES:
        raise ValueError(f"tile_schedule must be None or one of {_native.GROUPED_SCHEDULES}, got {tile_schedule!r}")
    if tile_schedule in ("stealing", "streamk") and split_k is not None and split_k > 1:
        raise ValueError(f"the {tile_schedule} schedule runs unsplit launches only (split_k must be 1)")
    if b_stream not in (None, 0, 1):
        raise ValueError(f"b_stream must be None, 0 or 1, got {b_stream!r}")
    _require_runtime()
    cfg = config or workspace.config
    if workspace.problem_count == 1:
        launch_matmul(workspace.a[0], workspace.b[0], workspace.c[0], cfg, input_precision, autotune=autotune,
                      split_k=split_k, b_stream=b_stream)
        workspace.config = last_matmul_config(cfg) if autotune else cfg
        workspace.scheduler = "single_problem_matmul"
        workspace.split_k = last_matmul_split()
        workspace.tile_schedule = last_matmul_schedule()
        workspace.b_stream = last_matmul_b_stream()
        return
    dtype_code = _check_workspace(workspace)
    precision = _native.precision_code(input_precision, dtype_code)
    scheduler = "homogeneous_persistent" if workspace.homogeneous else "generic_persistent"
    if autotune:
        key = _grouped_tuning_key(workspace, scheduler, dtype_code, precision, split_k, tile_schedule, b_stream)
        tuned = _GROUPED_AUTOTUNE_CACHE.get(key)
        if tuned is None:
            candidates = grouped_candidate_configs(
                workspace.max_m, workspace.max_n, workspace.max_k,
                problem_count=workspace.problem_count, sm_count=workspace.sm_count, dtype=workspace.a[0].dtype,
            )
            splittable = workspace.homogeneous and _vector_layout(workspace, dtype_code)
            options = with_schedule_options(
                with_split_options(candidates, workspace.tile_count_for, workspace.max_k, workspace.sm_count,
                                   split_k, splittable),
                tile_schedule,
                lambda cfg: streamk_tail_for(workspace, cfg, dtype_code) > 0,
            )
            options = [(cfg, split, schedule, b_stream or 0) for cfg, split, schedule in options]
            # The B copy policy is timed on the finalists where it is not pinned and the LDS-DMA kernels run.
            twin = ((lambda o: (o[0], o[1], o[2], 1))
                    if b_stream is None and _vector_layout(workspace, dtype_code) else None)
            tuned = _tune(options, lambda o: _launch_grouped_fixed(workspace, o[0], dtype_code, precision, *o[1:]),
                          twin=twin)
            _GROUPED_AUTOTUNE_CACHE[key] = tuned
        cfg, split_k, schedule, stream_b = tuned
    else:
        schedule = tile_schedule or "static"
        stream_b = b_stream or 0
        if schedule in ("stealing", "streamk") and split_k is None:
            split_k = 1
    workspace.split_k = _launch_grouped_fixed(workspace, cfg, dtype_code, precision, split_k, schedule, stream_b)
    workspace.config = cfg
    workspace.scheduler = scheduler
    workspace.b_stream = stream_b
    if schedule == "streamk" and not streamk_tail_for(workspace, cfg, dtype_code):
        schedule = "static"
    workspace.tile_schedule = schedule


# ---------------------------------------------------------------------------------------------
# Packed Gate+Up with the SwiGLU activation fused into the epilogue (one launch).

def _swiglu_problem_ok(a, b, h) -> bool:
    m, k = a.shape
    n = b.shape[1]
    sam, sak = a.stride()
    sbk, sbn = b.stride()
    shm, shn = h.stride()
    return (
        sak == 1 and sbn == 1 and shn == 1 and n % 16 == 0 and tuple(h.shape) == (m, n // 2)
        and k % 8 == 0 and sam % 8 == 0 and sbk % 8 == 0 and shm % 4 == 0
        and sam >= k and sbk >= n and shm >= n // 2
        and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0 and h.data_ptr() % 8 == 0
        and _native.panels_fit(k, sam, sbk, shm)
    )


def _swiglu_outputs(workspace: GroupedWorkspace):
    import torch

    if workspace.h is None:
        device = workspace.a[0].device
        workspace.h = [torch.empty((m, n // 2), device=device, dtype=workspace.a[0].dtype)
                       for m, _, n in workspace.shapes]
        workspace.h_ptrs = torch.tensor([t.data_ptr() for t in workspace.h], device=device, dtype=torch.int64)
        rows = [(a.stride(0), a.stride(1), b.stride(0), b.stride(1), h.stride(0), h.stride(1))
                for a, b, h in zip(workspace.a, workspace.b, workspace.h)]
        workspace.h_strides = torch.tensor(rows, device=device, dtype=torch.int64)
    return workspace.h


def _launch_swiglu_fixed(workspace: GroupedWorkspace, cfg: KernelConfig, dtype_code: int, b_stream: int = 0) -> None:
    m, k, n = workspace.shapes[0]
    status = _native.library().moegemm_grouped_gemm_swiglu(
        workspace.a_ptrs.data_ptr(), workspace.b_ptrs.data_ptr(), workspace.h_ptrs.data_ptr(),
        workspace.dims.data_ptr(), workspace.h_strides.data_ptr(),
        workspace.problem_count, m, n, k, 1 if workspace.homogeneous else 0,
        workspace.tile_count_for(cfg), dtype_code,
        cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages,
        _grid_size(workspace, cfg), 1, b_stream, _native.current_stream_handle(workspace.a[0].device),
    )
    _native.check(status)


_SWIGLU_AUTOTUNE_CACHE: dict[tuple, tuple[KernelConfig, int]] = {}


def swiglu_candidate_configs(workspace: GroupedWorkspace) -> tuple[KernelConfig, ...]:
    """Grouped candidates restricted to tiles whose waves pair gate and up fragments."""
    dtype_code = _native.dtype_code(workspace.a[0].dtype)
    allowed = _native.swiglu_tiles(dtype_code)
    ranked = grouped_candidate_configs(workspace.max_m, workspace.max_n, workspace.max_k,
                                       problem_count=max(workspace.problem_count, 2),
                                       sm_count=workspace.sm_count, dtype=workspace.a[0].dtype)
    kept = tuple(c for c in ranked if c.tile_key in allowed)
    if kept:
        return kept
    pool = [c for c in config_pool(workspace.a[0].dtype) if c.tile_key in allowed and c.group_size_m == 8]
    return tuple(pool[:6])


def launch_gate_up_swiglu(
    workspace: GroupedWorkspace,
    config: KernelConfig | None = None,
    *,
    autotune: bool = True,
) -> list:
    """H_e = silu(A_e @ B_e[:, :F]) * (A_e @ B_e[:, F:]) for every problem, in one kernel launch.

    ``workspace`` holds packed Gate+Up weights (``build_fused_gate_up_workspace``): B_e has
    2F columns, [gate | up].  The outputs H_e [M_e, F] are allocated on the first call and kept
    in ``workspace.h``; the activation is computed from the fp32 accumulators, so H differs from
    silu applied to a rounded C by at most the output rounding.  fp16/bf16 operands in the vector
    layout only (ValueError otherwise).  Autotuning follows ``launch_grouped``: the first call per
    workload measures the candidates, later calls are a cache lookup plus one launch.
    """
    _require_runtime()
    dtype_code = _check_workspace(workspace)
    if dtype_code == _native.DTYPE_F32:
        raise ValueError("the fused SwiGLU epilogue needs fp16 or bf16 operands")
    outputs = _swiglu_outputs(workspace)
    if not all(_swiglu_problem_ok(a, b, h) for a, b, h in zip(workspace.a, workspace.b, outputs)):
        raise ValueError("the fused SwiGLU epilogue needs unit inner strides, 16-byte aligned rows, "
                         "K a multiple of 8 and a packed width N = 2F with F a multiple of 8")
    cfg = config or workspace.swiglu_config
    if autotune:
        key = ("swiglu", workspace.problem_count, workspace.max_m, workspace.max_n, workspace.max_k,
               workspace.shape_signature, workspace.device_signature, workspace.sm_count, dtype_code)
        tuned = _SWIGLU_AUTOTUNE_CACHE.get(key)
        if tuned is None:
            # The plain W13 GEMM of the same workload, if already tuned, gives the preferred tile and
            # B copy policy: the activation changes only the epilogue, so a different pick would be
            # timing noise.
            scheduler = "homogeneous_persistent" if workspace.homogeneous else "generic_persistent"
            plain = _GROUPED_AUTOTUNE_CACHE.get(_grouped_tuning_key(
                workspace, scheduler, dtype_code, _native.PRECISION_IEEE, None, None))
            allowed = _native.swiglu_tiles(dtype_code)
            prefer = (plain[0], plain[3]) if plain is not None and plain[0].tile_key in allowed else None
            candidates = [(c, 0) for c in swiglu_candidate_configs(workspace)]
            if prefer is not None and prefer not in candidates:
                candidates.append(prefer)
            tuned = _tune(candidates, lambda o: _launch_swiglu_fixed(workspace, o[0], dtype_code, o[1]),
                          prefer=prefer, twin=lambda o: (o[0], 1))
            _SWIGLU_AUTOTUNE_CACHE[key] = tuned
        cfg, stream_b = tuned
    else:
        cfg, stream_b = cfg or swiglu_candidate_configs(workspace)[0], 0
    _launch_swiglu_fixed(workspace, cfg, dtype_code, stream_b)
    workspace.swiglu_config = cfg
    workspace.swiglu_b_stream = stream_b
    workspace.scheduler = "homogeneous_persistent" if workspace.homogeneous else "generic_persistent"
    return outputs
