"""CSV rows of the result files (column set: ``utils.io.CSV_FIELDS``, the result wire format).

A row starts from ``base_row`` (run provenance + workload labels + the heuristic tile metrics),
gets the provider's execution facts from its ``Selection``, and the measurement from
``measured_row``; files are finished by ``annotate`` (efficiency relative to the best row).
Column semantics that the result contract checks are listed in the harness validator.
"""

from __future__ import annotations

import json

from kernels.matmul import select_config
from utils.benchmark import TIMING_METHOD, dtype_size
from utils.metrics import arithmetic_intensity, tile_metrics

SCHEMA_MOE = "1.4"
SCHEMA_SINGLE = "1.3"
_TILE_FIELDS = ("block_m", "block_n", "block_k", "group_size_m", "num_warps", "num_stages")


def config_columns(config) -> dict:
    """Tile columns of a KernelConfig, or empty cells for library providers."""
    if config is None:
        return {name: "" for name in (*_TILE_FIELDS, "cta_multiplier")}
    return {name: getattr(config, name) for name in (*_TILE_FIELDS, "cta_multiplier")}


def base_row(case, provider, settings, env) -> dict:
    """Provenance and workload columns of one (case, provider) row; status "error" until measured."""
    operation, fused, layout = case.projection_labels
    heuristic = select_config(case.m, max(case.n, 1), case.k, settings.torch_dtype)
    row = {
        "schema_version": SCHEMA_MOE if case.experiment == "moe" else SCHEMA_SINGLE,
        "run_id": settings.run_id,
        "timestamp": settings.timestamp,
        "gpu_name": env.get("gpu_name"),
        "cuda_version": env.get("cuda_version"),
        "torch_version": env.get("torch_version"),
        "triton_version": env.get("triton_version"),
        "dtype": settings.dtype,
        "experiment": case.experiment,
        "projection": case.projection,
        "operation": operation,
        "fused_projections": fused,
        "output_layout": layout,
        "activation_in_timed_region": False if case.projection else "",
        "mode": provider.mode_for(case),
        "provider": provider.name,
        "parallel_type": case.parallel_type,
        "parallel_size": settings.parallel_size,
        "num_experts": settings.num_experts,
        "topk": settings.topk,
        "T": case.tokens if case.tokens is not None else "",
        "M": case.m,
        "K": case.k,
        "N": case.n,
        "num_gemms": case.problem_count,
        "active_gemms": case.problem_count,
        "total_flops": case.total_flops,
        "timing_method": TIMING_METHOD,
        "arithmetic_intensity": arithmetic_intensity(case.m, case.k, case.n, dtype_size(settings.dtype))
        if case.n else "",
        "correct": False,
        "cache_mode": settings.cache_mode,
        "tokens_per_expert": case.m if case.experiment == "moe" else "",
        "weight_shard_factor": (1 if case.parallel_type == "EP" else settings.parallel_size)
        if case.experiment == "moe" else "",
        "flops_equal": True if case.experiment == "moe" else "",
        "requested_warmup": settings.warmup,
        "requested_repeat": settings.repeat,
        "model_config": settings.model_config,
        "model_type": settings.model.model_type,
        "requested_parameters": json.dumps(settings.requested_parameters, sort_keys=True),
        "effective_parameters": json.dumps(settings.effective_parameters, sort_keys=True),
        "status": "error",
        **provider.static_columns(case),
    }
    if case.n:
        row.update(tile_metrics(case.shapes, heuristic.block_m, heuristic.block_n, heuristic.block_k,
                                int(env.get("sm_count") or 0)))
    if provider.tiled:
        row.update(config_columns(heuristic), config_source="heuristic_fallback", autotune_status="not_run")
    return row


def selected_row(row: dict, case, selection, env) -> dict:
    """The provider's execution facts, and tile metrics of the config that actually ran."""
    row.update(selection.columns)
    if selection.config is not None:
        cfg = selection.config
        row.update(config_columns(cfg))
        row.update(tile_metrics(case.shapes, cfg.block_m, cfg.block_n, cfg.block_k, int(env.get("sm_count") or 0)))
    return row


def measured_row(row: dict, case, timing, errors: tuple[float, float], settings) -> dict:
    tflops = case.total_flops / (timing.median_ms * 1e9)
    row.update(
        status="ok", skip_reason="", error="", correct=True,
        max_abs_error=errors[0], max_rel_error=errors[1],
        latency_ms=timing.median_ms, latency_p20_ms=timing.p20_ms, latency_p80_ms=timing.p80_ms,
        tflops=tflops, peak_efficiency=tflops / settings.peak_tflops if settings.peak_tflops else "",
        warmup=timing.warmup, repeat=timing.repeat,
    )
    return row


def outcome_row(row: dict, status: str, reason: str) -> dict:
    """A row that ends without a measurement: skipped (reason) or invalid / error (error text)."""
    row.update(status=status, correct=False,
               skip_reason=reason if status == "skipped" else "",
               error=reason if status in ("invalid", "error") else "")
    return row


def annotate(rows: list[dict], experiment: str, threshold: float = 0.90) -> None:
    """normalized_efficiency against the best row of the file, and the near-best columns.

    For MoE files every ok row competes for "best" and near-best compares providers at equal
    (M, parallel type); for single-GEMM files "best" is the best HIP row and near-best compares
    providers at the same (G, M, K, N).
    """
    ok = [r for r in rows if r.get("status") == "ok"]
    if experiment == "moe":
        pool = ok
        key = lambda r: (int(r["M"]), r["parallel_type"])  # noqa: E731
    else:
        pool = [r for r in ok if r.get("provider") == "hip"]
        key = lambda r: (int(r["num_gemms"]), int(r["M"]), int(r["K"]), int(r["N"]))  # noqa: E731
    best_file = max((float(r["tflops"]) for r in pool), default=0.0)
    best_at: dict = {}
    for row in ok:
        best_at[key(row)] = max(best_at.get(key(row), 0.0), float(row["tflops"]))
    for row in ok:
        if best_file:
            row["normalized_efficiency"] = float(row["tflops"]) / best_file
        ratio = float(row["tflops"]) / best_at[key(row)]
        row.update(best_measured_tflops=best_at[key(row)], best_measured_ratio=ratio,
                   near_best_threshold=threshold, near_best=ratio >= threshold)
