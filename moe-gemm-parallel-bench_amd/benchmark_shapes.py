"""Single-GEMM experiments: fixed-product shape sweep and the M x N efficiency heatmap.

Same experiments as the reference's benchmark_shapes.py: each (M, K, N) point builds seeded
``normal_() * 0.1`` operands (hot: one workspace, cold: a rotating ring), tunes ``launch_matmul``
(hot: per-shape autotune; cold: rotating-ring tuner), NaN-poisons C and relaunches the winner,
checks against a float32 torch product, times with graph-replay timing, and adds a ``torch.mm``
(hipBLASLt on ROCm) row timed the same way.  Rows use schema 1.3.

The heatmap also takes lists of K and of group sizes G (the reference's is G = 1 at one K,
``benchmark_shapes.py:321-335``).  A point with G > 1 runs G equal problems in one homogeneous
``launch_grouped`` call, checks every problem, and its baseline is the per-problem ``torch.mm``
loop timed the same way.
"""

from __future__ import annotations

import json
from typing import Any

from kernels.grouped_gemm import build_grouped_workspace, grouped_candidate_configs, launch_grouped
from kernels.matmul import last_matmul_config, launch_matmul, matmul_candidate_configs, select_config
from utils.benchmark import (
    TIMING_METHOD,
    assert_close,
    available_budget,
    dtype_size,
    time_cuda,
    torch_dtype,
    tune_rotating_configs,
)
from utils.io import write_rows
from utils.metrics import arithmetic_intensity, gemm_flops, tile_metrics


def _base(args, env: dict[str, Any], experiment: str) -> dict[str, Any]:
    return {
        "schema_version": "1.3",
        "timing_method": TIMING_METHOD,
        "run_id": args.run_id,
        "timestamp": args.timestamp,
        "gpu_name": env.get("gpu_name"),
        "cuda_version": env.get("cuda_version"),
        "torch_version": env.get("torch_version"),
        "triton_version": env.get("triton_version"),
        "dtype": args.dtype,
        "experiment": experiment,
        "projection": "",
        "mode": "single",
        "provider": "hip",
        "parallel_type": "",
        "parallel_size": args.parallel_size,
        "num_experts": args.num_experts,
        "topk": args.topk,
        "T": "",
        "num_gemms": 1,
        "active_gemms": 1,
        "correct": False,
        "cache_mode": args.cache_mode,
        "model_config": args.model_config,
        "model_type": args.model_defaults.model_type,
        "requested_warmup": args.warmup,
        "requested_repeat": args.repeat,
        "requested_parameters": json.dumps(args.requested_parameters, sort_keys=True),
        "effective_parameters": json.dumps(args.effective_parameters, sort_keys=True),
        "status": "error",
    }


def _config_fields(cfg) -> dict[str, Any]:
    return {"block_m": cfg.block_m, "block_n": cfg.block_n, "block_k": cfg.block_k,
            "group_size_m": cfg.group_size_m, "num_warps": cfg.num_warps, "num_stages": cfg.num_stages}


def _run_one(args, env, m: int, k: int, n: int, experiment: str) -> list[dict[str, Any]]:
    import torch

    dtype = torch_dtype(args.dtype)
    cfg = select_config(m, n, k, dtype)
    sm_count = int(env.get("sm_count") or 0)
    base = _base(args, env, experiment)
    base.update(M=m, K=k, N=n, total_flops=gemm_flops(m, k, n),
                arithmetic_intensity=arithmetic_intensity(m, k, n, dtype_size(args.dtype)),
                **_config_fields(cfg), **tile_metrics([(m, k, n)], cfg.block_m, cfg.block_n, cfg.block_k, sm_count),
                launches_per_iteration=1, autotune_enabled=True, autotune_status="not_run",
                config_source="heuristic_fallback")
    torch.cuda.empty_cache()
    budget = available_budget(args.memory_fraction)
    per_workspace = dtype_size(args.dtype) * (m * k + k * n + m * n)
    wanted = 1 if args.cache_mode == "hot" else max(2, args.cold_buffers)
    ring = min(wanted, max(1, budget // max(per_workspace, 1)))
    base.update(estimated_memory_bytes=per_workspace * ring, memory_budget_bytes=budget, workspace_count=ring,
                workspace_bytes=per_workspace * ring)
    if per_workspace > budget or (args.max_matrix_bytes and per_workspace > args.max_matrix_bytes):
        reason = "estimated memory exceeds budget" if per_workspace > budget else "shape exceeds --max-matrix-bytes"
        base.update(status="skipped", skip_reason=reason, error="")
        return [base]
    if args.cache_mode == "cold" and ring < 2:
        base.update(status="skipped", skip_reason="rotating-cold needs at least two resident workspaces", error="")
        return [base]
    workspaces: list[tuple[Any, Any, Any]] = []
    minimum = 2 if args.cache_mode == "cold" else 1
    while ring >= minimum:
        try:
            generator = torch.Generator(device="cuda").manual_seed(args.seed + m + n)
            workspaces = [
                (torch.empty((m, k), device="cuda", dtype=dtype).normal_(generator=generator).mul_(0.1),
                 torch.empty((k, n), device="cuda", dtype=dtype).normal_(generator=generator).mul_(0.1),
                 torch.empty((m, n), device="cuda", dtype=dtype))
                for _ in range(ring)
            ]
            break
        except torch.OutOfMemoryError:
            workspaces = []
            torch.cuda.empty_cache()
            ring -= 1
    if not workspaces:
        base.update(status="skipped", correct=False, error="", workspace_count=0, workspace_bytes=0,
                    skip_reason="device OOM while allocating the minimum resident workspace count")
        return [base]
    base.update(workspace_count=ring, workspace_bytes=sum(t.numel() * t.element_size() for w in workspaces for t in w))
    rows: list[dict[str, Any]] = []
    hot = args.cache_mode == "hot"
    try:
        tuning = None
        if not hot:
            tuning = tune_rotating_configs(
                matmul_candidate_configs(m, n, k, dtype=dtype, sm_count=sm_count or 256),
                lambda c, i: launch_matmul(*workspaces[i % ring], c, args.input_precision, autotune=False), ring)
            cfg = tuning.config
        for a, b, c in workspaces:
            launch_matmul(a, b, c, cfg, args.input_precision, autotune=hot)
        torch.cuda.synchronize()
        if hot:
            cfg = last_matmul_config(cfg)
        for a, b, c in workspaces:
            c.fill_(float("nan"))
            launch_matmul(a, b, c, cfg, args.input_precision, autotune=False)
        torch.cuda.synchronize()
        max_abs = max_rel = 0.0
        for a, b, c in workspaces:
            abs_err, rel_err = assert_close(c, torch.matmul(a.float(), b.float()).to(dtype), args.dtype)
            max_abs, max_rel = max(max_abs, abs_err), max(max_rel, rel_err)
        base.update(**_config_fields(cfg), autotune_status="selected",
                    config_source="shape_family_autotune" if hot else "cold_ring_autotune",
                    scheduler="single_problem_matmul",
                    **tile_metrics([(m, k, n)], cfg.block_m, cfg.block_n, cfg.block_k, sm_count))
        if tuning is not None:
            base.update(autotune_candidates_tested=tuning.candidates_tested,
                        autotune_candidates_failed=tuning.candidates_failed,
                        autotune_selection_ms=tuning.median_ms)
        timing = time_cuda(lambda i: launch_matmul(*workspaces[i % ring], cfg, args.input_precision, autotune=hot),
                           args.warmup, args.repeat, args.target_timing_ms, workspace_count=ring)
        tflops = gemm_flops(m, k, n) / (timing.median_ms * 1e9)
        hip_row = dict(base)
        hip_row.update(status="ok", error="", skip_reason="", correct=True, max_abs_error=max_abs,
                       max_rel_error=max_rel, latency_ms=timing.median_ms, latency_p20_ms=timing.p20_ms,
                       latency_p80_ms=timing.p80_ms, tflops=tflops,
                       peak_efficiency=tflops / args.peak_tflops if args.peak_tflops else "",
                       warmup=timing.warmup, repeat=timing.repeat)
        rows.append(hip_row)
        if args.torch_baseline:
            for a, b, c in workspaces:
                torch.mm(a, b, out=c)
            torch.cuda.synchronize()
            t_abs = t_rel = 0.0
            for a, b, c in workspaces:
                abs_err, rel_err = assert_close(c, torch.matmul(a.float(), b.float()).to(dtype), args.dtype)
                t_abs, t_rel = max(t_abs, abs_err), max(t_rel, rel_err)
            t_timing = time_cuda(lambda i: torch.mm(workspaces[i % ring][0], workspaces[i % ring][1],
                                                    out=workspaces[i % ring][2]),
                                 args.warmup, args.repeat, args.target_timing_ms, workspace_count=ring)
            t_tflops = gemm_flops(m, k, n) / (t_timing.median_ms * 1e9)
            torch_row = dict(hip_row)
            torch_row.update(provider="torch", latency_ms=t_timing.median_ms, latency_p20_ms=t_timing.p20_ms,
                             latency_p80_ms=t_timing.p80_ms, tflops=t_tflops, correct=True, max_abs_error=t_abs,
                             max_rel_error=t_rel, peak_efficiency=t_tflops / args.peak_tflops if args.peak_tflops else "",
                             block_m="", block_n="", block_k="", group_size_m="", num_warps="", num_stages="",
                             autotune_enabled=False, autotune_status="not_applicable", config_source="library",
                             scheduler="torch_mm", warmup=t_timing.warmup, repeat=t_timing.repeat)
            rows.append(torch_row)
    except AssertionError as exc:
        base.update(status="invalid", error=f"correctness failure: {exc}", skip_reason="", correct=False)
        rows.append(base)
    except torch.OutOfMemoryError as exc:
        base.update(status="skipped", error="", skip_reason=f"device OOM during correctness: {exc}", correct=False)
        rows.append(base)
    except RuntimeError as exc:
        base.update(status="error", error=repr(exc), skip_reason="", correct=False)
        rows.append(base)
    finally:
        workspaces.clear()
        torch.cuda.empty_cache()
    return rows


def _run_grouped_one(args, env, g: int, m: int, k: int, n: int) -> list[dict[str, Any]]:
    """One heatmap point with G equal problems (M, K, N): one homogeneous grouped launch per call."""
    import torch

    dtype = torch_dtype(args.dtype)
    shapes = [(m, k, n)] * g
    cfg = select_config(m, n, k, dtype)
    sm_count = int(env.get("sm_count") or 0)
    base = _base(args, env, "heatmap")
    base.update(M=m, K=k, N=n, mode="grouped", num_gemms=g, active_gemms=g, total_flops=g * gemm_flops(m, k, n),
                arithmetic_intensity=arithmetic_intensity(m, k, n, dtype_size(args.dtype)),
                **_config_fields(cfg), **tile_metrics(shapes, cfg.block_m, cfg.block_n, cfg.block_k, sm_count),
                launches_per_iteration=1, autotune_enabled=True, autotune_status="not_run",
                config_source="heuristic_fallback", output_preallocated=True)
    torch.cuda.empty_cache()
    budget = available_budget(args.memory_fraction)
    per_workspace = g * dtype_size(args.dtype) * (m * k + k * n + m * n)
    wanted = 1 if args.cache_mode == "hot" else max(2, args.cold_buffers)
    ring = min(wanted, max(1, budget // max(per_workspace, 1)))
    base.update(estimated_memory_bytes=per_workspace * ring, memory_budget_bytes=budget, workspace_count=ring,
                workspace_bytes=per_workspace * ring)
    if per_workspace > budget or (args.max_matrix_bytes and per_workspace // g > args.max_matrix_bytes):
        reason = "estimated memory exceeds budget" if per_workspace > budget else "shape exceeds --max-matrix-bytes"
        base.update(status="skipped", skip_reason=reason, error="")
        return [base]
    if args.cache_mode == "cold" and ring < 2:
        base.update(status="skipped", skip_reason="rotating-cold needs at least two resident workspaces", error="")
        return [base]
    workspaces = []
    minimum = 2 if args.cache_mode == "cold" else 1
    while ring >= minimum:
        try:
            workspaces = [build_grouped_workspace(shapes, dtype, args.seed + i * 100003, cfg) for i in range(ring)]
            break
        except torch.OutOfMemoryError:
            workspaces = []
            torch.cuda.empty_cache()
            ring -= 1
    if not workspaces:
        base.update(status="skipped", correct=False, error="", workspace_count=0, workspace_bytes=0,
                    skip_reason="device OOM while allocating the minimum resident workspace count")
        return [base]
    base.update(workspace_count=ring, workspace_bytes=sum(w.storage_bytes for w in workspaces))
    rows: list[dict[str, Any]] = []
    hot = args.cache_mode == "hot"
    try:
        tuning = None
        if not hot:
            candidates = grouped_candidate_configs(m, n, k, problem_count=g, sm_count=workspaces[0].sm_count,
                                                   dtype=dtype)
            tuning = tune_rotating_configs(
                candidates, lambda c, i: launch_grouped(workspaces[i % ring], args.input_precision, c,
                                                        autotune=False), ring)
            cfg = tuning.config
        for workspace in workspaces:
            launch_grouped(workspace, args.input_precision, cfg, autotune=hot)
        torch.cuda.synchronize()
        cfg = workspaces[0].config
        for workspace in workspaces:
            for output in workspace.c:
                output.fill_(float("nan"))
            launch_grouped(workspace, args.input_precision, cfg, autotune=False)
        torch.cuda.synchronize()
        max_abs = max_rel = 0.0
        for workspace in workspaces:
            for a, b, c in workspace.problem_tensors():
                abs_err, rel_err = assert_close(c, torch.matmul(a.float(), b.float()).to(dtype), args.dtype)
                max_abs, max_rel = max(max_abs, abs_err), max(max_rel, rel_err)
        base.update(**_config_fields(cfg), cta_multiplier=cfg.cta_multiplier, autotune_status="selected",
                    config_source="workload_autotune" if hot else "cold_ring_autotune",
                    scheduler=workspaces[0].scheduler,
                    **tile_metrics(shapes, cfg.block_m, cfg.block_n, cfg.block_k, sm_count))
        if tuning is not None:
            base.update(autotune_candidates_tested=tuning.candidates_tested,
                        autotune_candidates_failed=tuning.candidates_failed,
                        autotune_selection_ms=tuning.median_ms)
        timing = time_cuda(lambda i: launch_grouped(workspaces[i % ring], args.input_precision, cfg, autotune=False),
                           args.warmup, args.repeat, args.target_timing_ms, workspace_count=ring)
        tflops = base["total_flops"] / (timing.median_ms * 1e9)
        hip_row = dict(base)
        hip_row.update(status="ok", error="", skip_reason="", correct=True, max_abs_error=max_abs,
                       max_rel_error=max_rel, latency_ms=timing.median_ms, latency_p20_ms=timing.p20_ms,
                       latency_p80_ms=timing.p80_ms, tflops=tflops,
                       peak_efficiency=tflops / args.peak_tflops if args.peak_tflops else "",
                       warmup=timing.warmup, repeat=timing.repeat)
        rows.append(hip_row)
        if args.torch_baseline:
            def torch_loop(index: int) -> None:
                for a, b, c in workspaces[index % ring].problem_tensors():
                    torch.mm(a, b, out=c)

            for index in range(ring):
                torch_loop(index)
            torch.cuda.synchronize()
            t_abs = t_rel = 0.0
            for workspace in workspaces:
                for a, b, c in workspace.problem_tensors():
                    abs_err, rel_err = assert_close(c, torch.matmul(a.float(), b.float()).to(dtype), args.dtype)
                    t_abs, t_rel = max(t_abs, abs_err), max(t_rel, rel_err)
            t_timing = time_cuda(torch_loop, args.warmup, args.repeat, args.target_timing_ms, workspace_count=ring)
            t_tflops = base["total_flops"] / (t_timing.median_ms * 1e9)
            torch_row = dict(hip_row)
            torch_row.update(provider="torch", latency_ms=t_timing.median_ms, latency_p20_ms=t_timing.p20_ms,
                             latency_p80_ms=t_timing.p80_ms, tflops=t_tflops, correct=True, max_abs_error=t_abs,
                             max_rel_error=t_rel, peak_efficiency=t_tflops / args.peak_tflops if args.peak_tflops else "",
                             block_m="", block_n="", block_k="", group_size_m="", num_warps="", num_stages="",
                             cta_multiplier="", autotune_enabled=False, autotune_status="not_applicable",
                             config_source="library", scheduler="torch_mm_loop", launches_per_iteration=g,
                             warmup=t_timing.warmup, repeat=t_timing.repeat)
            rows.append(torch_row)
    except AssertionError as exc:
        base.update(status="invalid", error=f"correctness failure: {exc}", skip_reason="", correct=False)
        rows.append(base)
    except torch.OutOfMemoryError as exc:
        base.update(status="skipped", error="", skip_reason=f"device OOM during correctness: {exc}", correct=False)
        rows.append(base)
    except RuntimeError as exc:
        base.update(status="error", error=repr(exc), skip_reason="", correct=False)
        rows.append(base)
    finally:
        workspaces.clear()
        torch.cuda.empty_cache()
    return rows


def _finish(rows: list[dict[str, Any]], path) -> list[dict[str, Any]]:
    hip_ok = [r for r in rows if r.get("status") == "ok" and r.get("provider") == "hip"]
    best = max((float(r["tflops"]) for r in hip_ok), default=0.0)
    for row in rows:
        if row.get("status") == "ok" and best:
            row["normalized_efficiency"] = float(row["tflops"]) / best
    _annotate_best_measured(rows)
    write_rows(path, rows)
    return rows


def run_shape_sweep(args, env: dict[str, Any]) -> list[dict[str, Any]]:
    ms = args.shape_ms or [8192, 4096, 2048, 1024, 512, 256, 128, 64, 32, 16]
    rows: list[dict[str, Any]] = []
    for m in ms:
        if args.shape_product % m:
            row = _base(args, env, "shapes")
            row.update(M=m, K=args.shape_k, N="", status="skipped", skip_reason="M does not divide shape product")
            rows.append(row)
            continue
        rows.extend(_run_one(args, env, m, args.shape_k, args.shape_product // m, "shapes"))
    return _finish(rows, args.results_dir / "gemm_shape_sweep.csv")


def run_heatmap(args, env: dict[str, Any]) -> list[dict[str, Any]]:
    ms = args.heatmap_ms or [1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024]
    ns = args.heatmap_ns or [256, 512, 1024, 2048, 4096, 8192, 14336]
    ks = getattr(args, "heatmap_ks", None) or [args.heatmap_k]
    gs = getattr(args, "heatmap_gs", None) or [1]
    rows: list[dict[str, Any]] = []
    for g in gs:
        for k in ks:
            for m in ms:
                for n in ns:
                    point = (_run_one(args, env, m, k, n, "heatmap") if g == 1
                             else _run_grouped_one(args, env, g, m, k, n))
                    rows.extend(point)
                    summary = ", ".join(f"{r.get('provider', 'hip')} {r.get('status')}"
                                        + (f" {float(r['tflops']):.1f} TFLOP/s" if r.get("status") == "ok" else "")
                                        for r in point)
                    print(f"heatmap G={g} M={m} K={k} N={n}: {summary}", flush=True)
    return _finish(rows, args.results_dir / "gemm_heatmap.csv")


def _annotate_best_measured(rows: list[dict[str, Any]], threshold: float = 0.90) -> None:
    """Ratio of each ok row to the best provider on the same exact (G, M, K, N)."""
    best: dict[tuple[int, int, int, int], float] = {}
    ok = [r for r in rows if r.get("status") == "ok"]
    for row in ok:
        key = (int(row.get("num_gemms") or 1), int(row["M"]), int(row["K"]), int(row["N"]))
        best[key] = max(best.get(key, 0.0), float(row["tflops"]))
    for row in ok:
        key = (int(row.get("num_gemms") or 1), int(row["M"]), int(row["K"]), int(row["N"]))
        ratio = float(row["tflops"]) / best[key]
        row.update(best_measured_tflops=best[key], best_measured_ratio=ratio, near_best_threshold=threshold,
                   near_best=ratio >= threshold)
