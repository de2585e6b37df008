"""Per-rank EP versus TP MoE expert GEMMs at equal useful FLOPs (uniform top-k routing, no router).

Same experiment as the reference's benchmark_moe.py: for W1 (packed Gate+Up) and W2 (Down), each
tokens-per-expert M_e, each mode (``grouped`` = this project's HIP kernel over per-expert pointer
tables, ``offsets`` = the same kernel over the expert-sorted 2-D A / 3-D B / int32 offsets layout
(opt-in, ``--offsets-layout``), ``torch`` = one verified ``torch.nn.functional.grouped_mm`` call)
and each parallel type, the case
  1. checks exact EP/TP FLOP equality and builds the per-rank shapes (utils/metrics.py);
  2. admits the case against the memory budget and sizes the hot (1) or rotating-cold ring;
  3. tunes (hot: autotuned launcher; cold: rotating-ring tuner over fixed candidates);
  4. gates correctness on every ring workspace: NaN-poison C, launch the winner alone, compare
     per expert with a float32-accumulated torch product (W1 as cat(A@B_gate, A@B_up));
  5. times the call with graph-replay timing and writes one CSV row (schema 1.4).
Exceptions map to row status: AssertionError -> invalid, TorchGroupedMMUnavailable/OOM -> skipped,
RuntimeError -> error.
"""

from __future__ import annotations

import json
from typing import Any

from kernels.grouped_gemm import (
    build_fused_gate_up_workspace,
    build_grouped_workspace,
    grouped_candidate_configs,
    launch_grouped,
)
from kernels.grouped_mm import build_offsets_workspace, launch_grouped_offsets
from kernels.matmul import select_config
from kernels.torch_grouped_gemm import (
    TorchGroupedMMUnavailable,
    build_torch_grouped_workspace,
    launch_torch_grouped,
    torch_grouped_mm_unavailable_reason,
    verify_torch_grouped_execution,
)
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
from utils.metrics import arithmetic_intensity, moe_shapes, tile_metrics, verify_ep_tp_flops

_TABLE_BYTES_PER_PROBLEM = 3 * 8 + 3 * 4 + 6 * 8  # pointer tables, dims, strides


def _estimate(shapes: list[tuple[int, int, int]], item_size: int, mode: str) -> int:
    """Bytes one workspace of this case needs (torch and offsets modes pad row strides to 16 bytes)."""
    if mode in ("torch", "offsets"):
        step = max(1, 16 // item_size)
        pad = lambda v: -(-v // step) * step  # noqa: E731
        return sum(item_size * (m * pad(k) + k * pad(n) + m * pad(n)) for m, k, n in shapes) + 4 * len(shapes)
    return sum(item_size * (m * k + k * n + m * n) for m, k, n in shapes) + _TABLE_BYTES_PER_PROBLEM * len(shapes)


def _base(args, env, projection: str, parallel_type: str, mode: str, m: int, shape, count: int, total: int):
    _, k, n = shape
    cfg = select_config(m, n, k, args.dtype)
    torch_mode = mode == "torch"
    row: dict[str, Any] = {
        "schema_version": "1.4",
        "timing_method": TIMING_METHOD,
        "run_id": args.run_id,
        "timestamp": args.timestamp,
        "gpu_name": env.get("gpu_name"),
        "cuda_version": env.get("cuda_version"),
        "torch_version": env.get("torch_version"),
        "triton_version": env.get("triton_version"),
        "dtype": args.dtype,
        "experiment": "moe",
        "projection": projection,
        "operation": "gate_up" if projection == "W1" else "down",
        "fused_projections": 2 if projection == "W1" else 1,
        "output_layout": "gate_then_up" if projection == "W1" else "down",
        "activation_in_timed_region": False,
        "mode": mode,
        "provider": "torch" if torch_mode else "hip",
        "parallel_type": parallel_type,
        "parallel_size": args.parallel_size,
        "num_experts": args.num_experts,
        "topk": args.topk,
        "T": m * args.num_experts // args.topk,
        "M": m,
        "K": k,
        "N": n,
        "num_gemms": count,
        "active_gemms": count,
        "total_flops": total,
        "arithmetic_intensity": arithmetic_intensity(m, k, n, dtype_size(args.dtype)),
        "correct": False,
        "cache_mode": args.cache_mode,
        "tokens_per_expert": m,
        "weight_shard_factor": 1 if parallel_type == "EP" else args.parallel_size,
        "flops_equal": True,
        **tile_metrics([shape] * count, cfg.block_m, cfg.block_n, cfg.block_k, int(env.get("sm_count") or 0)),
        "api_calls_per_iteration": 1,
        "launches_per_iteration": "" if torch_mode else 1,
        "grouped_compute_launches": "" if torch_mode else 1,
        "execution_verified": not torch_mode,
        "output_preallocated": not torch_mode,
        "autotune_enabled": not torch_mode,
        "autotune_status": "not_applicable" if torch_mode else "not_run",
        "config_source": "library" if torch_mode else "heuristic_fallback",
        "requested_warmup": args.warmup,
        "requested_repeat": args.repeat,
        "model_config": args.model_config,
        "model_type": args.model_defaults.model_type,
        "requested_parameters": json.dumps(args.requested_parameters, sort_keys=True),
        "effective_parameters": json.dumps(args.effective_parameters, sort_keys=True),
        "status": "error",
    }
    if not torch_mode:
        row.update(block_m=cfg.block_m, block_n=cfg.block_n, block_k=cfg.block_k, group_size_m=cfg.group_size_m,
                   num_warps=cfg.num_warps, num_stages=cfg.num_stages)
    return row


def _build_ring(args, shapes, projection: str, mode: str, ring: int, minimum: int):
    """Build ``ring`` workspaces, shrinking the ring (never the shapes) on allocator OOM."""
    import torch

    dtype = torch_dtype(args.dtype)
    cfg = select_config(shapes[0][0], shapes[0][2], shapes[0][1], dtype)
    while ring >= minimum:
        try:
            operation = "gate_up" if projection == "W1" else "down"
            if mode == "torch":
                return [build_torch_grouped_workspace(shapes, dtype, args.seed + i * 100003, operation=operation)
                        for i in range(ring)], ring
            if mode == "offsets":
                return [build_offsets_workspace(shapes, dtype, args.seed + i * 100003, operation=operation)
                        for i in range(ring)], ring
            builder = build_fused_gate_up_workspace if projection == "W1" else build_grouped_workspace
            return [builder(shapes, dtype, args.seed + i * 100003, cfg) for i in range(ring)], ring
        except torch.OutOfMemoryError:
            torch.cuda.empty_cache()
            ring -= 1
    return [], 0


def _reference(a, b, projection: str):
    import torch

    if projection == "W1":
        half = b.shape[1] // 2
        return torch.cat((torch.matmul(a.float(), b[:, :half].float()),
                          torch.matmul(a.float(), b[:, half:].float())), dim=1).to(a.dtype)
    return torch.matmul(a.float(), b.float()).to(a.dtype)


def _launch_hip(workspace, mode: str, precision: str, cfg, autotune: bool) -> None:
    if mode == "offsets":
        launch_grouped_offsets(workspace, precision, cfg, autotune=autotune)
    else:
        launch_grouped(workspace, precision, cfg, autotune=autotune)


def _outputs(workspace, mode: str):
    return [workspace.output] if mode == "offsets" else workspace.c


def _run_case(args, env: dict[str, Any], projection: str, parallel_type: str, mode: str, m: int) -> dict[str, Any]:
    import torch

    total = verify_ep_tp_flops(projection, m, args.hidden_size, args.ffn_size, args.num_experts, args.parallel_size)
    shapes = moe_shapes(projection, parallel_type, m, args.hidden_size, args.ffn_size, args.num_experts,
                        args.parallel_size)
    row = _base(args, env, projection, parallel_type, mode, m, shapes[0], len(shapes), total)
    if mode == "torch":
        reason = torch_grouped_mm_unavailable_reason(torch_dtype(args.dtype), len(shapes))
        if reason:
            row.update(status="skipped", skip_reason=reason, error="")
            return row
    torch.cuda.empty_cache()
    budget = available_budget(args.memory_fraction)
    per_workspace = _estimate(shapes, dtype_size(args.dtype), mode)
    wanted = 1 if args.cache_mode == "hot" else max(2, args.cold_buffers)
    ring = min(wanted, budget // max(per_workspace, 1))
    row.update(estimated_memory_bytes=per_workspace * max(ring, 1), memory_budget_bytes=budget,
               workspace_count=ring, workspace_bytes=per_workspace * max(ring, 1))
    if per_workspace > budget:
        row.update(status="skipped", skip_reason="estimated one-workspace memory exceeds budget", error="")
        return row
    minimum = 2 if args.cache_mode == "cold" else 1
    if ring < minimum:
        row.update(status="skipped", skip_reason="rotating-cold needs at least two resident workspaces", error="")
        return row
    workspaces, ring = _build_ring(args, shapes, projection, mode, ring, minimum)
    if not workspaces:
        row.update(status="skipped", correct=False, error="", workspace_count=0, workspace_bytes=0,
                   skip_reason="device OOM while allocating the minimum resident workspace count")
        return row
    row.update(workspace_count=ring, workspace_bytes=sum(w.storage_bytes for w in workspaces),
               estimated_memory_bytes=per_workspace * ring)
    try:
        cfg = select_config(m, shapes[0][2], shapes[0][1], torch_dtype(args.dtype))
        tuning = None
        if mode == "torch":
            row.update(verify_torch_grouped_execution(workspaces[0]))
        elif args.cache_mode == "cold":
            candidates = grouped_candidate_configs(
                max(s[0] for s in shapes), max(s[2] for s in shapes), max(s[1] for s in shapes),
                problem_count=len(shapes), sm_count=workspaces[0].sm_count, dtype=torch_dtype(args.dtype))
            tuning = tune_rotating_configs(
                candidates, lambda c, i: _launch_hip(workspaces[i % ring], mode, args.input_precision, c, False),
                ring)
            cfg = tuning.config
        hot = args.cache_mode == "hot"
        for workspace in workspaces:
            if mode == "torch":
                launch_torch_grouped(workspace)
            else:
                _launch_hip(workspace, mode, args.input_precision, cfg, hot)
        torch.cuda.synchronize()
        if mode != "torch":
            # Tuning wrote C with several candidates: poison it and run the winner alone.
            for workspace in workspaces:
                for output in _outputs(workspace, mode):
                    output.fill_(float("nan"))
                _launch_hip(workspace, mode, args.input_precision, workspace.config, False)
            torch.cuda.synchronize()
        max_abs = max_rel = 0.0
        for workspace in workspaces:
            for a, b, c in workspace.problem_tensors():
                abs_err, rel_err = assert_close(c, _reference(a, b, projection), args.dtype)
                max_abs, max_rel = max(max_abs, abs_err), max(max_rel, rel_err)
        row["workspace_bytes"] = sum(w.storage_bytes for w in workspaces)
        if mode != "torch":
            cfg = workspaces[0].config
            row.update(
                block_m=cfg.block_m, block_n=cfg.block_n, block_k=cfg.block_k, group_size_m=cfg.group_size_m,
                num_warps=cfg.num_warps, num_stages=cfg.num_stages, cta_multiplier=cfg.cta_multiplier,
                autotune_status="selected", scheduler=workspaces[0].scheduler,
                config_source="cold_ring_autotune" if args.cache_mode == "cold" else "workload_autotune",
                **tile_metrics(shapes, cfg.block_m, cfg.block_n, cfg.block_k, int(env.get("sm_count") or 0)),
            )
            if tuning is not None:
                row.update(autotune_candidates_tested=tuning.candidates_tested,
                           autotune_candidates_failed=tuning.candidates_failed,
                           autotune_selection_ms=tuning.median_ms)
        else:
            row["scheduler"] = workspaces[0].scheduler

        def invoke(index: int) -> None:
            current = workspaces[index % ring]
            if mode == "torch":
                launch_torch_grouped(current)
            else:
                _launch_hip(current, mode, args.input_precision, cfg, hot)

        timing = time_cuda(invoke, args.warmup, args.repeat, args.target_timing_ms, workspace_count=ring)
        tflops = total / (timing.median_ms * 1e9)
        row.update(status="ok", skip_reason="", error="", correct=True, max_abs_error=max_abs,
                   max_rel_error=max_rel, latency_ms=timing.median_ms, latency_p20_ms=timing.p20_ms,
                   latency_p80_ms=timing.p80_ms, tflops=tflops,
                   peak_efficiency=tflops / args.peak_tflops if args.peak_tflops else "",
                   warmup=timing.warmup, repeat=timing.repeat)
    except AssertionError as exc:
        row.update(status="invalid", correct=False, error=f"correctness failure: {exc}", skip_reason="")
        print(f"INVALID {projection} {parallel_type} {mode} M={m}: {exc}")
    except TorchGroupedMMUnavailable as exc:
        row.update(status="skipped", correct=False, error="", skip_reason=str(exc))
        print(f"SKIP {projection} {parallel_type} {mode} M={m}: {exc}")
    except torch.OutOfMemoryError as exc:
        row.update(status="skipped", correct=False, error="", skip_reason=f"device OOM during correctness: {exc}")
        print(f"SKIP {projection} {parallel_type} {mode} M={m}: device OOM")
    except RuntimeError as exc:
        row.update(status="error", correct=False, error=repr(exc), skip_reason="")
        print(f"ERROR {projection} {parallel_type} {mode} M={m}: {exc}")
    finally:
        workspaces.clear()
        torch.cuda.empty_cache()
    return row


def run_moe(args, env: dict[str, Any]) -> dict[str, list[dict[str, Any]]]:
    if args.num_experts % args.parallel_size:
        raise ValueError("num_experts must be divisible by parallel_size")
    if args.ffn_size % args.parallel_size:
        raise ValueError("ffn_size must be divisible by parallel_size")
    ms = args.moe_ms or [1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024]
    if args.tokens is not None:
        assignments = args.tokens * args.topk
        if assignments % args.num_experts:
            raise ValueError("tokens * topk must be divisible by num_experts")
        ms = [assignments // args.num_experts]
    if any(m <= 0 for m in ms):
        raise ValueError("all tokens-per-expert M values must be positive")
    nonintegral = [m for m in ms if (m * args.num_experts) % args.topk]
    if nonintegral:
        raise ValueError("M*num_experts must be divisible by topk so T is integral; invalid M values: "
                         + ",".join(map(str, nonintegral)))
    modes = (["grouped"] + (["offsets"] if getattr(args, "offsets_layout", False) else [])
             + (["torch"] if args.torch_baseline else []))
    outputs: dict[str, list[dict[str, Any]]] = {"W1": [], "W2": []}
    for projection in ("W1", "W2"):
        for m in ms:
            for mode in modes:
                for parallel_type in ("EP", "TP"):
                    outputs[projection].append(_run_case(args, env, projection, parallel_type, mode, m))
        ok = [r for r in outputs[projection] if r.get("status") == "ok"]
        best = max((float(r["tflops"]) for r in ok), default=0.0)
        for row in ok:
            if best:
                row["normalized_efficiency"] = float(row["tflops"]) / best
        _annotate_best_measured(outputs[projection])
        write_rows(args.results_dir / f"moe_{projection.lower()}.csv", outputs[projection])
    return outputs


def _annotate_best_measured(rows: list[dict[str, Any]], threshold: float = 0.90) -> None:
    """Ratio of each ok row to the best provider at the same (M, parallel type)."""
    best: dict[tuple[int, str], float] = {}
    ok = [r for r in rows if r.get("status") == "ok"]
    for row in ok:
        key = (int(row["M"]), str(row["parallel_type"]))
        best[key] = max(best.get(key, 0.0), float(row["tflops"]))
    for row in ok:
        key = (int(row["M"]), str(row["parallel_type"]))
        ratio = float(row["tflops"]) / best[key]
        row.update(best_measured_tflops=best[key], best_measured_ratio=ratio, near_best_threshold=threshold,
                   near_best=ratio >= threshold)
