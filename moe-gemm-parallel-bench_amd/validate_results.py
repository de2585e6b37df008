"""Offline validation of persisted benchmark CSVs (and plot artifacts when plots were requested).

Applies the reference's validation contract (validate_results.py:46-248 of the reference):
  * every ``ok`` row has positive finite latency/FLOPs/TFLOP/s, ``correct`` set, and FLOPs and
    TFLOP/s that recompute exactly from M, K, N, num_gemms and the latency;
  * MoE rows keep the W13 Gate+Up / W2 Down semantics and EP/TP FLOP equality;
  * grouped MoE rows prove one tuned kernel launch per iteration on a named persistent scheduler
    with positive tile parameters; torch rows prove one verified grouped_mm compute launch;
  * invalid/error rows or a missing file for a selected experiment make the run invalid.
Writes ``validation.json`` next to the CSVs and returns the report.
"""

from __future__ import annotations

import argparse
import csv
import json
import math
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

SCHEDULERS = {"homogeneous_persistent", "generic_persistent", "single_problem_matmul"}
OFFSETS_SCHEDULER = "offsets_persistent"  # the HIP kernel over the expert-sorted (offsets) layout
EXPERIMENT_FILES = {
    "shapes": ["gemm_shape_sweep.csv"],
    "moe": ["moe_w1.csv", "moe_w2.csv"],
    "heatmap": ["gemm_heatmap.csv"],
}
PLOTS_PER_FILE = {"gemm_shape_sweep.csv": 3, "moe_w1.csv": 3, "moe_w2.csv": 3, "gemm_heatmap.csv": 2}
MOE_FILES = {"moe_w1.csv", "moe_w2.csv"}


def _rows_for_run(path: Path, run_id: str) -> list[dict[str, str]]:
    if not path.exists():
        return []
    with path.open(newline="", encoding="utf-8") as handle:
        rows = list(csv.DictReader(handle))
    return [row for row in rows if not run_id or row.get("run_id") == run_id]


def _truthy(value: str | None) -> bool:
    return str(value or "").strip().lower() in {"1", "true", "yes"}


def _falsey(value: str | None) -> bool:
    return str(value or "").strip().lower() in {"0", "false", "no"}


def _finite_positive(value: str | None) -> bool:
    try:
        number = float(value)
    except (TypeError, ValueError, OverflowError):
        return False
    return math.isfinite(number) and number > 0.0


def _positive_integer(value: str | None) -> bool:
    try:
        number = float(value)
    except (TypeError, ValueError, OverflowError):
        return False
    return math.isfinite(number) and number > 0 and number == int(number)


def _moe_execution_contract_valid(row: dict[str, str]) -> bool:
    mode = row.get("mode")
    if mode == "torch":
        return (
            row.get("scheduler") == "torch_grouped_mm"
            and row.get("api_calls_per_iteration") == "1"
            and row.get("grouped_compute_launches") == "1"
            and _positive_integer(row.get("launches_per_iteration"))
            and _truthy(row.get("execution_verified"))
            and _falsey(row.get("output_preallocated"))
        )
    if mode not in ("grouped", "offsets"):
        return False
    schedulers = SCHEDULERS if mode == "grouped" else {OFFSETS_SCHEDULER}
    tile_fields = ("block_m", "block_n", "block_k", "num_warps", "num_stages", "cta_multiplier")
    return (
        _truthy(row.get("autotune_enabled"))
        and row.get("autotune_status") == "selected"
        and row.get("config_source") in {"workload_autotune", "cold_ring_autotune"}
        and row.get("scheduler") in schedulers
        and row.get("launches_per_iteration") == "1"
        and _truthy(row.get("output_preallocated"))
        and all(_positive_integer(row.get(field)) for field in tile_fields)
    )


def _derivable_metrics_valid(row: dict[str, str]) -> bool:
    try:
        m, k, n = (int(float(row[key])) for key in ("M", "K", "N"))
        gemms = int(float(row.get("num_gemms", "1")))
        total = float(row["total_flops"])
        latency_ms = float(row["latency_ms"])
        tflops = float(row["tflops"])
    except (KeyError, TypeError, ValueError):
        return False
    if min(m, k, n, gemms) <= 0 or latency_ms <= 0:
        return False
    expected_flops = 2 * m * k * n * gemms
    expected_tflops = expected_flops / (latency_ms * 1e9)
    return (math.isclose(total, expected_flops, rel_tol=1e-12, abs_tol=0.5)
            and math.isclose(tflops, expected_tflops, rel_tol=1e-6, abs_tol=1e-12))


def _projection_contract_valid(row: dict[str, str], filename: str) -> bool:
    expected = {
        "moe_w1.csv": ("W1", "gate_up", "2", "gate_then_up"),
        "moe_w2.csv": ("W2", "down", "1", "down"),
    }.get(filename)
    if expected is None:
        return True
    projection, operation, fused, layout = expected
    return (row.get("projection") == projection and row.get("operation") == operation
            and row.get("fused_projections") == fused and row.get("output_layout") == layout
            and _falsey(row.get("activation_in_timed_region")))


def _matched_moe_flops_equal(rows: list[dict[str, str]]) -> bool:
    keys = ("M", "mode", "provider", "cache_mode", "dtype", "parallel_size", "num_experts", "topk", "T")
    totals: dict[tuple[str, ...], dict[str, int]] = {}
    try:
        for row in rows:
            if row.get("status") == "ok":
                totals.setdefault(tuple(row.get(key, "") for key in keys), {})[row["parallel_type"]] = int(
                    float(row["total_flops"]))
    except (KeyError, TypeError, ValueError):
        return False
    return all(pair["EP"] == pair["TP"] for pair in totals.values() if {"EP", "TP"} <= set(pair))


def validate_results(results_dir: str | Path = "results", plots_dir: str | Path = "plots") -> dict[str, Any]:
    results, plots = Path(results_dir), Path(plots_dir)
    env_path = results / "environment.json"
    environment = json.loads(env_path.read_text(encoding="utf-8")) if env_path.exists() else {}
    run_id = str(environment.get("run_id") or "")
    requested = environment.get("requested_parameters") or {}
    plots_requested = not bool(requested.get("no_plots", False))
    experiment = str(requested.get("experiment") or "all")
    selected = set(EXPERIMENT_FILES) if experiment == "all" else {experiment}
    report: dict[str, Any] = {
        "timestamp": datetime.now(timezone.utc).isoformat(),
        "run_id": run_id,
        "selected_experiments": sorted(selected),
        "environment_present": env_path.exists(),
        "files": {},
        "plots": {},
        "issues": [],
    }
    if not run_id:
        report["issues"].append("environment.json has no run_id")
    ok_files: set[str] = set()
    for group in sorted(selected):
        for filename in EXPERIMENT_FILES[group]:
            rows = _rows_for_run(results / filename, run_id)
            ok = [r for r in rows if r.get("status") == "ok"]
            bad = [r for r in rows if r.get("status") in {"invalid", "error"}]
            moe = filename in MOE_FILES
            checks = {
                "all_correct": all(_truthy(r.get("correct")) for r in ok),
                "positive_finite_metrics": all(
                    all(_finite_positive(r.get(f)) for f in ("latency_ms", "total_flops", "tflops")) for r in ok),
                "derivable_metrics_recomputed": all(_derivable_metrics_valid(r) for r in ok),
                "projection_contract": all(_projection_contract_valid(r, filename) for r in ok),
                "flops_equal": (not moe) or (all(_truthy(r.get("flops_equal")) for r in ok)
                                             and _matched_moe_flops_equal(ok)),
                "execution_contract": (not moe) or all(_moe_execution_contract_valid(r) for r in ok),
            }
            report["files"][filename] = {
                "rows_for_current_run": len(rows),
                "ok": len(ok),
                "skipped": sum(1 for r in rows if r.get("status") == "skipped"),
                "invalid_or_error": len(bad),
                **checks,
            }
            if ok:
                ok_files.add(filename)
            if not rows:
                report["issues"].append(f"{filename}: no rows for run_id={run_id}")
            if bad:
                report["issues"].append(f"{filename}: {len(bad)} invalid/error rows")
            if not all(checks.values()):
                report["issues"].append(f"{filename}: failed numeric/correctness/FLOP/execution checks")
    plot_files = sorted(plots.glob("figure_*.png"))
    pdfs = sorted(plots.glob("figure_*.pdf"))
    signatures_ok = True
    expected_count = 0
    if plots_requested:
        if pdfs:
            report["issues"].append(f"unexpected PDF plot artifacts: {len(pdfs)}")
        for path in plot_files:
            if path.stat().st_size == 0 or path.read_bytes()[:4] != b"\x89PNG":
                signatures_ok = False
                report["issues"].append(f"invalid plot artifact: {path}")
        if ok_files:
            expected_count = sum(PLOTS_PER_FILE[name] for name in ok_files)
            if len(plot_files) != expected_count:
                report["issues"].append(f"expected {expected_count} current plot files, found {len(plot_files)}")
    report["plots"] = {
        "requested": plots_requested,
        "count": len(plot_files) if plots_requested else 0,
        "expected_count": expected_count,
        "format": "png",
        "unexpected_pdf_count": len(pdfs),
        "nonempty_and_decodable_signature": signatures_ok,
    }
    report["valid"] = not report["issues"]
    results.mkdir(parents=True, exist_ok=True)
    (results / "validation.json").write_text(json.dumps(report, indent=2, ensure_ascii=False) + "\n", encoding="utf-8")
    return report


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--results-dir", type=Path, default=Path("results"))
    parser.add_argument("--plots-dir", type=Path, default=Path("plots"))
    args = parser.parse_args(argv)
    report = validate_results(args.results_dir, args.plots_dir)
    print(json.dumps(report, indent=2, ensure_ascii=False))
    return 0 if report["valid"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
