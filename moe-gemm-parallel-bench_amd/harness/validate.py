"""``python -m harness.validate --results-dir DIR``: check a results directory against the contract.

The contract (the reference's result semantics, reference validate_results.py:46-248, restated
as rules; this checker is written from that statement):

Scope.  ``environment.json`` must carry a ``run_id``; only rows of that run are checked.  The
files checked follow ``requested_parameters.experiment``: shapes -> ``gemm_shape_sweep.csv``,
moe -> ``moe_w1.csv`` + ``moe_w2.csv`` (+ ``moe_offsets_w1/w2.csv`` when the run used the
expert-sorted layout), heatmap -> ``gemm_heatmap.csv``; "all" selects every one.

Per file.  At least one row for the run; no row with status "invalid" or "error"; and every row
with status "ok" passes each rule that applies to the file:

  metrics_positive     latency_ms, total_flops and tflops are finite and > 0
  correct              correct is true
  flops_recomputed     total_flops == 2 M K N num_gemms (to 0.5) and
                       tflops == total_flops / (latency_ms 1e9) (relative 1e-6)
  projection (MoE)     W1 rows: projection W1, operation gate_up, fused_projections 2,
                       output_layout gate_then_up, activation not timed;
                       W2 rows: projection W2, operation down, fused_projections 1,
                       output_layout down, activation not timed
  flops_equal (MoE)    flops_equal is true, and EP and TP rows that agree on
                       (M, mode, provider, cache_mode, dtype, parallel_size, num_experts, topk, T)
                       have equal total_flops
  execution (MoE)      mode "grouped": autotune enabled and selected, config_source
                       workload_autotune or cold_ring_autotune, scheduler one of
                       homogeneous_persistent / generic_persistent / single_problem_matmul,
                       exactly one launch per iteration, output preallocated, positive integer
                       block_m/n/k, num_warps, num_stages, cta_multiplier;
                       mode "torch": scheduler torch_grouped_mm, one API call and one grouped
                       compute launch per iteration, a positive launch count, execution verified,
                       output not preallocated;
                       mode "offsets" (this build's expert-sorted layout): as "grouped" but with
                       scheduler offsets_persistent.
Booleans are read as true from 1/true/yes and false from 0/false/no (any case).  Plots are not
part of this build, so figures are never required.
"""

from __future__ import annotations

import argparse
import csv
import json
import math
from collections.abc import Callable
from datetime import datetime, timezone
from pathlib import Path

_TRUE = {"1", "true", "yes"}
_FALSE = {"0", "false", "no"}
_FILES = {
    "shapes": ("gemm_shape_sweep.csv",),
    "moe": ("moe_w1.csv", "moe_w2.csv"),
    "heatmap": ("gemm_heatmap.csv",),
}
_OFFSETS_FILES = ("moe_offsets_w1.csv", "moe_offsets_w2.csv")
_GROUPED_SCHEDULERS = {"homogeneous_persistent", "generic_persistent", "single_problem_matmul"}
_TILE_COLUMNS = ("block_m", "block_n", "block_k", "num_warps", "num_stages", "cta_multiplier")
_PROJECTIONS = {
    "W1": {"projection": "W1", "operation": "gate_up", "fused_projections": "2", "output_layout": "gate_then_up"},
    "W2": {"projection": "W2", "operation": "down", "fused_projections": "1", "output_layout": "down"},
}
_MATCH_KEY = ("M", "mode", "provider", "cache_mode", "dtype", "parallel_size", "num_experts", "topk", "T")


def _flag(value, expected: bool) -> bool:
    return str(value or "").strip().lower() in (_TRUE if expected else _FALSE)


def _number(value) -> float | None:
    try:
        number = float(value)
    except (TypeError, ValueError, OverflowError):
        return None
    return number if math.isfinite(number) else None


def _positive_int(value) -> bool:
    number = _number(value)
    return number is not None and number > 0 and number == int(number)


# --------------------------------------------------------------------------- row rules

def metrics_positive(row: dict) -> bool:
    return all((_number(row.get(c)) or 0.0) > 0 for c in ("latency_ms", "total_flops", "tflops"))


def correct(row: dict) -> bool:
    return _flag(row.get("correct"), True)


def flops_recomputed(row: dict) -> bool:
    values = [_number(row.get(c)) for c in ("M", "K", "N", "total_flops", "latency_ms", "tflops")]
    gemms = _number(row.get("num_gemms", "1"))
    if None in values or gemms is None:
        return False
    m, k, n, total, latency, tflops = values
    if min(m, k, n, gemms, latency) <= 0:
        return False
    expected_flops = 2 * int(m) * int(k) * int(n) * int(gemms)
    return abs(total - expected_flops) <= 0.5 and math.isclose(tflops, expected_flops / (latency * 1e9),
                                                               rel_tol=1e-6, abs_tol=1e-12)


def projection_for(filename: str) -> Callable[[dict], bool]:
    projection = "W1" if filename.endswith("w1.csv") else "W2"
    wanted = _PROJECTIONS[projection]

    def check(row: dict) -> bool:
        return all(row.get(c) == v for c, v in wanted.items()) and _flag(row.get("activation_in_timed_region"),
                                                                           False)
    return check


def execution(row: dict) -> bool:
    mode = row.get("mode")
    if mode == "torch":
        return (row.get("scheduler") == "torch_grouped_mm" and row.get("api_calls_per_iteration") == "1"
                and row.get("grouped_compute_launches") == "1" and _positive_int(row.get("launches_per_iteration"))
                and _flag(row.get("execution_verified"), True) and _flag(row.get("output_preallocated"), False))
    schedulers = {"grouped": _GROUPED_SCHEDULERS, "offsets": {"offsets_persistent"}}.get(mode)
    if schedulers is None:
        return False
    return (_flag(row.get("autotune_enabled"), True) and row.get("autotune_status") == "selected"
            and row.get("config_source") in ("workload_autotune", "cold_ring_autotune")
            and row.get("scheduler") in schedulers and row.get("launches_per_iteration") == "1"
            and _flag(row.get("output_preallocated"), True) and all(_positive_int(row.get(c)) for c in _TILE_COLUMNS))


def flops_equal(rows: list[dict]) -> bool:
    """Row flag plus the EP == TP FLOP equality of matched rows (file-level)."""
    if not all(_flag(r.get("flops_equal"), True) for r in rows):
        return False
    totals: dict[tuple, dict[str, float | None]] = {}
    for row in rows:
        totals.setdefault(tuple(row.get(c, "") for c in _MATCH_KEY), {})[row.get("parallel_type")] = \
            _number(row.get("total_flops"))
    return all(pair["EP"] == pair["TP"] for pair in totals.values() if {"EP", "TP"} <= pair.keys())


def _rules_for(filename: str) -> dict[str, Callable[[list[dict]], bool]]:
    """Rule name -> check over the file's ok rows."""
    rules: dict[str, Callable[[list[dict]], bool]] = {
        "metrics_positive": lambda rows: all(map(metrics_positive, rows)),
        "correct": lambda rows: all(map(correct, rows)),
        "flops_recomputed": lambda rows: all(map(flops_recomputed, rows)),
    }
    if filename.startswith("moe_"):
        projection = projection_for(filename)
        rules["projection"] = lambda rows: all(map(projection, rows))
        rules["flops_equal"] = flops_equal
        rules["execution"] = lambda rows: all(map(execution, rows))
    return rules


# --------------------------------------------------------------------------- files

def _rows_of_run(path: Path, run_id: str) -> list[dict]:
    if not path.exists():
        return []
    with path.open(newline="", encoding="utf-8") as handle:
        return [row for row in csv.DictReader(handle) if not run_id or row.get("run_id") == run_id]


def validate_results(results_dir: str | Path = "results", plots_dir: str | Path | None = None) -> dict:
    """Check the directory, write ``validation.json`` into it and return the report.
    (``plots_dir`` is accepted for call compatibility; figures are not part of this build.)"""
    results = Path(results_dir)
    environment_path = results / "environment.json"
    environment = json.loads(environment_path.read_text(encoding="utf-8")) if environment_path.exists() else {}
    run_id = str(environment.get("run_id") or "")
    requested = environment.get("requested_parameters") or {}
    experiment = str(requested.get("experiment") or "all")
    selected = sorted(_FILES) if experiment == "all" else [experiment]
    filenames = [name for group in selected for name in _FILES[group]]
    if "moe" in selected and requested.get("offsets_layout"):
        filenames += list(_OFFSETS_FILES)
    report: dict = {"timestamp": datetime.now(timezone.utc).isoformat(), "run_id": run_id,
                    "selected_experiments": selected, "environment_present": environment_path.exists(),
                    "files": {}, "issues": []}
    if not run_id:
        report["issues"].append("environment.json has no run_id")
    for filename in filenames:
        rows = _rows_of_run(results / filename, run_id)
        by_status: dict[str, list[dict]] = {}
        for row in rows:
            by_status.setdefault(row.get("status", ""), []).append(row)
        ok = by_status.get("ok", [])
        failed = by_status.get("invalid", []) + by_status.get("error", [])
        checks = {name: bool(rule(ok)) for name, rule in _rules_for(filename).items()}
        report["files"][filename] = {"rows_for_current_run": len(rows), "ok": len(ok),
                                     "skipped": len(by_status.get("skipped", [])),
                                     "invalid_or_error": len(failed), "checks": checks}
        if not rows:
            report["issues"].append(f"{filename}: no rows for run_id={run_id}")
        if failed:
            report["issues"].append(f"{filename}: {len(failed)} invalid/error rows")
        broken = sorted(name for name, passed in checks.items() if not passed)
        if broken:
            report["issues"].append(f"{filename}: ok rows fail {', '.join(broken)}")
    report["valid"] = not report["issues"]
    (results / "validation.json").write_text(json.dumps(report, indent=2) + "\n", encoding="utf-8")
    return report


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(prog="python -m harness.validate", description=__doc__.splitlines()[0])
    parser.add_argument("--results-dir", type=Path, default=Path("results"))
    parser.add_argument("--plots-dir", type=Path, default=None, help="ignored: no figures are produced")
    args = parser.parse_args(argv)
    report = validate_results(args.results_dir)
    print(json.dumps(report, indent=2))
    return 0 if report["valid"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
