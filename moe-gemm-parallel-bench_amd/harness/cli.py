"""``python -m harness``: run the shape sweep, the MoE EP/TP sweep and/or the heatmap; write CSVs.

The command-line flags are the reference's driver interface (reference benchmark.py:50-96), so a
sweep written for it runs here unchanged; three flags are added: ``--heatmap-gs`` (group counts of
the heatmap), ``--heatmap-ks`` (its K values) and ``--offsets-layout`` (also time MoE cases on the
expert-sorted layout, written to ``moe_offsets_w1.csv`` / ``moe_offsets_w2.csv``).

Outputs in ``--results-dir``: ``environment.json`` (run provenance), one CSV per experiment
(``gemm_shape_sweep.csv``, ``moe_w1.csv``, ``moe_w2.csv``, ``gemm_heatmap.csv``) and
``validation.json``.  Plots are not produced by this build (out of its scope): the run records
``no_plots`` so validators do not expect figures.  Exit status 0 when the results validate, 2
otherwise.
"""

from __future__ import annotations

import argparse
import json
import uuid
from dataclasses import dataclass, field
from datetime import datetime, timezone
from pathlib import Path

from utils.benchmark import TIMING_METHOD, configure_torch_matmul, dtype_supported, select_cuda_device
from utils.config import ModelDefaults, load_model_defaults
from utils.hardware import write_environment
from utils.io import write_rows

from . import cases as case_lists
from .measure import measure_case
from .providers import providers_for
from .rows import annotate, base_row, outcome_row
from .validate import validate_results

PACKAGE_ROOT = Path(__file__).resolve().parents[1]
DEFAULT_MODEL_CONFIG = Path("model_configs/deepseek-v3.json")


def _ints(text: str) -> list[int]:
    return [int(part) for part in text.split(",") if part.strip()]


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(prog="python -m harness",
                                description="MoE expert GEMM benchmark (HIP grouped GEMM on MI355X), EP vs TP")
    add = p.add_argument
    add("--experiment", choices=["all", "shapes", "moe", "heatmap"], default="all")
    add("--model-config", type=Path, default=DEFAULT_MODEL_CONFIG)
    add("--dtype", choices=["fp16", "bf16", "fp32"], default="fp16")
    add("--parallel-size", type=int, default=8)
    add("--num-experts", type=int)
    add("--topk", type=int)
    add("--hidden-size", type=int)
    add("--ffn-size", type=int)
    add("--tokens", type=int, help="pre-routing token count T: one MoE M = T * topk / E instead of the sweep")
    add("--moe-ms", type=_ints, help="comma-separated tokens-per-expert sweep")
    add("--warmup", type=int, default=25)
    add("--repeat", type=int, default=100)
    add("--target-timing-ms", type=float, default=2000.0, help="cap on measured device time per case")
    add("--cache-mode", choices=["hot", "cold"], default="hot")
    add("--cold-buffers", type=int, default=2)
    add("--memory-fraction", type=float, default=0.8)
    add("--peak-tflops", type=float)
    add("--input-precision", choices=["ieee", "tf32"], default="ieee")
    add("--device", default="cuda", help="logical GPU (cuda or cuda:N)")
    add("--seed", type=int, default=1234)
    add("--torch-baseline", action=argparse.BooleanOptionalAction, default=True,
        help="add torch.mm rows to single-GEMM sweeps and trace-verified torch grouped_mm rows to MoE")
    add("--offsets-layout", action=argparse.BooleanOptionalAction, default=False,
        help="also time MoE cases on the expert-sorted 2-D A / 3-D B / int32 offsets layout")
    add("--shape-k", type=int, default=4096)
    add("--shape-product", type=int, default=1024 * 1024)
    add("--shape-ms", type=_ints)
    add("--max-matrix-bytes", type=int, default=0)
    add("--heatmap-k", type=int, help="defaults to the model's hidden size")
    add("--heatmap-ms", type=_ints)
    add("--heatmap-ns", type=_ints)
    add("--heatmap-ks", type=_ints, help="K values of the heatmap (default: --heatmap-k alone)")
    add("--heatmap-gs", type=_ints, help="group counts G of the heatmap (default: 1, the single GEMM)")
    add("--results-dir", type=Path, default=Path("results"))
    add("--plots-dir", type=Path, default=Path("plots"))
    add("--no-plots", action="store_true", help="accepted for compatibility; plots are never produced")
    return p


@dataclass
class Settings:
    experiment: str
    dtype: str
    model: ModelDefaults
    model_config: str
    hidden_size: int
    ffn_size: int
    num_experts: int
    topk: int
    parallel_size: int
    tokens: int | None
    moe_ms: list | None
    warmup: int
    repeat: int
    target_timing_ms: float
    cache_mode: str
    cold_buffers: int
    memory_fraction: float
    peak_tflops: float | None
    input_precision: str
    device: str
    seed: int
    torch_baseline: bool
    offsets_layout: bool
    shape_k: int
    shape_product: int
    shape_ms: list | None
    max_matrix_bytes: int
    heatmap_k: int
    heatmap_ms: list | None
    heatmap_ns: list | None
    heatmap_ks: list | None
    heatmap_gs: list | None
    results_dir: Path
    plots_dir: Path
    run_id: str = field(default_factory=lambda: uuid.uuid4().hex[:12])
    timestamp: str = field(default_factory=lambda: datetime.now(timezone.utc).isoformat())
    requested_parameters: dict = field(default_factory=dict)
    effective_parameters: dict = field(default_factory=dict)

    @property
    def torch_dtype(self):
        from utils.benchmark import torch_dtype

        return torch_dtype(self.dtype)


def _model_path(path: Path) -> Path:
    """A relative path that does not exist from the working directory is looked up in the package."""
    path = path.expanduser()
    if not path.is_absolute() and not path.exists() and (PACKAGE_ROOT / path).exists():
        path = PACKAGE_ROOT / path
    return path.resolve()


def _portable(path: Path) -> str:
    """Provenance path without the local absolute prefix: relative to the package, else the name."""
    try:
        return str(Path(path).resolve().relative_to(PACKAGE_ROOT))
    except ValueError:
        return Path(path).name


def settings_from_args(ns: argparse.Namespace) -> Settings:
    """Resolve model defaults and check every value that can be checked without a GPU (ValueError)."""
    checks = [
        (0 < ns.memory_fraction <= 1, "--memory-fraction must be in (0, 1]"),
        (ns.warmup >= 0, "--warmup must be non-negative"),
        (ns.repeat > 0 and ns.target_timing_ms > 0, "--repeat and --target-timing-ms must be positive"),
        (ns.cold_buffers > 0, "--cold-buffers must be positive"),
        (ns.max_matrix_bytes >= 0, "--max-matrix-bytes must be non-negative"),
        (ns.peak_tflops is None or ns.peak_tflops > 0, "--peak-tflops must be positive"),
        (ns.tokens is None or ns.tokens > 0, "--tokens must be positive"),
        (ns.input_precision != "tf32" or ns.dtype == "fp32", "--input-precision tf32 requires --dtype fp32"),
    ]
    for ok, message in checks:
        if not ok:
            raise ValueError(message)
    model_path = _model_path(ns.model_config)
    model = load_model_defaults(model_path)
    dims = {name: getattr(ns, name) if getattr(ns, name) is not None else getattr(model, name)
            for name in ("hidden_size", "ffn_size", "num_experts", "topk")}
    heatmap_k = ns.heatmap_k if ns.heatmap_k is not None else dims["hidden_size"]
    positive = {"--parallel-size": ns.parallel_size, "--num-experts": dims["num_experts"], "--topk": dims["topk"],
                "--hidden-size": dims["hidden_size"], "--ffn-size": dims["ffn_size"], "--shape-k": ns.shape_k,
                "--shape-product": ns.shape_product, "--heatmap-k": heatmap_k}
    bad = [flag for flag, value in positive.items() if value <= 0]
    if bad:
        raise ValueError("these parameters must be positive: " + ", ".join(bad))
    for flag in ("moe_ms", "shape_ms", "heatmap_ms", "heatmap_ns", "heatmap_ks", "heatmap_gs"):
        values = getattr(ns, flag)
        if values is not None and (not values or min(values) <= 0):
            raise ValueError(f"--{flag.replace('_', '-')} must list positive integers")
    requested = {key: (_portable(value) if key in ("model_config", "results_dir", "plots_dir")
                       else str(value) if isinstance(value, Path) else value)
                 for key, value in vars(ns).items()}
    requested["no_plots"] = True  # this build never draws figures
    settings = Settings(
        experiment=ns.experiment, dtype=ns.dtype, model=model, model_config=_portable(model_path),
        parallel_size=ns.parallel_size, tokens=ns.tokens, moe_ms=ns.moe_ms, warmup=ns.warmup, repeat=ns.repeat,
        target_timing_ms=ns.target_timing_ms, cache_mode=ns.cache_mode, cold_buffers=ns.cold_buffers,
        memory_fraction=ns.memory_fraction, peak_tflops=ns.peak_tflops, input_precision=ns.input_precision,
        device=ns.device, seed=ns.seed, torch_baseline=ns.torch_baseline, offsets_layout=ns.offsets_layout,
        shape_k=ns.shape_k, shape_product=ns.shape_product, shape_ms=ns.shape_ms,
        max_matrix_bytes=ns.max_matrix_bytes, heatmap_k=heatmap_k, heatmap_ms=ns.heatmap_ms,
        heatmap_ns=ns.heatmap_ns, heatmap_ks=ns.heatmap_ks, heatmap_gs=ns.heatmap_gs,
        results_dir=ns.results_dir, plots_dir=ns.plots_dir, requested_parameters=requested, **dims,
    )
    settings.effective_parameters = {
        "timing_method": TIMING_METHOD, **dims, "parallel_size": ns.parallel_size, "dtype": ns.dtype,
        "config_ep_size": model.config_ep_size, "model_declared_dtype": model.dtype,
        "model_quantization": model.quantization, "cache_mode": ns.cache_mode, "device": ns.device,
        "torch_fp32_matmul_precision": ns.input_precision,
        "kernels": "libmoegemm: hand-written gfx950 HIP grouped/single GEMM (MFMA, LDS-DMA), one launch per call",
        "hot_autotune": "per-workload: every candidate timed by hipGraph replay, five finalists re-timed",
        "cold_autotune": "one fixed config timed across the complete rotating workspace ring",
        "torch_moe_baseline": "torch.nn.functional.grouped_mm, admitted only when a trace shows one grouped kernel",
        "w1_semantics": "one-launch packed W13 Gate+Up GEMM, [gate | up] output; activation excluded",
        "near_best_threshold": 0.90,
        "plots": "not produced by this build",
    }
    return settings


def _ep_tp_table(rows: list[dict], projection: str) -> str:
    by_m: dict[int, dict[str, dict]] = {}
    for row in rows:
        if row.get("mode") == "grouped" and row.get("status") == "ok":
            by_m.setdefault(int(row["M"]), {})[row["parallel_type"]] = row
    lines = [f"\n{'W1/W3 Gate+Up' if projection == 'W1' else 'W2 Down'} grouped GEMM (per rank)",
             "| M_e | EP TFLOP/s | TP TFLOP/s | TP/EP | EP ms | TP ms |", "|---:|---:|---:|---:|---:|---:|"]
    for m in sorted(by_m):
        pair = by_m[m]
        if {"EP", "TP"} <= pair.keys():
            ep, tp = pair["EP"], pair["TP"]
            lines.append(f"| {m} | {ep['tflops']:.3f} | {tp['tflops']:.3f} | {tp['tflops'] / ep['tflops']:.3f} "
                         f"| {ep['latency_ms']:.4f} | {tp['latency_ms']:.4f} |")
    return "\n".join(lines)


def _unavailable_rows(settings, env, plan, reason: str) -> dict[str, list[dict]]:
    """One skipped row per output file when nothing can run on this machine."""
    from .providers import HipGrouped

    out = {}
    for stem, cases in plan:
        first = cases[0] if cases else case_lists.Case("moe" if stem.startswith("moe") else "heatmap", ((1, 1, 1),))
        out[stem] = [outcome_row(base_row(first, HipGrouped(), settings, env), "skipped", reason)]
    return out


def run(settings: Settings) -> dict[str, list[dict]]:
    """Measure every planned case; returns rows per CSV stem (also written to the results dir)."""
    from kernels import _native

    plan = list(case_lists.iter_experiments(settings))  # all argument checks before any GPU work
    settings.device = select_cuda_device(settings.device)
    configure_torch_matmul(settings.input_precision)
    settings.results_dir.mkdir(parents=True, exist_ok=True)
    env = write_environment(settings.results_dir / "environment.json", {
        "run_id": settings.run_id, "timestamp": settings.timestamp, "model_config": settings.model_config,
        "model_type": settings.model.model_type, "model_declared_dtype": settings.model.dtype,
        "model_quantization": settings.model.quantization,
        "requested_parameters": settings.requested_parameters,
        "effective_parameters": settings.effective_parameters,
        "note": "Synthetic dense-dtype benchmark of one rank's expert GEMMs; deployed quantization and "
                "communication are not emulated.",
    })
    print(f"GPU: {env.get('gpu_name')} ({env.get('gfx_arch')}, {env.get('sm_count')} CUs) | HIP: "
          f"{env.get('cuda_version')} | torch: {env.get('torch_version')} | kernels: {env.get('triton_version')} "
          f"| dtype: {settings.dtype}", flush=True)
    supported, reason = dtype_supported(settings.dtype)
    if supported and not _native.available():
        supported, reason = False, "libmoegemm.so is not built"
    if not supported:
        print(f"benchmark skipped: {reason}")
        results = _unavailable_rows(settings, env, plan, reason)
    else:
        results = {}
        for stem, cases in plan:
            rows = []
            for case in cases:
                print(f"case {case.name}", flush=True)
                rows.extend(measure_case(case, providers_for(case, settings), settings, env))
            extension = [r for r in rows if r.get("mode") == "offsets"]
            rows = [r for r in rows if r.get("mode") != "offsets"]
            experiment = "moe" if stem.startswith("moe") else "single"
            annotate(rows, experiment)
            results[stem] = rows
            if extension:
                annotate(extension, experiment)
                results[stem.replace("moe_", "moe_offsets_")] = extension
    for stem, rows in results.items():
        write_rows(settings.results_dir / f"{stem}.csv", rows)
    for projection in ("W1", "W2"):
        if f"moe_{projection.lower()}" in results and supported:
            print(_ep_tp_table(results[f"moe_{projection.lower()}"], projection))
    return results


def main(argv: list[str] | None = None) -> int:
    settings = settings_from_args(build_parser().parse_args(argv))
    run(settings)
    report = validate_results(settings.results_dir)
    print(f"Validation: {'PASS' if report['valid'] else 'FAIL'} ({settings.results_dir / 'validation.json'})")
    for issue in report["issues"]:
        print(f"  - {issue}")
    print(json.dumps({"results": sorted(p.name for p in settings.results_dir.iterdir())}))
    return 0 if report["valid"] else 2
