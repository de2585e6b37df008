"""CPU tests of the benchmark harness: argument checks, case plans, providers, rows, validator."""

from __future__ import annotations

import json
import math

import pytest
import torch

from harness import cases as case_lists
from harness.cli import build_parser, main, settings_from_args
from harness.compare import build_parser as compare_parser
from harness.compare import comparison_cases, parse_shape
from harness.measure import measure_case
from harness.providers import HipGrouped, HipOffsets, TorchGrouped, TorchLoop, providers_for
from harness.rows import annotate, base_row
from harness.validate import execution, flops_equal, flops_recomputed, projection_for, validate_results
from utils.io import CSV_FIELDS, write_rows


def _settings(*argv):
    return settings_from_args(build_parser().parse_args(list(argv)))


@pytest.mark.parametrize("argv", [
    ["--hidden-size", "0"], ["--ffn-size", "0"], ["--num-experts", "0"], ["--topk", "0"], ["--heatmap-k", "0"],
    ["--peak-tflops", "-1"], ["--input-precision", "tf32", "--dtype", "bf16"], ["--memory-fraction", "0"],
    ["--heatmap-gs", "0"], ["--heatmap-ks", "1,0"], ["--moe-ms", "0"], ["--tokens", "0"], ["--repeat", "0"],
    ["--cold-buffers", "0"], ["--warmup", "-1"],
])
def test_cli_rejects_bad_values_before_touching_a_gpu(argv, tmp_path):
    with pytest.raises(ValueError):
        main([*argv, "--results-dir", str(tmp_path)])
    assert not (tmp_path / "environment.json").exists()


def test_cli_flags_and_resolved_settings():
    ns = build_parser().parse_args([])
    assert ns.torch_baseline and not ns.offsets_layout and ns.dtype == "fp16" and ns.experiment == "all"
    assert not build_parser().parse_args(["--no-torch-baseline"]).torch_baseline
    assert build_parser().parse_args(["--heatmap-gs", "1,8", "--heatmap-ks", "256,2880"]).heatmap_gs == [1, 8]
    s = _settings("--model-config", "model_configs/mixtral-8x7b.json", "--topk", "1")
    assert (s.hidden_size, s.ffn_size, s.num_experts, s.topk, s.heatmap_k) == (4096, 14336, 8, 1, 4096)
    assert s.model_config == "model_configs/mixtral-8x7b.json"
    assert s.requested_parameters["no_plots"] is True and s.requested_parameters["topk"] == 1
    assert s.effective_parameters["topk"] == 1 and s.torch_dtype == torch.float16
    assert json.dumps(s.requested_parameters)  # provenance is JSON-serialisable


def test_moe_cases_pair_ep_and_tp_with_equal_flops():
    s = _settings("--moe-ms", "8,512")
    w1 = case_lists.moe_cases(s, "W1")
    assert [(c.m, c.parallel_type) for c in w1] == [(8, "EP"), (8, "TP"), (512, "EP"), (512, "TP")]
    assert w1[0].shapes == ((8, 7168, 4096),) * 32 and w1[1].shapes == ((8, 7168, 512),) * 256
    assert w1[0].total_flops == w1[1].total_flops and w1[0].tokens == 8 * 256 // 8
    assert w1[0].projection_labels == ("gate_up", 2, "gate_then_up")
    w2 = case_lists.moe_cases(s, "W2")
    assert w2[1].shapes == ((8, 256, 7168),) * 256 and w2[0].projection_labels == ("down", 1, "down")
    assert case_lists.moe_token_counts(_settings("--tokens", "4096")) == (4096 * 8 // 256,)


def test_moe_sweep_argument_checks():
    with pytest.raises(ValueError, match="divisible by topk"):
        case_lists.moe_token_counts(_settings("--num-experts", "8", "--topk", "5", "--parallel-size", "4",
                                              "--moe-ms", "3"))
    with pytest.raises(ValueError, match="tokens"):
        case_lists.moe_token_counts(_settings("--num-experts", "8", "--topk", "5", "--parallel-size", "4",
                                              "--tokens", "3"))
    with pytest.raises(ValueError, match="parallel_size"):
        case_lists.moe_token_counts(_settings("--parallel-size", "3"))


def test_shape_and_heatmap_plans():
    shapes = case_lists.shape_cases(_settings("--shape-ms", "16,3", "--shape-product", "1024", "--shape-k", "64"))
    assert shapes[0].shapes == ((16, 64, 64),) and not shapes[0].skip_reason
    assert shapes[1].skip_reason == "M does not divide shape product"
    grid = case_lists.heatmap_cases(_settings("--heatmap-gs", "1,8", "--heatmap-ks", "256,2880",
                                              "--heatmap-ms", "8,128", "--heatmap-ns", "256"))
    assert [(c.problem_count, c.k, c.m, c.n) for c in grid] == [
        (g, k, m, 256) for g in (1, 8) for k in (256, 2880) for m in (8, 128)]
    default = case_lists.heatmap_cases(_settings("--heatmap-ms", "8", "--heatmap-ns", "256"))
    assert [c.shapes for c in default] == [((8, 7168, 256),)]  # the reference's grid: G = 1 at the hidden size
    plan = dict(case_lists.iter_experiments(_settings("--moe-ms", "8", "--shape-ms", "16", "--heatmap-ms", "8",
                                                      "--heatmap-ns", "256")))
    assert list(plan) == ["gemm_shape_sweep", "moe_w1", "moe_w2", "gemm_heatmap"]


def test_providers_per_experiment():
    s = _settings("--moe-ms", "8")
    moe = case_lists.moe_cases(s, "W1")[0]
    assert [type(p) for p in providers_for(moe, s)] == [HipGrouped, TorchGrouped]
    s.offsets_layout = True
    assert [type(p) for p in providers_for(moe, s)] == [HipGrouped, HipOffsets, TorchGrouped]
    s.torch_baseline = False
    assert [type(p) for p in providers_for(moe, s)] == [HipGrouped, HipOffsets]
    single = case_lists.Case("heatmap", ((8, 64, 32),))
    grouped = case_lists.Case("heatmap", ((8, 64, 32),) * 4)
    assert [type(p) for p in providers_for(single, _settings())] == [HipGrouped, TorchLoop]
    assert HipGrouped().mode_for(single) == "single" and HipGrouped().mode_for(grouped) == "grouped"
    assert HipGrouped().mode_for(moe) == "grouped" and TorchLoop().static_columns(grouped)["scheduler"] == "torch_mm_loop"


def test_workspace_estimates():
    s = _settings("--dtype", "bf16")
    case = case_lists.Case("moe", ((16, 64, 128),) * 2, "W2", "EP")
    assert HipGrouped().workspace_bytes(case, s) == 2 * 2 * (16 * 64 + 64 * 128 + 16 * 128) + 2 * 84
    odd = case_lists.Case("moe", ((16, 13, 31),), "W2", "EP")
    assert TorchGrouped().workspace_bytes(odd, s) == 2 * (16 * 16 + 13 * 32 + 16 * 32) + 4
    assert HipOffsets().workspace_bytes(odd, s) == TorchGrouped().workspace_bytes(odd, s)


def test_base_row_has_the_wire_columns_and_provider_facts():
    s = _settings("--moe-ms", "8", "--dtype", "bf16")
    case = case_lists.moe_cases(s, "W1")[1]
    env = {"gpu_name": "MI355X", "sm_count": 256, "cuda_version": "7.0", "torch_version": "2.10",
           "triton_version": "libmoegemm-abi5"}
    row = base_row(case, HipGrouped(), s, env)
    assert set(row) <= set(CSV_FIELDS)
    assert (row["mode"], row["provider"], row["parallel_type"], row["num_gemms"]) == ("grouped", "hip", "TP", 256)
    assert row["total_flops"] == case.total_flops and row["weight_shard_factor"] == 8 and row["T"] == 256
    assert row["launches_per_iteration"] == 1 and row["config_source"] == "heuristic_fallback"
    torch_row = base_row(case, TorchGrouped(), s, env)
    assert "block_m" not in torch_row  # library rows leave the tile columns empty
    assert torch_row["mode"] == "torch" and torch_row["output_preallocated"] is False


def test_unavailable_provider_is_a_skipped_row_without_touching_the_gpu():
    s = _settings("--moe-ms", "8", "--dtype", "fp16")
    case = case_lists.moe_cases(s, "W2")[0]
    rows = measure_case(case, [TorchGrouped()], s, {})
    assert rows[0]["status"] == "skipped" and rows[0]["skip_reason"]
    formed = case_lists.Case("shapes", ((3, 64, 0),), skip_reason="M does not divide shape product")
    assert measure_case(formed, [HipGrouped(), TorchLoop()], s, {})[1]["skip_reason"] == formed.skip_reason


def test_annotate_efficiency_and_near_best():
    rows = [{"status": "ok", "tflops": 100.0, "M": 8, "parallel_type": "EP"},
            {"status": "ok", "tflops": 80.0, "M": 8, "parallel_type": "EP"},
            {"status": "ok", "tflops": 50.0, "M": 8, "parallel_type": "TP"},
            {"status": "skipped", "M": 8, "parallel_type": "TP"}]
    annotate(rows, "moe")
    assert [r.get("normalized_efficiency") for r in rows[:3]] == [1.0, 0.8, 0.5]
    assert rows[1]["best_measured_ratio"] == 0.8 and not rows[1]["near_best"] and rows[2]["near_best"]
    single = [{"status": "ok", "tflops": 10.0, "provider": "hip", "num_gemms": 1, "M": 1, "K": 2, "N": 3},
              {"status": "ok", "tflops": 20.0, "provider": "torch", "num_gemms": 1, "M": 1, "K": 2, "N": 3}]
    annotate(single, "single")
    assert single[1]["normalized_efficiency"] == 2.0 and single[0]["best_measured_ratio"] == 0.5


# ------------------------------------------------------------------------------------ validator

GROUPED = {"mode": "grouped", "autotune_enabled": "True", "autotune_status": "selected",
           "config_source": "workload_autotune", "scheduler": "homogeneous_persistent",
           "launches_per_iteration": "1", "output_preallocated": "True", "block_m": "256", "block_n": "256",
           "block_k": "64", "num_warps": "8", "num_stages": "2", "cta_multiplier": "2"}


def test_flops_are_recomputed_from_the_shape():
    row = {"M": "2", "K": "3", "N": "4", "num_gemms": "5", "total_flops": "240", "latency_ms": "2",
           "tflops": "0.00000012"}
    assert flops_recomputed(row)
    assert not flops_recomputed({**row, "total_flops": "241"})
    assert not flops_recomputed({**row, "tflops": "1"})
    assert not flops_recomputed({**row, "latency_ms": "0"})
    assert not flops_recomputed({**row, "M": "nan"})


def test_execution_contract_per_mode():
    assert execution(GROUPED)
    for broken in ({"mode": "single"}, {"autotune_status": "not_run"}, {"launches_per_iteration": "2"},
                   {"num_stages": "0"}, {"config_source": "heuristic_fallback"}, {"output_preallocated": "no"},
                   {"scheduler": "offsets_persistent"}, {"cta_multiplier": "1.5"}):
        assert not execution({**GROUPED, **broken}), broken
    offsets = {**GROUPED, "mode": "offsets", "scheduler": "offsets_persistent"}
    assert execution(offsets) and not execution({**offsets, "scheduler": "homogeneous_persistent"})
    torch_row = {"mode": "torch", "scheduler": "torch_grouped_mm", "launches_per_iteration": "2",
                 "api_calls_per_iteration": "1", "grouped_compute_launches": "1", "execution_verified": "yes",
                 "output_preallocated": "False"}
    assert execution(torch_row)
    assert not execution({**torch_row, "execution_verified": "False"})
    assert not execution({**torch_row, "scheduler": "torch_mm_loop"})


def test_projection_semantics_and_flops_equality():
    w1 = {"projection": "W1", "operation": "gate_up", "fused_projections": "2", "output_layout": "gate_then_up",
          "activation_in_timed_region": "False"}
    assert projection_for("moe_w1.csv")(w1) and not projection_for("moe_w2.csv")(w1)
    assert not projection_for("moe_w1.csv")({**w1, "activation_in_timed_region": "True"})
    ep = {"flops_equal": "True", "parallel_type": "EP", "total_flops": "64", "M": "4", "mode": "grouped"}
    assert flops_equal([ep, {**ep, "parallel_type": "TP"}])
    assert not flops_equal([ep, {**ep, "parallel_type": "TP", "total_flops": "65"}])
    assert not flops_equal([{**ep, "flops_equal": "False"}])


def _moe_row(parallel_type: str, **extra):
    m, k, n, g = 4, 8, 16, 2
    flops = 2 * m * k * n * g
    return {**GROUPED, "run_id": "r1", "status": "ok", "correct": "True", "projection": "W1",
            "operation": "gate_up", "fused_projections": "2", "output_layout": "gate_then_up",
            "activation_in_timed_region": "False", "M": str(m), "K": str(k), "N": str(n), "num_gemms": str(g),
            "total_flops": str(flops), "latency_ms": "0.5", "tflops": repr(flops / (0.5 * 1e9)),
            "flops_equal": "True", "parallel_type": parallel_type, "provider": "hip", "cache_mode": "hot",
            "dtype": "bf16", "parallel_size": "4", "num_experts": "8", "topk": "2", "T": "16", **extra}


def test_validate_results_end_to_end(tmp_path):
    (tmp_path / "environment.json").write_text(json.dumps(
        {"run_id": "r1", "requested_parameters": {"experiment": "moe", "no_plots": True}}))
    down = {"projection": "W2", "operation": "down", "fused_projections": "1", "output_layout": "down"}
    write_rows(tmp_path / "moe_w1.csv", [_moe_row("EP"), _moe_row("TP"), {**_moe_row("TP"), "run_id": "old",
                                                                          "status": "error"}])
    write_rows(tmp_path / "moe_w2.csv", [_moe_row("EP", **down), _moe_row("TP", **down)])
    report = validate_results(tmp_path)
    assert report["valid"], report["issues"]
    assert report["files"]["moe_w1.csv"]["rows_for_current_run"] == 2  # the other run's row is ignored
    assert json.loads((tmp_path / "validation.json").read_text())["valid"]
    write_rows(tmp_path / "moe_w2.csv", [_moe_row("EP", **down), _moe_row("TP", **down, total_flops="1")])
    assert not validate_results(tmp_path)["valid"]
    write_rows(tmp_path / "moe_w2.csv", [_moe_row("EP", **down, status="error")])
    report = validate_results(tmp_path)
    assert not report["valid"] and any("invalid/error" in issue for issue in report["issues"])
    (tmp_path / "moe_w2.csv").unlink()
    assert any("no rows" in issue for issue in validate_results(tmp_path)["issues"])
    (tmp_path / "environment.json").write_text("{}")
    assert "environment.json has no run_id" in validate_results(tmp_path)["issues"]


def test_compare_arguments_and_default_cases():
    assert parse_shape("1,2,3") == (1, 2, 3)
    for bad in ("1,2", "a,b,c", "0,1,1"):
        with pytest.raises(Exception):
            parse_shape(bad)
    args = compare_parser().parse_args(["--experts", "3"])
    names = {name: shapes for name, shapes in comparison_cases(args, 16)}
    assert names["homogeneous"] == [(128, 256, 128)] * 3 and len(names["persistent_rounds"]) == 17
    assert len({s for s in names["heterogeneous"]}) == 3
    args = compare_parser().parse_args(["--moe-config", "moe-gemm-parallel-bench_amd/model_configs/deepseek-v3.json",
                                        "--moe-ms", "8"])
    moe = dict(comparison_cases(args, 256))
    assert list(moe) == ["W1_EP_M8", "W1_TP_M8", "W2_EP_M8", "W2_TP_M8"]
    assert math.prod(moe["W2_TP_M8"][0]) == 8 * 256 * 7168


def test_power_harness_parses_amd_smi_and_kernel_config():
    """harness.power reads SOCKET_POWER and every XCD's GFX clock from amd-smi's text output, and
    takes --kernel-config in bench.py's order (BM,BN,BK,WARPS,STAGES,GROUP_M,MULT)."""
    from harness.power import parse_amd_smi, parse_kernel_config

    text = """GPU: 0
    POWER:
        SOCKET_POWER: 1399 W
        GFX_VOLTAGE: N/A
    CLOCK:
        GFX_0:
            CLK: 1456 MHz
            MIN_CLK: 500 MHz
        GFX_1:
            CLK: 1470 MHz
            MIN_CLK: 500 MHz
        MEM_0:
            CLK: 1900 MHz
"""
    power, clocks = parse_amd_smi(text)
    assert power == 1399.0
    assert clocks == [1456.0, 1470.0]
    assert parse_amd_smi("") == (None, [])
    cfg = parse_kernel_config("256,256,32,8,4,8,1")
    assert (cfg.block_m, cfg.block_n, cfg.block_k, cfg.num_warps, cfg.num_stages, cfg.group_size_m,
            cfg.cta_multiplier) == (256, 256, 32, 8, 4, 8, 1)
    assert parse_kernel_config(None) is None


def test_bench_reads_the_traffic_figure_of_the_policy_that_ran():
    """bench.py's roofline.traffic comes from the committed counter summary of the headline, which
    gives one figure per B copy policy; a policy without its own line takes the plain one."""
    import importlib.util
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("bench_under_test", root / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    case = "dsv3_w1_ep_me512"
    ordinary, streamed = bench._traffic_from_profiles(case, 0), bench._traffic_from_profiles(case, 1)
    algorithmic = 2 * 32 * (512 * 7168 + 7168 * 4096 + 512 * 4096)
    assert ordinary is not None and streamed is not None and ordinary != streamed
    for measured in (ordinary, streamed):
        assert abs(measured / algorithmic - 1) < 0.01
    assert bench._traffic_from_profiles("no_such_case", 1) is None
