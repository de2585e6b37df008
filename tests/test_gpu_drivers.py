"""GPU runs of the harness end to end: experiment driver, validator, comparison runner, torch provider.

* the heatmap driver over G in {1, 8} and K in {256, 2880} (a K tail on every BK): one HIP row
  and one torch.mm row per point, every HIP row gated against torch per problem before timing,
  the run passing the harness validator (FLOPs recomputed from M, K, N and num_gemms);
* the MoE driver, hot with the expert-sorted layout and torch grouped_mm rows, and rotating-cold
  with its ring tuner, on small EP/TP per-rank shapes and at DeepSeek-V3's full per-rank shapes;
* the comparison runner against the per-expert hipBLASLt loop (NaN-poisoned, checked candidates,
  two reversed rounds), and its verdict on a contender that writes nothing;
* the torch grouped_mm provider: admitted or not by its trace check, its results are right;
* the power probe: a short pinned run prints one table row per workload.
"""

from __future__ import annotations

import json

import pytest
import torch

pytestmark = pytest.mark.gpu

_FAST = ["--warmup", "2", "--repeat", "5", "--target-timing-ms", "50"]


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


def test_heatmap_driver_rows_validate(tmp_path):
    from harness.cli import main
    from harness.validate import validate_results
    from utils.io import read_rows

    results = tmp_path / "results"
    print("driver heatmap G=1,8 K=256,2880 M=8,128 N=256", flush=True)
    assert main(["--experiment", "heatmap", "--dtype", "bf16", "--heatmap-gs", "1,8", "--heatmap-ks", "256,2880",
                 "--heatmap-ms", "8,128", "--heatmap-ns", "256", *_FAST, "--results-dir", str(results)]) == 0
    rows = read_rows(results / "gemm_heatmap.csv")
    ok = [r for r in rows if r["status"] == "ok"]
    assert len(ok) == len(rows) == 16, [(r["status"], r["skip_reason"], r["error"]) for r in rows]
    for row in (r for r in ok if r["num_gemms"] == "8"):
        assert row["total_flops"] == str(8 * 2 * int(row["M"]) * int(row["K"]) * int(row["N"]))
        if row["provider"] == "hip":
            assert row["mode"] == "grouped" and row["scheduler"] == "homogeneous_persistent"
            assert row["correct"] == "True" and row["config_source"] == "workload_autotune"
        else:
            assert row["provider"] == "torch" and row["scheduler"] == "torch_mm_loop"
    singles = {r["scheduler"] for r in ok if r["num_gemms"] == "1" and r["provider"] == "hip"}
    assert singles == {"single_problem_matmul"}
    assert validate_results(results)["valid"]


def test_moe_driver_hot_with_offsets_and_torch_rows(tmp_path):
    from harness.cli import main
    from utils.io import read_rows

    results = tmp_path / "hot"
    print("driver moe hot M=8 H=512 F=256 E=16 P=4 bf16 + offsets + torch", flush=True)
    code = main(["--experiment", "moe", "--dtype", "bf16", "--hidden-size", "512", "--ffn-size", "256",
                 "--num-experts", "16", "--topk", "2", "--parallel-size", "4", "--moe-ms", "8", "--offsets-layout",
                 *_FAST, "--results-dir", str(results)])
    report = json.loads((results / "validation.json").read_text())
    assert code == 0 and report["valid"], report["issues"]
    for projection in ("w1", "w2"):
        rows = read_rows(results / f"moe_{projection}.csv")
        hip = [r for r in rows if r["mode"] == "grouped"]
        assert {(r["parallel_type"], r["status"]) for r in hip} == {("EP", "ok"), ("TP", "ok")}
        assert hip[0]["total_flops"] == hip[1]["total_flops"]
        for row in (r for r in rows if r["mode"] == "torch"):
            assert row["status"] in ("ok", "skipped"), row["error"]
            assert row["status"] == "ok" or row["skip_reason"]
        offsets = read_rows(results / f"moe_offsets_{projection}.csv")
        assert {r["status"] for r in offsets} == {"ok"} and {r["scheduler"] for r in offsets} == {"offsets_persistent"}


def test_moe_driver_rotating_cold_ring(tmp_path):
    from harness.cli import main
    from utils.io import read_rows

    results = tmp_path / "cold"
    print("driver moe cold M=64 ring=2", flush=True)
    assert main(["--experiment", "moe", "--dtype", "fp16", "--hidden-size", "512", "--ffn-size", "256",
                 "--num-experts", "16", "--topk", "2", "--parallel-size", "4", "--moe-ms", "64", "--cache-mode", "cold",
                 "--cold-buffers", "2", "--no-torch-baseline", *_FAST, "--results-dir", str(results)]) == 0
    rows = read_rows(results / "moe_w2.csv")
    assert len(rows) == 2
    for row in rows:
        assert row["status"] == "ok" and row["config_source"] == "cold_ring_autotune"
        assert row["workspace_count"] == "2" and int(row["autotune_candidates_tested"]) > 0
        assert int(row["repeat"]) % 2 == 0  # whole rings


def test_moe_driver_rotating_cold_full_size_dsv3(tmp_path):
    """DeepSeek-V3 at its real per-rank shapes (P = 8) in the rotating-cold regime with two
    resident workspaces, M_e in {8, 512}: the ring admission, the cold-ring tuner and the gate on
    every buffer, for W13 and W2, EP and TP (reference benchmark_moe.py:155-206)."""
    from harness.cli import main
    from utils.io import read_rows

    results = tmp_path / "dsv3_cold"
    print("driver moe cold DSV3 full size M=8,512 ring=2", flush=True)
    assert main(["--experiment", "moe", "--dtype", "bf16", "--model-config", "model_configs/deepseek-v3.json",
                 "--parallel-size", "8", "--moe-ms", "8,512", "--cache-mode", "cold", "--cold-buffers", "2",
                 "--no-torch-baseline", "--warmup", "2", "--repeat", "6", "--target-timing-ms", "50",
                 "--results-dir", str(results)]) == 0
    shapes = {("w1", "EP"): (32, 7168, 4096), ("w1", "TP"): (256, 7168, 512),
              ("w2", "EP"): (32, 2048, 7168), ("w2", "TP"): (256, 256, 7168)}  # (G, K, N) per rank
    for projection in ("w1", "w2"):
        rows = read_rows(results / f"moe_{projection}.csv")
        assert len(rows) == 4, [(r["parallel_type"], r["M"], r["status"]) for r in rows]
        assert {(r["parallel_type"], int(r["M"])) for r in rows} == {(p, m) for p in ("EP", "TP") for m in (8, 512)}
        for row in rows:
            label = f"{projection} {row['parallel_type']} M={row['M']}: {row['skip_reason'] or row['error']}"
            assert row["status"] == "ok" and row["correct"] == "True", label
            assert row["config_source"] == "cold_ring_autotune" and row["workspace_count"] == "2", label
            assert int(row["repeat"]) % 2 == 0, label  # whole rings
            got = (int(row["num_gemms"]), int(row["K"]), int(row["N"]))
            assert got == shapes[projection, row["parallel_type"]], label


def test_compare_runner_against_the_hipblaslt_loop(tmp_path):
    from harness.compare import main

    output = tmp_path / "comparison.json"
    print("compare default cases bf16", flush=True)
    assert main(["--dtype", "bf16", "--experts", "4", "--repeat", "5", "--warmup", "1", "--target-timing-ms", "20",
                 "--output", str(output)]) == 0
    report = json.loads(output.read_text())
    assert report["status"] == "passed"
    assert [c["case"] for c in report["cases"]] == ["homogeneous", "heterogeneous", "persistent_rounds"]
    for case in report["cases"]:
        assert case["status"] == "ok" and case["correct"]
        assert {"hip", "hipblaslt_loop"} <= set(case["latency_ms"])
        assert all(len(rounds) == 2 for rounds in case["round_latency_ms"].values())
        assert case["searches"]["hip"]["tested"] >= 1 and case["hip_over_hipblaslt_loop_latency"] > 0


def test_compare_runner_rejects_a_contender_that_writes_nothing(tmp_path):
    from harness.compare import main

    def no_op_hip(contenders):
        for contender in contenders:
            if contender.name == "hip":
                contender.launch = lambda _cfg, _index: None
        return contenders

    output = tmp_path / "broken.json"
    print("compare with a contender that skips its launch", flush=True)
    assert main(["--shape", "64,128,64", "--experts", "2", "--repeat", "3", "--warmup", "0", "--output", str(output)],
                contenders_hook=no_op_hip) == 2
    report = json.loads(output.read_text())
    assert report["status"] == "failed" and report["cases"][0]["status"] == "invalid"


def test_torch_grouped_mm_provider_results_whether_or_not_admitted():
    from kernels.torch_grouped_gemm import (
        TorchGroupedMMUnavailable,
        build_torch_grouped_workspace,
        launch_torch_grouped,
        verify_torch_grouped_execution,
    )

    workspace = build_torch_grouped_workspace([(64, 256, 128)] * 4, torch.bfloat16, seed=3)
    assert workspace.offs.tolist() == [64, 128, 192, 256]
    try:
        evidence = verify_torch_grouped_execution(workspace)
        print(f"torch grouped_mm admitted: {evidence}", flush=True)
        assert evidence["grouped_compute_launches"] == 1 and evidence["execution_verified"]
    except TorchGroupedMMUnavailable as exc:
        print(f"torch grouped_mm not admitted: {exc}", flush=True)
        assert str(exc)
    launch_torch_grouped(workspace)
    torch.cuda.synchronize()
    for a, b, c in workspace.problem_tensors():
        torch.testing.assert_close(c.float(), a.float() @ b.float(), rtol=2e-2, atol=2e-2)


def test_power_probe_prints_a_row_per_workload(capsys):
    """harness.power, shortened: the pinned grouped and single workloads each print a table row with
    a positive rate (power and clock read "n/a" where amd-smi is absent)."""
    from harness.power import main

    assert main(["--seconds", "1", "--skip", "0.3", "--pause", "0", "--workloads", "grouped,single",
                 "--kernel-config", "256,256,32,8,4,8,1"]) == 0
    rows = [line for line in capsys.readouterr().out.splitlines() if line.startswith("| grouped") or
            line.startswith("| single")]
    assert len(rows) == 2, rows
    for row in rows:
        cells = [c.strip() for c in row.strip("|").split("|")]
        assert float(cells[1]) > 0 and float(cells[2]) > 0, row
