"""GPU end-to-end run of the benchmark driver's heatmap over group sizes and K values.

``benchmark.py --experiment heatmap`` with G in {1, 8} and K in {256, 2880} (2880 leaves a K tail
on every BK) writes one HIP row and one torch row per point; the HIP rows of G = 8 come from one
homogeneous grouped launch, each checked against a float32 torch product per problem with the
reference's tolerances before timing, and the run passes the reference's result validator
(FLOPs recomputed from M, K, N and num_gemms).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


def test_grouped_heatmap_rows_validate(tmp_path):
    from benchmark import main
    from utils.io import read_rows
    from validate_results import validate_results

    results, plots = tmp_path / "results", tmp_path / "plots"
    print("driver heatmap G=1,8 K=256,2880 M=8,128 N=256", flush=True)
    main(["--experiment", "heatmap", "--dtype", "bf16", "--heatmap-gs", "1,8", "--heatmap-ks", "256,2880",
          "--heatmap-ms", "8,128", "--heatmap-ns", "256", "--warmup", "2", "--repeat", "5",
          "--target-timing-ms", "50", "--results-dir", str(results), "--plots-dir", str(plots), "--no-plots"])
    rows = read_rows(results / "gemm_heatmap.csv")
    ok = [r for r in rows if r["status"] == "ok"]
    assert len(ok) == len(rows) == 16, [(r["status"], r["skip_reason"], r["error"]) for r in rows]
    grouped = [r for r in ok if r["num_gemms"] == "8"]
    assert len(grouped) == 8
    for row in grouped:
        assert row["total_flops"] == str(8 * 2 * int(row["M"]) * int(row["K"]) * int(row["N"]))
        if row["provider"] == "hip":
            assert row["mode"] == "grouped" and row["scheduler"] == "homogeneous_persistent"
            assert row["correct"] == "True" and row["config_source"] == "workload_autotune"
        else:
            assert row["provider"] == "torch" and row["scheduler"] == "torch_mm_loop"
    assert {r["scheduler"] for r in ok if r["num_gemms"] == "1" and r["provider"] == "hip"} == {"single_problem_matmul"}
    report = validate_results(results, plots)
    assert report["valid"], report["issues"]
