"""Hardware-independent contract tests of the host layer (mirrors the reference's tests/test_cpu.py
where the contract carries over; Triton-tutorial and plotting checks have no counterpart here)."""

from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import torch

from kernels.grouped_gemm import (
    _GROUPED_BASE_CONFIG_POOL,
    _shape_signature,
    build_fused_gate_up_workspace,
    build_grouped_workspace,
    grouped_candidate_configs,
    workspace_from_tensors,
)
from kernels.matmul import (
    _MATMUL_CONFIG_POOL,
    _MATMUL_CONFIG_POOL_F32,
    KernelConfig,
    diverse_configs,
    matmul_candidate_configs,
    select_config,
)
from kernels.torch_grouped_gemm import (
    TorchGroupedMMUnavailable,
    build_torch_grouped_workspace,
    inspect_grouped_trace,
    launch_torch_grouped,
)
from utils.benchmark import _whole_ring_count, percentile, time_cuda
from utils.config import load_model_defaults
from utils.io import CSV_FIELDS, read_rows, write_rows
from utils.metrics import arithmetic_intensity, gemm_flops, moe_shapes, tile_metrics, verify_ep_tp_flops

CONFIGS = Path(__file__).resolve().parents[1] / "moe-gemm-parallel-bench_amd" / "model_configs"


def test_timing_counts_visit_complete_workspace_rings():
    assert _whole_ring_count(1, 3, 8) == 8
    assert _whole_ring_count(5, 3, 2) == 6
    assert _whole_ring_count(100, 3, 1) == 100


def test_percentile_interpolates():
    assert percentile([4.0, 1.0, 3.0, 2.0], 0.5) == 2.5
    assert percentile([1.0], 0.2) == 1.0
    assert math.isnan(percentile([], 0.5))


def test_time_cuda_rejects_invalid_counts_before_touching_a_gpu():
    for args in ((0, 1), (-1, 1)):
        with pytest.raises(ValueError):
            time_cuda(lambda _: None, args[1], args[0])
    with pytest.raises(ValueError):
        time_cuda(lambda _: None, 1, 1, workspace_count=0)


def test_deepseek_v3_mapping():
    config = load_model_defaults(CONFIGS / "deepseek-v3.json")
    assert (config.hidden_size, config.ffn_size, config.num_experts, config.topk) == (7168, 2048, 256, 8)
    assert config.dtype == "bf16"


def test_all_bundled_model_config_schemas():
    expected = {
        "deepseek-v3.json": (7168, 2048, 256, 8), "deepseek-v4-flash.json": (4096, 2048, 256, 6),
        "glm-5.2.json": (6144, 2048, 256, 8), "gpt-oss-120b.json": (2880, 2880, 128, 4),
        "kimi-k3.json": (7168, 3072, 896, 16), "llama-4-maverick-17b-128e.json": (5120, 8192, 128, 1),
        "llama-4-scout-17b-16e.json": (5120, 8192, 16, 1), "mixtral-8x7b.json": (4096, 14336, 8, 2),
        "qwen3-235b-a22b.json": (4096, 1536, 128, 8), "qwen3-30b-a3b.json": (2048, 768, 128, 8),
    }
    for filename, dims in expected.items():
        config = load_model_defaults(CONFIGS / filename)
        assert (config.hidden_size, config.ffn_size, config.num_experts, config.topk) == dims, filename


def test_config_schema_errors_name_the_missing_field(tmp_path):
    path = tmp_path / "bad.json"
    path.write_text(json.dumps({"hidden_size": 8, "num_experts": 4}))
    with pytest.raises(ValueError, match="ffn_size"):
        load_model_defaults(path)


def test_ep_tp_flops_equal_w1_and_w2():
    for projection in ("W1", "W2"):
        total = verify_ep_tp_flops(projection, 17, 7168, 2048, 256, 8)
        ep = sum(gemm_flops(*s) for s in moe_shapes(projection, "EP", 17, 7168, 2048, 256, 8))
        tp = sum(gemm_flops(*s) for s in moe_shapes(projection, "TP", 17, 7168, 2048, 256, 8))
        assert total == ep == tp
    assert verify_ep_tp_flops("W1", 17, 7168, 2048, 256, 8) == 2 * verify_ep_tp_flops("W2", 17, 7168, 2048, 256, 8)


def test_ep_tp_shapes_split_the_intended_dimension():
    assert moe_shapes("W1", "EP", 17, 7168, 2048, 256, 8) == [(17, 7168, 4096)] * 32
    assert moe_shapes("W1", "TP", 17, 7168, 2048, 256, 8) == [(17, 7168, 512)] * 256
    assert moe_shapes("W2", "EP", 17, 7168, 2048, 256, 8) == [(17, 2048, 7168)] * 32
    assert moe_shapes("W2", "TP", 17, 7168, 2048, 256, 8) == [(17, 256, 7168)] * 256


def test_baseline_config_shapes():
    # Mixtral P=8, Qwen3-30B-A3B P=4.
    assert moe_shapes("W1", "EP", 16, 4096, 14336, 8, 8) == [(16, 4096, 28672)]
    assert moe_shapes("W2", "TP", 16, 4096, 14336, 8, 8) == [(16, 1792, 4096)] * 8
    assert moe_shapes("W1", "TP", 4, 2048, 768, 128, 4) == [(4, 2048, 384)] * 128
    assert moe_shapes("W2", "EP", 4, 2048, 768, 128, 4) == [(4, 768, 2048)] * 32


def test_shape_and_tile_metrics():
    assert gemm_flops(2, 3, 4) == 48
    assert arithmetic_intensity(16, 32, 64, 2) == pytest.approx(2 * 16 * 32 * 64 / (2 * (16 * 32 + 32 * 64 + 16 * 64)))
    metrics = tile_metrics([(17, 31, 65)] * 3, 16, 64, 32, 30)
    assert metrics["total_output_tiles_per_rank"] == 12
    assert metrics["estimated_waves"] == 1
    assert metrics["dot_tiles"] == 12
    assert 0 < metrics["tile_efficiency"] < 1


def test_divisibility_rejected():
    with pytest.raises(ValueError):
        moe_shapes("W1", "TP", 1, 8, 10, 8, 4)
    with pytest.raises(ValueError):
        moe_shapes("W3", "EP", 1, 8, 8, 8, 4)


@pytest.mark.parametrize("dtype", [None, torch.float32])
def test_select_config_is_always_compiled(dtype):
    pool = set(_MATMUL_CONFIG_POOL_F32 if dtype == torch.float32 else _MATMUL_CONFIG_POOL)
    for m in (1, 8, 16, 17, 32, 64, 100, 512, 4096):
        for n in (1, 31, 64, 65, 256, 4096):
            for k in (1, 70, 128, 7168):
                assert select_config(m, n, k, dtype) in pool


def test_candidate_sets_are_bounded_unique_and_compiled():
    for m in (1, 16, 32, 64, 128, 512):
        for n in (3, 32, 64, 128, 512):
            for k in (1, 32, 128, 8192):
                single = matmul_candidate_configs(m, n, k)
                assert 0 < len(single) <= 10 and len(set(single)) == len(single)
                assert set(single) <= set(_MATMUL_CONFIG_POOL)
                grouped = grouped_candidate_configs(m, n, k, problem_count=8, sm_count=16)
                assert 0 < len(grouped) <= 36 and len(set(grouped)) == len(grouped)
                for cfg in grouped:
                    assert KernelConfig(**{**cfg.as_dict(), "cta_multiplier": 1}) in _GROUPED_BASE_CONFIG_POOL


def test_large_single_gemms_measure_the_eight_wave_256_tiles_first():
    """The cost model ranks the 8-wave 256x256 schedules (ping-pong first) above the 4-wave
    256x256 tiles, whose 128x128 wave tiles spill, so large single GEMMs always measure them."""
    for m, n, k in ((2048, 7168, 7168), (2048, 7168, 2880), (1024, 28672, 4096), (8192, 8192, 8192),
                    (2048, 7168, 256)):
        keys = [cfg.tile_key for cfg in matmul_candidate_configs(m, n, k, dtype=torch.bfloat16, sm_count=256)]
        assert keys[0] == (256, 256, 32, 8, 4), (m, n, k, keys)
        assert (256, 256, 64, 4, 2) not in keys[:3] and (256, 256, 32, 4, 4) not in keys[:3]


def test_grouped_candidates_cover_the_workload_families():
    skinny = grouped_candidate_configs(8, 4096, 7168, problem_count=32, sm_count=256)
    assert {c.block_m for c in skinny} <= {16, 32}
    # Decode groups (M_e <= 16) time 32-row tiles next to the 16-row ones: the 32x512x32
    # four-stage tile is the measured best on DSV3 EP W2 at M_e = 8.
    decode = grouped_candidate_configs(8, 7168, 2048, problem_count=32, sm_count=256, dtype=torch.bfloat16)
    assert {c.block_m for c in decode} == {16, 32}
    assert any(c.tile_key == (32, 512, 32, 4, 4) for c in decode)
    wide = grouped_candidate_configs(512, 4096, 7168, problem_count=32, sm_count=256)
    assert any(c.block_m == 256 and c.block_n == 256 for c in wide)
    assert {c.cta_multiplier for c in wide} >= {1, 2}
    one = grouped_candidate_configs(16, 256, 7168, problem_count=1, sm_count=256)
    assert {c.cta_multiplier for c in one} == {1}
    tiny_grid = grouped_candidate_configs(16, 64, 64, problem_count=2, sm_count=256)
    assert {c.cta_multiplier for c in tiny_grid} == {1}  # fewer tiles than CUs: no duplicate grids
    fp32 = grouped_candidate_configs(64, 64, 64, problem_count=4, sm_count=256, dtype=torch.float32)
    assert set(KernelConfig(**{**c.as_dict(), "cta_multiplier": 1}) for c in fp32) <= set(_MATMUL_CONFIG_POOL_F32)
    with pytest.raises(ValueError):
        grouped_candidate_configs(0, 1, 1)
    with pytest.raises(ValueError):
        grouped_candidate_configs(1, 1, 1, sm_count=-1)


def test_diverse_configs_keeps_coverage_then_rank_order():
    ranked = list(_MATMUL_CONFIG_POOL)
    picked = diverse_configs(ranked, 5)
    assert len(picked) == 5 and picked[0] == ranked[0]
    assert len({(c.block_m, c.block_n) for c in picked}) >= 3
    assert diverse_configs(ranked, 0) == ranked[:1]


def test_shape_signature_is_order_sensitive_31_bit():
    a = _shape_signature([(17, 13, 31), (1, 5, 3)])
    b = _shape_signature([(1, 5, 3), (17, 13, 31)])
    assert a != b and 0 <= a < 2**31 and a == _shape_signature([(17, 13, 31), (1, 5, 3)])


def test_cpu_workspace_tables_and_flags():
    shapes = [(1, 5, 3), (17, 13, 31), (9, 70, 65)]
    ws = build_grouped_workspace(shapes, torch.bfloat16, seed=99, device="cpu")
    assert ws.dims.tolist() == [[1, 3, 5], [17, 31, 13], [9, 65, 70]]
    assert ws.strides.tolist()[2] == [70, 1, 65, 1, 65, 1]
    assert ws.a_ptrs.tolist() == [t.data_ptr() for t in ws.a]
    assert not ws.homogeneous and ws.problem_count == 3 and (ws.max_m, ws.max_n, ws.max_k) == (17, 65, 70)
    assert ws.tile_count_for(KernelConfig(16, 64, 32, 1, 4, 2)) == 1 + 2 + 2
    same = build_grouped_workspace([(17, 13, 31)] * 3, torch.float16, device="cpu")
    assert same.homogeneous
    strided = workspace_from_tensors([t.t() for t in same.b], [t.t() for t in same.a],
                                     [torch.empty(31, 17, dtype=torch.float16) for _ in range(3)])
    assert not strided.homogeneous
    with pytest.raises(ValueError):
        build_grouped_workspace([], torch.float16, device="cpu")
    with pytest.raises(ValueError):
        build_grouped_workspace([(1, 0, 3)], torch.float16, device="cpu")
    with pytest.raises(ValueError):
        build_fused_gate_up_workspace([(17, 13, 31)], torch.float16, device="cpu")
    w13 = build_fused_gate_up_workspace([(17, 13, 62)] * 2, torch.float16, device="cpu")
    assert w13.operation == "gate_up"


def test_seeded_workspaces_are_reproducible():
    first = build_grouped_workspace([(4, 8, 16)] * 2, torch.bfloat16, seed=7, device="cpu")
    second = build_grouped_workspace([(4, 8, 16)] * 2, torch.bfloat16, seed=7, device="cpu")
    assert all(torch.equal(x, y) for x, y in zip(first.a + first.b, second.a + second.b))


def test_torch_grouped_workspace_layout_on_cpu():
    ws = build_torch_grouped_workspace([(17, 13, 31)] * 3, torch.bfloat16, seed=104, device="cpu")
    assert ws.offs.tolist() == [17, 34, 51]
    assert ws.mat_a.stride(0) % 8 == 0 and ws.mat_b.stride(1) % 8 == 0
    launch_torch_grouped(ws)
    for a, b, c in ws.problem_tensors():
        torch.testing.assert_close(c.float(), a.float() @ b.float(), rtol=2e-2, atol=2e-2)
    with pytest.raises(ValueError):
        build_torch_grouped_workspace([(17, 13, 31), (17, 14, 31)], torch.bfloat16, device="cpu")


def test_grouped_trace_inspector_fails_closed():
    compute = "void ck::kernel_grouped_gemm_xdl_splitk<...>"
    ok = inspect_grouped_trace(["aten::_grouped_mm"], ["prepare_grouped_gemm_data", compute])
    assert ok["grouped_compute_launches"] == 1 and ok["launches_per_iteration"] == 2
    for cpu, gpu in (
        (["aten::_grouped_mm", "aten::mm"], [compute]),
        (["aten::_grouped_mm"], []),
        (["aten::_grouped_mm"], ["Cijk_Ailk_Bljk_gemm", "Cijk_Ailk_Bljk_gemm"]),
        (["aten::_grouped_mm"], [compute, "Memcpy DtoH"]),
        (["aten::_grouped_mm"], [compute, compute]),
        ([], [compute]),
    ):
        with pytest.raises(TorchGroupedMMUnavailable):
            inspect_grouped_trace(cpu, gpu)


def test_result_schema_columns():
    for field in ("operation", "fused_projections", "output_layout", "activation_in_timed_region", "scheduler",
                  "cta_multiplier", "output_preallocated", "best_measured_ratio", "near_best",
                  "autotune_candidates_tested"):
        assert field in CSV_FIELDS
    assert len(CSV_FIELDS) == len(set(CSV_FIELDS)) == 87


def test_csv_roundtrip(tmp_path):
    path = tmp_path / "rows.csv"
    write_rows(path, [{"M": 4, "status": "ok", "unknown_column": 1}])
    rows = read_rows(path)
    assert rows[0]["M"] == "4" and rows[0]["status"] == "ok" and "unknown_column" not in rows[0]
    assert list(rows[0]) == CSV_FIELDS
    assert read_rows(tmp_path / "absent.csv") == []


def test_offsets_workspace_layout_on_cpu():
    from kernels.grouped_mm import build_offsets_workspace, offsets_tile_bound
    from oracle import oracle

    ws = build_offsets_workspace([(17, 13, 31), (0, 13, 31), (5, 13, 31)], torch.bfloat16, seed=3, device="cpu")
    assert ws.offs.dtype == torch.int32 and ws.offs.tolist() == [17, 17, 22]
    assert ws.mat_a.shape == (22, 13) and ws.mat_b.shape == (3, 13, 31) and ws.output.shape == (22, 31)
    assert ws.mat_a.stride(0) % 8 == 0 and ws.mat_b.stride(1) % 8 == 0 and ws.output.stride(0) % 8 == 0
    assert [a.shape[0] for a, _, _ in ws.problem_tensors()] == [17, 0, 5]
    for rows, groups, n, bm, bn in ((22, 3, 31, 16, 64), (0, 3, 31, 16, 64), (1000, 7, 300, 256, 256)):
        assert offsets_tile_bound(rows, groups, n, bm, bn) == oracle.offsets_tile_bound(rows, groups, n, bm, bn)
    with pytest.raises(ValueError):
        build_offsets_workspace([(17, 13, 31), (17, 14, 31)], torch.bfloat16, device="cpu")
    with pytest.raises(ValueError):
        build_offsets_workspace([(-1, 13, 31)], torch.bfloat16, device="cpu")


def test_grouped_mm_validates_before_touching_a_gpu():
    from kernels.grouped_mm import grouped_mm

    a = torch.zeros((8, 16), dtype=torch.bfloat16)
    b = torch.zeros((2, 16, 8), dtype=torch.bfloat16)
    offs = torch.tensor([4, 8], dtype=torch.int32)
    with pytest.raises(ValueError):  # host tensors: the kernel path needs a GPU device
        grouped_mm(a, b, offs)
    with pytest.raises(ValueError):
        grouped_mm(a, b, offs.long())
    with pytest.raises(ValueError):
        grouped_mm(a, b[:, :8], offs)


def test_grouped_mm_rejects_strided_and_expanded_offs():
    """The kernel reads offs as a dense int32 array: a strided view would give wrong group
    boundaries and an expanded (stride 0) one would read past its storage."""
    from kernels.grouped_mm import grouped_mm, grouped_mm_swiglu

    a = torch.zeros((8, 16), dtype=torch.bfloat16)
    b = torch.zeros((2, 16, 32), dtype=torch.bfloat16)
    strided = torch.tensor([[4, 0], [8, 0]], dtype=torch.int32)[:, 0]
    expanded = torch.tensor([8], dtype=torch.int32).expand(2)
    for offs in (strided, expanded):
        assert not offs.is_contiguous()
        for launch in (grouped_mm, grouped_mm_swiglu):
            with pytest.raises(ValueError, match="contiguous"):
                launch(a, b, offs)


def test_grouped_mm_swiglu_validates_before_touching_a_gpu():
    from kernels.grouped_mm import grouped_mm_swiglu

    a = torch.zeros((8, 16), dtype=torch.bfloat16)
    offs = torch.tensor([4, 8], dtype=torch.int32)
    with pytest.raises(ValueError):  # host tensors: the kernel path needs a GPU device
        grouped_mm_swiglu(a, torch.zeros((2, 16, 32), dtype=torch.bfloat16), offs)
    with pytest.raises(ValueError):
        grouped_mm_swiglu(a, torch.zeros((2, 16, 32), dtype=torch.bfloat16), offs.long())


def test_schedule_options_pair_unsplit_candidates_with_both_schedules():
    from kernels.grouped_gemm import with_schedule_options

    a, b = KernelConfig(16, 256, 64, 8, 4, 4, 1), KernelConfig(64, 128, 64, 8, 4, 4, 1)
    options = [(a, 1), (a, 4), (b, 1)]
    assert with_schedule_options(options, None) == [(a, 1, "static"), (a, 1, "stealing"), (a, 4, "static"),
                                                    (b, 1, "static"), (b, 1, "stealing")]
    assert with_schedule_options(options, "static") == [(a, 1, "static"), (a, 4, "static"), (b, 1, "static")]
    assert with_schedule_options(options, "stealing") == [(a, 1, "stealing"), (b, 1, "stealing")]


def test_tile_schedule_is_validated_before_touching_a_gpu():
    from kernels.grouped_gemm import launch_grouped
    from kernels.grouped_mm import grouped_mm

    workspace = build_grouped_workspace([(8, 16, 32)] * 2, torch.bfloat16, device="cpu")
    with pytest.raises(ValueError, match="tile_schedule"):
        launch_grouped(workspace, tile_schedule="dynamic")
    with pytest.raises(ValueError, match="unsplit"):
        launch_grouped(workspace, tile_schedule="stealing", split_k=2)
    a = torch.zeros((8, 16), dtype=torch.bfloat16)
    b = torch.zeros((2, 16, 8), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="tile_schedule"):
        grouped_mm(a, b, torch.tensor([4, 8], dtype=torch.int32), tile_schedule="dynamic")


def _fake_tuner_timing(monkeypatch, base_ms, first_penalty=None, failing=()):
    """Replace the tuner's GPU timing with a deterministic model: each candidate's time is its
    base, plus ``first_penalty`` on the very first timing after the clock warm-up; candidates in
    ``failing`` raise as a launch the library rejects would."""
    import kernels.matmul as mm

    calls = []

    def bench(fn, quantiles):
        name = fn()
        calls.append(name)
        extra = first_penalty if first_penalty is not None and len(calls) == 1 else 0.0
        return [base_ms[name] + extra for _ in quantiles]

    def launch(cfg):
        if cfg in failing:
            raise RuntimeError(f"{cfg} rejected")
        return cfg

    monkeypatch.setattr(mm, "hot_autotune_bench", bench)
    monkeypatch.setattr(mm, "_warm_clocks", lambda fn: fn())
    return launch, calls


def test_tuner_second_sweep_rescues_a_candidate_timed_while_the_clock_settled(monkeypatch):
    from kernels.matmul import _FINAL_ROUNDS, _FINALISTS, _tune

    base = {"best": 1.0, **{f"c{i}": 1.05 + 0.01 * i for i in range(8)}}
    launch, calls = _fake_tuner_timing(monkeypatch, base, first_penalty=1.0)
    candidates = ["best"] + [f"c{i}" for i in range(8)]
    assert _tune(candidates, launch) == "best"
    # Two sweeps over every candidate, then the finalists' interleaved rounds.
    assert len(calls) == 2 * len(candidates) + _FINALISTS * _FINAL_ROUNDS
    assert calls[:len(candidates)] == candidates and calls[len(candidates):2 * len(candidates)] == candidates[::-1]


def test_tuner_skips_rejected_candidates_and_keeps_a_preferred_one_within_its_margin(monkeypatch):
    from kernels.matmul import _tune

    base = {"a": 1.00, "b": 1.02, "c": 0.90}
    launch, _ = _fake_tuner_timing(monkeypatch, base, failing=("c",))
    assert _tune(["a", "b", "c"], launch) == "a"
    assert _tune(["a", "b", "c"], launch, prefer="b") == "b"  # 2 % slower: within the 3 % margin
    launch, _ = _fake_tuner_timing(monkeypatch, {"a": 1.0, "b": 1.1})
    assert _tune(["a", "b"], launch, prefer="b") == "a"
    launch, _ = _fake_tuner_timing(monkeypatch, {"a": 1.0}, failing=("a",))
    with pytest.raises(RuntimeError, match="every autotune candidate failed"):
        _tune(["a"], launch)


def test_workspace_shape_stats_follow_the_shapes_tuple():
    """max_m/max_n/max_k and tile_count_for are cached per ``shapes`` tuple; assigning a new tuple
    (a rebuilt routing) recomputes them."""
    from kernels.grouped_gemm import build_grouped_workspace
    from kernels.matmul import KernelConfig

    ws = build_grouped_workspace([(8, 64, 128)] * 3, torch.bfloat16, seed=1, device="cpu")
    cfg = KernelConfig(16, 128, 64, 8, 4, 2)
    assert (ws.max_m, ws.max_n, ws.max_k, ws.tile_count_for(cfg)) == (8, 128, 64, 3)
    ws.shapes = ((8, 64, 128), (40, 96, 256), (8, 64, 128))
    assert (ws.max_m, ws.max_n, ws.max_k) == (40, 256, 96)
    assert ws.tile_count_for(cfg) == 1 + 3 * 2 + 1
    assert ws.tile_count_for(KernelConfig(32, 256, 64, 8, 4, 2)) == 1 + 2 + 1
