"""Providers: the implementations a case can be measured with, behind one interface.

Each provider knows how to size, build and launch the operands of a case and which CSV columns
describe its execution.  Providers with the same ``layout`` share one rotating ring of operands
(the torch per-expert loop runs on exactly the tensors the HIP grouped launch used), so a
baseline is always measured on identical inputs and the ring is allocated once.

============  =======  ==========  ==============================================================
provider      name     mode        what one timed call is
============  =======  ==========  ==============================================================
HipGrouped    hip      grouped /   one ``launch_grouped`` (G = 1 dispatches to ``launch_matmul``;
                       single      mode "single" for the G = 1 single-GEMM experiments)
HipOffsets    hip      offsets     one ``launch_grouped_offsets`` over the expert-sorted layout
TorchLoop     torch    as HIP's    ``torch.mm(a, b, out=c)`` per problem (hipBLASLt), G calls
TorchGrouped  torch    torch       one ``F.grouped_mm`` call, admitted only on trace evidence
============  =======  ==========  ==============================================================
"""

from __future__ import annotations

from dataclasses import dataclass, field

from kernels.grouped_gemm import (
    build_fused_gate_up_workspace,
    build_grouped_workspace,
    grouped_candidate_configs,
    launch_grouped,
)
from kernels.grouped_mm import build_offsets_workspace, launch_grouped_offsets
from kernels.torch_grouped_gemm import (
    build_torch_grouped_workspace,
    launch_torch_grouped,
    torch_grouped_mm_unavailable_reason,
    verify_torch_grouped_execution,
)
from utils.benchmark import dtype_size, tune_rotating_configs

# Device bytes of a grouped launch's tables per problem: three int64 pointers, int32 (m, n, k)
# and six int64 strides.
TABLE_BYTES_PER_PROBLEM = 3 * 8 + 3 * 4 + 6 * 8


def _padded(columns: int, element_size: int) -> int:
    unit = max(1, 16 // element_size)
    return -(-columns // unit) * unit


@dataclass
class Selection:
    """The config a provider will time and the CSV columns describing how it runs."""
    config: object = None
    columns: dict = field(default_factory=dict)
    hot_autotune: bool = False  # timed calls go through the autotune cache (hot-mode semantics)
    b_stream: int | None = None  # B copy policy of the timed calls (None: the hot tuner's choice)


class Provider:
    name = "hip"
    layout = "tensors"
    tiled = True  # carries tile-config columns

    def mode_for(self, case) -> str:
        raise NotImplementedError

    def static_columns(self, case) -> dict:
        return {}

    def unavailable(self, case, settings) -> str:
        return ""

    def workspace_bytes(self, case, settings) -> int:
        es = dtype_size(settings.dtype)
        data = sum(es * (m * k + k * n + m * n) for m, k, n in case.shapes)
        return data + TABLE_BYTES_PER_PROBLEM * case.problem_count

    def build(self, case, settings, seed: int):
        raise NotImplementedError

    def select(self, ring: list, case, settings) -> Selection:
        raise NotImplementedError

    def call(self, operands, selection: Selection, settings) -> None:
        raise NotImplementedError

    def problems(self, operands):
        """(A_e, B_e, C_e) per problem after a call."""
        return operands.problem_tensors()

    def poison(self, operands) -> None:
        """NaN-fill preallocated outputs so an unwritten element fails the gate."""
        for _, _, c in self.problems(operands):
            c.fill_(float("nan"))


class HipGrouped(Provider):
    """The persistent HIP kernel through ``launch_grouped`` (per-expert pointer tables)."""

    def mode_for(self, case) -> str:
        return "single" if case.experiment != "moe" and case.problem_count == 1 else "grouped"

    def static_columns(self, case) -> dict:
        return {"launches_per_iteration": 1, "grouped_compute_launches": 1, "api_calls_per_iteration": 1,
                "execution_verified": True, "output_preallocated": True, "autotune_enabled": True}

    def build(self, case, settings, seed):
        builder = build_fused_gate_up_workspace if case.projection == "W1" else build_grouped_workspace
        return builder(case.shapes, settings.torch_dtype, seed)

    def select(self, ring, case, settings) -> Selection:
        precision = settings.input_precision
        hot = settings.cache_mode == "hot"
        columns = {"autotune_status": "selected"}
        if hot:
            launch_grouped(ring[0], precision, None, autotune=True)  # measures candidates on a cache miss
            config = ring[0].config
            columns["config_source"] = ("shape_family_autotune" if self.mode_for(case) == "single"
                                        else "workload_autotune")
        else:
            candidates = grouped_candidate_configs(
                max(m for m, _, _ in case.shapes), max(n for _, _, n in case.shapes),
                max(k for _, k, _ in case.shapes), problem_count=case.problem_count,
                sm_count=ring[0].sm_count, dtype=settings.torch_dtype)
            tuned = tune_rotating_configs(
                candidates, lambda cfg, index: launch_grouped(ring[index], precision, cfg, autotune=False), len(ring))
            config = tuned.config
            # The B copy policy, timed for the winning tile over the same ring, as the hot tuner
            # times it on its finalists (a launch that cannot stream B runs ordinary copies either way).
            policy = tune_rotating_configs(
                (0, 1), lambda b_stream, index: launch_grouped(ring[index], precision, config, autotune=False,
                                                                b_stream=b_stream), len(ring))
            columns.update(config_source="cold_ring_autotune", autotune_candidates_tested=tuned.candidates_tested,
                           autotune_candidates_failed=tuned.candidates_failed,
                           autotune_selection_ms=min(tuned.median_ms, policy.median_ms))
            return Selection(config, columns, hot_autotune=False, b_stream=policy.config)
        return Selection(config, columns, hot_autotune=hot)

    def call(self, operands, selection, settings) -> None:
        launch_grouped(operands, settings.input_precision, selection.config, autotune=selection.hot_autotune,
                       b_stream=selection.b_stream)

    def scheduler(self, operands) -> str:
        return operands.scheduler


class HipOffsets(HipGrouped):
    """The same kernel over the expert-sorted 2-D A / 3-D B / int32 offsets layout."""

    layout = "offsets"

    def mode_for(self, case) -> str:
        return "offsets"

    def workspace_bytes(self, case, settings) -> int:
        es = dtype_size(settings.dtype)
        k, n = case.k, case.n
        rows = sum(m for m, _, _ in case.shapes)
        return es * (rows * _padded(k, es) + case.problem_count * k * _padded(n, es) + rows * _padded(n, es)) \
            + 4 * case.problem_count

    def build(self, case, settings, seed):
        operation = {"W1": "gate_up", "W2": "down"}.get(case.projection, "gemm")
        return build_offsets_workspace(case.shapes, settings.torch_dtype, seed, operation=operation)

    def select(self, ring, case, settings) -> Selection:
        precision = settings.input_precision
        if settings.cache_mode == "hot":
            launch_grouped_offsets(ring[0], precision, None, autotune=True)
            return Selection(ring[0].config, {"autotune_status": "selected", "config_source": "workload_autotune"},
                             hot_autotune=True)
        candidates = grouped_candidate_configs(case.m, case.n, case.k, problem_count=max(2, case.problem_count),
                                               sm_count=ring[0].sm_count, dtype=settings.torch_dtype)
        tuned = tune_rotating_configs(
            candidates, lambda cfg, index: launch_grouped_offsets(ring[index], precision, cfg, autotune=False),
            len(ring))
        return Selection(tuned.config, {
            "autotune_status": "selected", "config_source": "cold_ring_autotune",
            "autotune_candidates_tested": tuned.candidates_tested,
            "autotune_candidates_failed": tuned.candidates_failed, "autotune_selection_ms": tuned.median_ms})

    def call(self, operands, selection, settings) -> None:
        launch_grouped_offsets(operands, settings.input_precision, selection.config,
                               autotune=selection.hot_autotune)


class TorchLoop(Provider):
    """Per-problem ``torch.mm`` into the preallocated outputs (hipBLASLt on ROCm)."""

    name = "torch"
    tiled = False

    def mode_for(self, case) -> str:
        return HipGrouped().mode_for(case)

    def static_columns(self, case) -> dict:
        calls = case.problem_count
        return {"launches_per_iteration": calls, "api_calls_per_iteration": calls, "grouped_compute_launches": "",
                "execution_verified": False, "output_preallocated": True, "autotune_enabled": False,
                "autotune_status": "not_applicable", "config_source": "library",
                "scheduler": "torch_mm" if calls == 1 else "torch_mm_loop"}

    def build(self, case, settings, seed):  # shares HipGrouped's operands
        return HipGrouped().build(case, settings, seed)

    def select(self, ring, case, settings) -> Selection:
        return Selection(None, {})

    def call(self, operands, selection, settings) -> None:
        import torch

        for a, b, c in operands.problem_tensors():
            torch.mm(a, b, out=c)

    def scheduler(self, operands) -> str:
        return "torch_mm" if operands.problem_count == 1 else "torch_mm_loop"


class TorchGrouped(Provider):
    """One ``torch.nn.functional.grouped_mm`` call, admitted only when a trace proves one
    grouped compute kernel (``kernels.torch_grouped_gemm``)."""

    name = "torch"
    layout = "torch_grouped"
    tiled = False

    def mode_for(self, case) -> str:
        return "torch"

    def static_columns(self, case) -> dict:
        return {"output_preallocated": False, "autotune_enabled": False, "autotune_status": "not_applicable",
                "config_source": "library", "scheduler": "torch_grouped_mm", "execution_verified": False,
                "api_calls_per_iteration": 1}

    def unavailable(self, case, settings) -> str:
        return torch_grouped_mm_unavailable_reason(settings.torch_dtype, case.problem_count)

    def workspace_bytes(self, case, settings) -> int:
        es = dtype_size(settings.dtype)
        data = sum(es * (m * _padded(k, es) + k * _padded(n, es) + m * _padded(n, es)) for m, k, n in case.shapes)
        return data + 4 * case.problem_count

    def build(self, case, settings, seed):
        operation = {"W1": "gate_up", "W2": "down"}.get(case.projection, "gemm")
        return build_torch_grouped_workspace(case.shapes, settings.torch_dtype, seed, operation=operation)

    def select(self, ring, case, settings) -> Selection:
        return Selection(None, dict(verify_torch_grouped_execution(ring[0])))

    def call(self, operands, selection, settings) -> None:
        launch_torch_grouped(operands)

    def poison(self, operands) -> None:
        operands.output = None  # a fresh output per call: nothing to poison

    def scheduler(self, operands) -> str:
        return "torch_grouped_mm"


def providers_for(case, settings) -> list[Provider]:
    """Providers of a case in measurement order (HIP first, then its baselines)."""
    if case.experiment == "moe":
        chosen: list[Provider] = [HipGrouped()]
        if getattr(settings, "offsets_layout", False):
            chosen.append(HipOffsets())
        if settings.torch_baseline:
            chosen.append(TorchGrouped())
        return chosen
    return [HipGrouped()] + ([TorchLoop()] if settings.torch_baseline else [])
