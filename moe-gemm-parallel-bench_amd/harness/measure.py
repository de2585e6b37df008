"""The measurement pipeline of one case: admission, ring allocation, tuning, gate, timing.

``measure_case(case, providers, settings, env)`` returns one CSV row per provider.  Providers are
grouped by operand layout; each group runs these stages on one shared rotating ring:

1. *skip checks* - a case that could not be formed, or a provider that cannot run here
   (reason recorded, status "skipped");
2. *admission*   - the ring size is 1 (hot) or ``cold_buffers`` >= 2 (rotating-cold), capped by
   the memory budget (free device memory x ``memory_fraction`` less a reserve) over the largest
   per-buffer estimate of the group; a case whose one buffer does not fit, or a cold case that
   cannot hold two, is skipped; ``--max-matrix-bytes`` bounds single-GEMM sweeps;
3. *allocation*  - buffer i is seeded ``seed + i * 100003``; an out-of-memory error retries with
   one buffer fewer, never below the regime's minimum, and never changes a shape;
4. per provider: *tuning* (hot: the launcher's per-workload autotune; cold: one fixed config
   timed across the whole ring), the *correctness gate* (every ring buffer NaN-poisoned,
   launched with the selected config alone, every problem compared with torch's matmul in the
   operand dtype: the W13 reference is [A B_gate | A B_up], checked with the reference's
   per-dtype tolerances), then *timing* with ``time_cuda`` over the ring.
A correctness failure gives status "invalid", an out-of-memory "skipped", any other runtime
failure "error"; the row records the message and the next provider still runs.
"""

from __future__ import annotations

from itertools import groupby

from kernels.torch_grouped_gemm import TorchGroupedMMUnavailable
from utils.benchmark import assert_close, available_budget, time_cuda

from .rows import base_row, measured_row, outcome_row, selected_row

SEED_STRIDE = 100003


def _reference(a, b, projection: str):
    import torch

    if projection == "W1":
        half = b.shape[1] // 2
        return torch.cat((torch.matmul(a, b[:, :half]), torch.matmul(a, b[:, half:])), dim=1)
    return torch.matmul(a, b)


def _gate(provider, ring, selection, case, settings) -> tuple[float, float]:
    """Launch the selected config alone on every buffer and check every problem."""
    import torch

    for operands in ring:
        provider.poison(operands)
        provider.call(operands, selection, settings)
    torch.cuda.synchronize()
    worst_abs = worst_rel = 0.0
    for operands in ring:
        for a, b, c in provider.problems(operands):
            errors = assert_close(c, _reference(a, b, case.projection), settings.dtype)
            worst_abs, worst_rel = max(worst_abs, errors[0]), max(worst_rel, errors[1])
    return worst_abs, worst_rel


class _RingBudget:
    def __init__(self, case, members, settings):
        self.per_buffer = max(p.workspace_bytes(case, settings) for p in members)
        self.budget = available_budget(settings.memory_fraction)
        self.minimum = 2 if settings.cache_mode == "cold" else 1
        wanted = 1 if settings.cache_mode == "hot" else max(2, settings.cold_buffers)
        self.count = min(wanted, self.budget // max(self.per_buffer, 1))

    def refusal(self, case, settings) -> str:
        if self.per_buffer > self.budget:
            return "estimated one-workspace memory exceeds budget"
        if case.experiment != "moe" and settings.max_matrix_bytes and self.per_buffer > settings.max_matrix_bytes:
            return "shape exceeds --max-matrix-bytes"
        if self.count < self.minimum:
            return "rotating-cold needs at least two resident workspaces"
        return ""

    def columns(self, count: int) -> dict:
        return {"estimated_memory_bytes": self.per_buffer * count, "memory_budget_bytes": self.budget,
                "workspace_count": count, "workspace_bytes": self.per_buffer * count}


def _allocate(builder, case, settings, ring_budget: _RingBudget) -> list:
    import torch

    count = ring_budget.count
    while count >= ring_budget.minimum:
        try:
            return [builder.build(case, settings, settings.seed + index * SEED_STRIDE) for index in range(count)]
        except torch.OutOfMemoryError:
            torch.cuda.empty_cache()
            count -= 1
    return []


def _measure_provider(provider, ring, case, settings, env, row) -> dict:
    import torch

    selection = provider.select(ring, case, settings)
    errors = _gate(provider, ring, selection, case, settings)
    row["scheduler"] = provider.scheduler(ring[0])
    selected_row(row, case, selection, env)
    timing = time_cuda(lambda index: provider.call(ring[index % len(ring)], selection, settings),
                       settings.warmup, settings.repeat, settings.target_timing_ms, workspace_count=len(ring))
    torch.cuda.synchronize()
    return measured_row(row, case, timing, errors, settings)


def _measure_layout(case, members, settings, env) -> list[dict]:
    import torch

    rows = [base_row(case, provider, settings, env) for provider in members]
    runnable = []
    for provider, row in zip(members, rows):
        reason = case.skip_reason or provider.unavailable(case, settings)
        if reason:
            outcome_row(row, "skipped", reason)
        else:
            runnable.append((provider, row))
    if not runnable:
        return rows
    torch.cuda.empty_cache()  # blocks freed by the previous case become reusable before the budget query
    ring_budget = _RingBudget(case, [p for p, _ in runnable], settings)
    refusal = ring_budget.refusal(case, settings)
    if refusal:
        for provider, row in runnable:
            outcome_row(row, "skipped", refusal).update(ring_budget.columns(ring_budget.count))
        return rows
    ring = _allocate(runnable[0][0], case, settings, ring_budget)
    if not ring:
        for provider, row in runnable:
            outcome_row(row, "skipped", "out of device memory at the minimum resident workspace count") \
                .update(ring_budget.columns(0))
        return rows
    actual = sum(getattr(ops, "storage_bytes", 0) for ops in ring)
    for provider, row in runnable:
        row.update(ring_budget.columns(len(ring)), workspace_bytes=actual or ring_budget.per_buffer * len(ring))
        try:
            _measure_provider(provider, ring, case, settings, env, row)
        except AssertionError as exc:
            outcome_row(row, "invalid", f"correctness failure: {exc}")
        except TorchGroupedMMUnavailable as exc:
            outcome_row(row, "skipped", str(exc))
        except torch.OutOfMemoryError as exc:
            outcome_row(row, "skipped", f"out of device memory during tuning/gate/timing: {exc}")
        except RuntimeError as exc:
            outcome_row(row, "error", repr(exc))
        if row["status"] != "ok":
            print(f"{row['status'].upper()} {case.name} {provider.name}/{row['mode']}: "
                  f"{row['skip_reason'] or row['error']}", flush=True)
        elif row.get("block_m"):
            # What ran, for the log (the CSV keeps the reference's columns): the tile config, and the
            # tile schedule, K splits and B copy policy the last launch of the HIP workspace recorded.
            schedule = getattr(ring[0], "tile_schedule", None)
            splits = getattr(ring[0], "split_k", None)
            streamed = getattr(ring[0], "b_stream", 0)
            print(f"  {provider.name}/{row['mode']}: {row['block_m']}x{row['block_n']}x{row['block_k']} "
                  f"{row['num_warps']} waves {row['num_stages']} stages GROUP_M {row['group_size_m']} "
                  f"x{row['cta_multiplier']}" + (f" {schedule}" if schedule else "")
                  + (f" split {splits}" if splits and splits > 1 else "")
                  + (" nt-B" if streamed else "") + f": {row['latency_ms'] * 1e3:.1f} us", flush=True)
    del ring
    torch.cuda.empty_cache()
    return rows


def measure_case(case, providers, settings, env) -> list[dict]:
    """One row per provider, in the providers' order."""
    order = {id(p): i for i, p in enumerate(providers)}
    rows: dict[int, dict] = {}
    for _, members in groupby(providers, key=lambda p: p.layout):
        members = list(members)
        for provider, row in zip(members, _measure_layout(case, members, settings, env)):
            rows[order[id(provider)]] = row
    return [rows[i] for i in range(len(providers))]
