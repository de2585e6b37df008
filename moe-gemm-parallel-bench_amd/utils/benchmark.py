"""Device timing, tuning, dtype, memory and correctness helpers (HIP/ROCm).

Same public names and semantics as the reference's utils/benchmark.py:
  * ``time_cuda`` (reference utils/benchmark.py:154-198) times device execution from graph
    replays, so host dispatch never lands inside a sample.  The reference captures one event pair
    per call inside the graph; ROCm torch forbids external events in a capture, so here each
    sample is one timed replay of a chunk of whole rings (mean per-call time of that replay).
    Warmup and repeat counts are capped towards a 250 ms warmup and ``target_ms`` measurement
    budget, then rounded up to whole workspace rings, as in the reference.
  * ``tune_rotating_configs`` (:201-246) picks a fixed config by timing each candidate across the
    whole rotating ring; candidates that raise ``RuntimeError``/``AssertionError`` are discarded.
  * ``hot_autotune_bench`` (:249-258) is the bounded hot timer used by the launchers' autotuner.
  * ``assert_close`` (:261-271) applies the per-dtype tolerances and reports max abs/rel error.
On ROCm the graph is a hipGraph.
"""

from __future__ import annotations

import math
import statistics
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import TypeVar

TIMING_METHOD = "hip_graph_replay_events"
ConfigT = TypeVar("ConfigT")

# Per-dtype assert_close tolerances (rtol, atol), as the reference's utils/benchmark.py:268.
TOLERANCES = {"fp16": (2e-2, 2e-2), "bf16": (5e-2, 5e-2), "fp32": (2e-3, 2e-3)}


@dataclass(frozen=True)
class TimingResult:
    p20_ms: float
    median_ms: float
    p80_ms: float
    mean_ms: float
    std_ms: float
    warmup: int
    repeat: int


@dataclass(frozen=True)
class TuningResult:
    config: object
    median_ms: float
    candidates_tested: int
    candidates_failed: int


def torch_dtype(name: str):
    import torch

    table = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
    if name not in table:
        raise ValueError(f"unknown dtype name {name!r}")
    return table[name]


def dtype_size(name: str) -> int:
    return {"fp16": 2, "bf16": 2, "fp32": 4}[name]


def select_cuda_device(device_spec: str) -> str:
    """Select one logical GPU (``cuda`` / ``cuda:N``; HIP_VISIBLE_DEVICES is honoured by torch)."""
    try:
        import torch
    except ImportError:
        if device_spec == "cuda" or device_spec.startswith("cuda:"):
            return device_spec
        raise ValueError("--device must name a GPU device (for example cuda or cuda:1)")
    device = torch.device(device_spec)
    if device.type != "cuda":
        raise ValueError("--device must name a GPU device (for example cuda or cuda:1)")
    if not torch.cuda.is_available():
        return device_spec
    index = torch.cuda.current_device() if device.index is None else device.index
    count = torch.cuda.device_count()
    if not 0 <= index < count:
        raise ValueError(f"--device selects logical GPU {index}, but only {count} device(s) are visible")
    torch.cuda.set_device(index)
    return f"cuda:{index}"


def configure_torch_matmul(input_precision: str) -> None:
    """Align torch's fp32 matmul policy with the kernels' ``input_precision``."""
    try:
        import torch
    except ImportError:
        return
    tf32 = input_precision == "tf32"
    torch.backends.cuda.matmul.allow_tf32 = tf32
    torch.set_float32_matmul_precision("high" if tf32 else "highest")


def dtype_supported(name: str) -> tuple[bool, str]:
    """Probe a dtype with a real device matmul."""
    try:
        import torch

        if not torch.cuda.is_available():
            return False, "GPU unavailable"
        x = torch.ones((16, 16), device="cuda", dtype=torch_dtype(name))
        y = torch.mm(x, x)
        torch.cuda.synchronize()
        if not bool(torch.isfinite(y).all().item()):
            return False, f"{name} device matmul produced non-finite output"
        return True, ""
    except Exception as exc:  # pragma: no cover - exercised only on broken stacks
        return False, f"{name} device matmul probe failed: {exc!r}"


def percentile(values: Sequence[float], q: float) -> float:
    """Linear-interpolated percentile, q in [0, 1]."""
    ordered = sorted(values)
    if not ordered:
        return math.nan
    position = (len(ordered) - 1) * q
    low = math.floor(position)
    high = math.ceil(position)
    if low == high:
        return ordered[low]
    return ordered[low] + (ordered[high] - ordered[low]) * (position - low)


def _whole_ring_count(requested: int, minimum: int, workspace_count: int) -> int:
    """Smallest multiple of ``workspace_count`` that is >= max(requested, minimum)."""
    needed = max(requested, minimum)
    return -(-needed // workspace_count) * workspace_count


# Shortest device time of one timed replay.  A replay this long also outlasts the host's
# submission of the next (event, replay, event) triple, so the device never idles inside a sample.
_MIN_SAMPLE_MS = 0.5


def _capture_calls(function: Callable[[int], None], count: int, workspace_count: int, stream):
    """Capture ``count`` consecutive calls (cycling through the ring) into one graph."""
    import torch

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for index in range(count):
            function(index % workspace_count)
    return graph


def _replay_samples(graph, calls_per_replay: int, samples: int, stream) -> list[float]:
    """Per-call milliseconds of ``samples`` timed replays, each the replay time / calls.

    One untimed lead replay runs first; every timed replay is bracketed by ordinary events
    recorded on the replay stream.  (ROCm torch forbids external events inside a capture, so
    per-call event nodes are not available; the graph holds only the calls themselves.)
    """
    import torch

    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(samples)]
    with torch.cuda.stream(stream):
        graph.replay()
        for start, end in pairs:
            start.record(stream)
            graph.replay()
            end.record(stream)
    stream.synchronize()
    return [start.elapsed_time(end) / calls_per_replay for start, end in pairs]


def time_cuda(
    function: Callable[[int], None],
    requested_warmup: int,
    requested_repeat: int,
    target_ms: float = 2000.0,
    *,
    workspace_count: int = 1,
) -> TimingResult:
    """Median/p20/p80 device time per call of ``function(index)``, measured from graph replays.

    The first call per workspace runs eagerly and untimed (autotuning, allocator warmup).  A
    pilot graph of one ring sizes the counts: warmup is capped towards 250 ms and repeat towards
    ``target_ms``, both rounded up to whole rings.  The measured calls are captured as a graph of
    ``chunk`` calls (whole rings, at least ~0.5 ms of device time) and replayed
    ``repeat / chunk`` times; each replay is one sample of the mean per-call time.  Host work done
    by ``function`` happens at capture time and never inside a sample.  Capture failures
    propagate: there is no eager timing fallback.
    """
    import torch

    if workspace_count < 1 or requested_warmup < 0 or requested_repeat < 1 or target_ms <= 0:
        raise ValueError("invalid graph timing counts or target")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for index in range(workspace_count):
            function(index)
    stream.synchronize()
    pilot = _capture_calls(function, workspace_count, workspace_count, stream)
    pilot_ms = max(statistics.median(_replay_samples(pilot, workspace_count, 3, stream)), 0.001)
    warmup = max(2, min(requested_warmup, int(max(2.0, 250.0 / pilot_ms))))
    repeat = max(3, min(requested_repeat, int(max(3.0, target_ms / pilot_ms))))
    warmup = _whole_ring_count(warmup, 2, workspace_count)
    repeat = _whole_ring_count(repeat, 3, workspace_count)
    with torch.cuda.stream(stream):
        for _ in range(warmup // workspace_count):
            pilot.replay()
    stream.synchronize()
    del pilot
    rings_per_chunk = max(1, math.ceil(_MIN_SAMPLE_MS / (pilot_ms * workspace_count)))
    chunk = min(repeat, rings_per_chunk * workspace_count)
    samples = max(1, math.ceil(repeat / chunk))
    repeat = samples * chunk
    graph = _capture_calls(function, chunk, workspace_count, stream)
    per_call = _replay_samples(graph, chunk, samples, stream)
    return TimingResult(
        p20_ms=percentile(per_call, 0.2),
        median_ms=statistics.median(per_call),
        p80_ms=percentile(per_call, 0.8),
        mean_ms=statistics.mean(per_call),
        std_ms=statistics.pstdev(per_call),
        warmup=warmup,
        repeat=repeat,
    )


def tune_rotating_configs(
    configs: Sequence[ConfigT],
    launch: Callable[[ConfigT, int], None],
    workspace_count: int,
    repeats_per_workspace: int = 2,
) -> TuningResult:
    """Pick the fastest fixed config while rotating through every resident workspace."""
    import torch

    if not configs:
        raise ValueError("at least one tuning config is required")
    if workspace_count < 2:
        raise ValueError("rotating autotune requires at least two workspaces")
    samples = max(3, workspace_count * max(1, repeats_per_workspace))
    best, best_ms, tested, failed = None, math.inf, 0, 0
    for config in configs:
        try:
            timing = time_cuda(lambda index, cfg=config: launch(cfg, index), 2, samples, workspace_count=workspace_count)
        except (RuntimeError, AssertionError):
            failed += 1
            torch.cuda.synchronize()
            continue
        tested += 1
        if timing.median_ms < best_ms:
            best, best_ms = config, timing.median_ms
    if best is None:
        raise RuntimeError(f"all {len(configs)} rotating-autotune candidates failed")
    return TuningResult(best, best_ms, tested, failed)


def hot_autotune_bench(function: Callable[[], None], quantiles):
    """Bounded hot timing (9 samples, 25 ms target) returning the requested quantiles."""
    timing = time_cuda(lambda _index: function(), 2, 9, target_ms=25.0)
    by_quantile = {0.2: timing.p20_ms, 0.5: timing.median_ms, 0.8: timing.p80_ms}
    return [by_quantile[q] for q in quantiles]


def assert_close(actual, reference, dtype_name: str) -> tuple[float, float]:
    """torch.testing.assert_close with the per-dtype tolerances; returns (max_abs, max_rel)."""
    import torch

    diff = (actual.float() - reference.float()).abs()
    if diff.numel():
        max_abs = float(diff.max().item())
        max_rel = float((diff / reference.float().abs().clamp_min(1e-6)).max().item())
    else:
        max_abs = max_rel = 0.0
    rtol, atol = TOLERANCES[dtype_name]
    torch.testing.assert_close(actual, reference, rtol=rtol, atol=atol)
    return max_abs, max_rel


def normwise_relative_error(actual, reference) -> float:
    """max|actual - reference| / max|reference| (0 when the reference is all zero)."""
    diff = (actual.double() - reference.double()).abs()
    scale = float(reference.double().abs().max().item()) if reference.numel() else 0.0
    err = float(diff.max().item()) if diff.numel() else 0.0
    return err / scale if scale > 0 else err


def available_budget(memory_fraction: float) -> int:
    """Bytes a case may allocate: free device memory * fraction, minus 256 MiB headroom."""
    import torch

    free, _total = torch.cuda.mem_get_info()
    return max(0, int(free * memory_fraction) - (256 << 20))
