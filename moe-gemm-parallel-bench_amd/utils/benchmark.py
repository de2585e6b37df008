"""Device timing, tuning, dtype, memory and correctness helpers on ROCm.

These names form the helper surface that the reference's drivers import from utils/benchmark.py
(reference utils/benchmark.py:13-278): the timing record, the graph timer, the rotating-ring
tuner, the hot timer behind the launchers' autotuner, dtype/device helpers, the memory budget and
the per-dtype closeness check.  The implementations are this project's own:
  * ``time_cuda`` measures device time from hipGraph replays of chunks of whole workspace rings
    (ROCm torch refuses external events inside a capture, so the reference's per-call event
    nodes are not available); counts are capped towards a 250 ms warm-up and ``target_ms`` of
    measurement and rounded up to whole rings;
  * ``tune_rotating_configs`` times every candidate across the complete rotating ring and keeps
    the lowest median; a candidate that cannot launch is counted as failed and skipped;
  * ``assert_close`` applies the reference's per-dtype (rtol, atol) and reports max abs / rel.
"""

from __future__ import annotations

import math
import statistics
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import TypeVar

import numpy as np

TIMING_METHOD = "hip_graph_replay_events"
ConfigT = TypeVar("ConfigT")

# name -> (torch dtype attribute, bytes per element, (rtol, atol) of assert_close).  The
# tolerances are the reference's result contract (utils/benchmark.py:268).
_DTYPE_TABLE = {
    "fp16": ("float16", 2, (2e-2, 2e-2)),
    "bf16": ("bfloat16", 2, (5e-2, 5e-2)),
    "fp32": ("float32", 4, (2e-3, 2e-3)),
}
TOLERANCES = {name: entry[2] for name, entry in _DTYPE_TABLE.items()}
_HEADROOM_BYTES = 256 << 20


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


def _dtype_entry(name: str):
    try:
        return _DTYPE_TABLE[name]
    except KeyError:
        raise ValueError(f"unknown dtype name {name!r}; expected one of {sorted(_DTYPE_TABLE)}") from None


def torch_dtype(name: str):
    import torch

    return getattr(torch, _dtype_entry(name)[0])


def dtype_size(name: str) -> int:
    return _dtype_entry(name)[1]


def select_cuda_device(device_spec: str) -> str:
    """Make one logical GPU current and return it as ``cuda:N``.

    ROCm torch names HIP devices ``cuda``; the index is logical within HIP_VISIBLE_DEVICES /
    ROCR_VISIBLE_DEVICES, exactly as torch enumerates them.
    """
    kind, _, index_text = device_spec.partition(":")
    if kind != "cuda" or (index_text and not index_text.isdigit()):
        raise ValueError("--device must name a GPU device (for example cuda or cuda:1)")
    try:
        import torch
    except ImportError:
        return device_spec
    if not torch.cuda.is_available():
        return device_spec
    visible = torch.cuda.device_count()
    index = int(index_text) if index_text else torch.cuda.current_device()
    if index >= visible:
        raise ValueError(f"--device selects logical GPU {index}, but only {visible} device(s) are visible")
    torch.cuda.set_device(index)
    return f"cuda:{index}"


def configure_torch_matmul(input_precision: str) -> None:
    """Give torch's fp32 matmuls (the correctness references) the kernels' input precision."""
    try:
        import torch
    except ImportError:
        return
    if input_precision not in ("ieee", "tf32"):
        raise ValueError(f"input_precision must be 'ieee' or 'tf32', got {input_precision!r}")
    torch.backends.cuda.matmul.allow_tf32 = input_precision == "tf32"
    torch.set_float32_matmul_precision({"ieee": "highest", "tf32": "high"}[input_precision])


def dtype_supported(name: str) -> tuple[bool, str]:
    """(supported, reason): run a small device matmul in the dtype and check it is finite."""
    try:
        import torch
    except ImportError:
        return False, "PyTorch unavailable"
    if not torch.cuda.is_available():
        return False, "GPU unavailable"
    try:
        probe = torch.full((16, 16), 0.5, device="cuda", dtype=torch_dtype(name))
        finite = bool(torch.isfinite(probe @ probe).all().item())
    except Exception as exc:  # noqa: BLE001 - any failure means "not usable"
        return False, f"{name} device matmul probe failed: {exc!r}"
    return (True, "") if finite else (False, f"{name} device matmul produced non-finite output")


def percentile(values: Sequence[float], q: float) -> float:
    """Linear-interpolation percentile for q in [0, 1] (numpy's default method); NaN when empty."""
    if len(values) == 0:
        return math.nan
    return float(np.percentile(np.asarray(values, dtype=np.float64), 100.0 * q))


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
    """Choose one fixed config by timing each candidate across the whole rotating ring.

    Each candidate gets the same graph timing as the measurement itself (``time_cuda`` over
    ``workspace_count`` buffers, at least three and ``repeats_per_workspace`` visits per buffer),
    so the choice reflects the cold-ring access pattern.  Candidates whose launch raises
    (``RuntimeError``, ``ValueError`` for an unusable tile, ``AssertionError``) are counted and
    skipped; if none survives, RuntimeError.
    """
    import torch

    if not configs:
        raise ValueError("at least one tuning config is required")
    if workspace_count < 2:
        raise ValueError("rotating autotune requires at least two workspaces")
    samples = max(3, workspace_count * max(1, repeats_per_workspace))
    medians: list[tuple[float, int]] = []
    failed = 0
    for position, config in enumerate(configs):
        try:
            median = time_cuda(lambda index, cfg=config: launch(cfg, index), 2, samples,
                               workspace_count=workspace_count).median_ms
        except (RuntimeError, ValueError, AssertionError):
            failed += 1
            torch.cuda.synchronize()
            continue
        medians.append((median, position))
    if not medians:
        raise RuntimeError(f"all {len(configs)} rotating-autotune candidates failed")
    best_ms, best_position = min(medians)
    return TuningResult(configs[best_position], best_ms, len(medians), failed)


def hot_autotune_bench(function: Callable[[], None], quantiles):
    """Bounded hot timing of one launch closure (9 samples, ~25 ms) at the given quantiles."""
    timing = time_cuda(lambda _index: function(), 2, 9, target_ms=25.0)
    by_quantile = {0.2: timing.p20_ms, 0.5: timing.median_ms, 0.8: timing.p80_ms}
    return [by_quantile.get(q, math.nan) for q in quantiles]


def assert_close(actual, reference, dtype_name: str) -> tuple[float, float]:
    """Raise AssertionError unless ``actual`` is within the dtype's (rtol, atol) of ``reference``.

    Returns (max absolute error, max relative error with the denominator clamped at 1e-6).
    """
    import torch

    rtol, atol = _dtype_entry(dtype_name)[2]
    got, want = actual.float(), reference.float()
    if got.numel() == 0:
        torch.testing.assert_close(actual, reference, rtol=rtol, atol=atol)
        return 0.0, 0.0
    error = (got - want).abs()
    max_abs = float(error.max().item())
    max_rel = float((error / want.abs().clamp_min(1e-6)).max().item())
    torch.testing.assert_close(actual, reference, rtol=rtol, atol=atol)
    return max_abs, max_rel


def normwise_relative_error(actual, reference) -> float:
    """max|actual - reference| / max|reference| (0 when the reference is all zero)."""
    diff = (actual.double() - reference.double()).abs()
    scale = float(reference.double().abs().max().item()) if reference.numel() else 0.0
    err = float(diff.max().item()) if diff.numel() else 0.0
    return err / scale if scale > 0 else err


def available_budget(memory_fraction: float) -> int:
    """Bytes one case may allocate: the device's free memory times ``memory_fraction``, less a
    256 MiB reserve for the library workspaces and the allocator."""
    import torch

    free_bytes, _total = torch.cuda.mem_get_info()
    return max(0, int(free_bytes * memory_fraction) - _HEADROOM_BYTES)
