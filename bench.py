"""Headline benchmark: one MI355X, DeepSeek-V3 EP W13 (packed Gate+Up) grouped GEMM, M_e = 512, bf16.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

* Workload (one EP rank of BASELINE.json configs[2], the north-star target case): 32 experts of
  [512, 7168] @ [7168, 4096] in bf16 with fp32 accumulation, synthetic ``normal_() * 0.1`` inputs
  resident in HBM.  A step is one ``launch_grouped`` call over the whole group (one kernel launch).
* ``value`` is whole-job TFLOP/s = 2 * sum_e M_e*K*N / (time per step), from HIP events recorded on
  the launch stream around exactly K back-to-back steps (synchronised before and after).  Before
  the W warmup steps the step runs back to back for ``--settle-seconds`` (3 s): at its 1400 W cap
  the GPU boosts, then throttles below its steady clock for about a second of sustained load, and
  K steps timed straight after an idle period measure that transient.  ``cold_ms_per_step`` is
  the same K steps timed without the settle period, reported beside it.
* ``roofline`` prices that kernel against the dense bf16 MFMA peak (2.5 PFLOP/s); ``traffic`` is
  the measured HBM bytes per launch from profiles/ (rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by a
  copy-kernel calibration) or null when no such profile is committed.
* ``cases`` adds the HBM-bound M_e = 8 EP case, the TP counterparts (EP/TP ratio), the DSV3 W2
  cases, the headline with the SwiGLU activation fused into the epilogue (a labelled variant:
  the reference times W13 without the activation) and the headline's work under lognormal routing
  (rows around 512 and around 64 per expert) over the expert-sorted layout, timed under the static
  and the work-stealing tile schedule; each
  is timed the same way and checked against a float32 torch reference on a sample of experts.  The
  DSV3 cases time K/2 steps or, for short kernels, as many as make up 10 ms (``timed_steps``).
* ``cpu_baseline`` times the reference's own CPU torch path for the headline step on the host cores
  (per-expert ``torch.mm`` and ``F.grouped_mm`` over the padded offs layout; the faster is
  reported, with core count and CPU model); ``cpu_oracle_port`` adds the oracle's C GEMM.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path[:0] = [str(REPO / "moe-gemm-parallel-bench_amd"), str(REPO)]

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
METRIC = "grouped-GEMM TFLOP/s + % MFMA/HBM roofline, EP vs TP per-rank, 1 MI355X"

# DeepSeek-V3: H=7168, F=2048, E=256, topk=8, P=8.
DSV3 = dict(hidden=7168, ffn=2048, experts=256, parallel=8)
# The BASELINE.json models for `--case` runs (profiles): name -> (H, F, E, P, dtype name).
MODELS = {"dsv3": (7168, 2048, 256, 8, "bf16"), "mixtral": (4096, 14336, 8, 8, "bf16"),
          "qwen3": (2048, 768, 128, 4, "fp16")}


def _shapes(projection: str, parallel_type: str, m: int, model: str = "dsv3"):
    from utils.metrics import moe_shapes

    hidden, ffn, experts, parallel, _ = MODELS[model]
    return moe_shapes(projection, parallel_type, m, hidden, ffn, experts, parallel)


def _workspace(projection: str, parallel_type: str, m: int, seed: int, model: str = "dsv3"):
    import torch

    from kernels.grouped_gemm import build_fused_gate_up_workspace, build_grouped_workspace

    builder = build_fused_gate_up_workspace if projection == "W1" else build_grouped_workspace
    dtype = torch.float16 if MODELS[model][4] == "fp16" else torch.bfloat16
    return builder(_shapes(projection, parallel_type, m, model), dtype, seed)


def _normwise(c, ref) -> float:
    """max|C - R| / max|R|; infinite when C holds a NaN or infinity (e.g. an unwritten row)."""
    err = float((c.float() - ref).abs().max()) / float(ref.abs().max())
    return err if math.isfinite(err) else math.inf


def _check_sample(workspace, experts=(0, -1)) -> float:
    """Normwise error of sampled experts against a float32 torch product (GPU)."""
    worst = 0.0
    for index in experts:
        a, b, c = workspace.a[index], workspace.b[index], workspace.c[index]
        worst = max(worst, _normwise(c, a.float() @ b.float()))
    return worst


def _settle(step, seconds: float) -> None:
    """Run ``step`` back to back for ``seconds`` (untimed), keeping the queue non-empty.

    An MI355X held at its board power cap boosts at the start of a sustained load, then throttles
    past its steady clock and takes one to two seconds to settle (kernel traces show single
    dispatches of the headline 45 % slower than the steady state a few launches in); steps timed
    right after an idle period measure that transient rather than the sustained rate."""
    import torch

    if seconds <= 0:
        return
    deadline = time.perf_counter() + seconds
    previous = None
    while time.perf_counter() < deadline:
        for _ in range(8):
            step()
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream())
        if previous is not None:
            previous.synchronize()
        previous = event
    torch.cuda.synchronize()


def _timed(step, steps: int, warmup: int, settle_s: float = 0.0) -> tuple[float, float]:
    """(ms per step from HIP events on the launch stream, wall ms per step) over exactly ``steps``
    back-to-back steps, after the settle period and ``warmup`` untimed steps."""
    import torch

    _settle(step, settle_s)
    for _ in range(warmup):
        step()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - wall) * 1e3
    return start.elapsed_time(end) / steps, wall / steps


def _case(projection: str, parallel_type: str, m: int, steps: int, warmup: int, seed: int = 1234,
          pinned=None, model: str = "dsv3", settle_s: float = 0.0, b_stream=None,
          min_timed_ms: float = 0.0) -> dict:
    """Time one case of a BASELINE.json model (DSV3 by default); ``pinned`` (a KernelConfig) skips autotuning.

    ``b_stream`` pins the B copy policy (None: the tuner times both; with ``pinned``, 0).  The settled
    timing runs ``steps`` steps, or more when they would take under ``min_timed_ms``: the latency from
    the start event to the first kernel (some 0.1-0.2 ms) is spread over the timed steps, which for a
    0.2 ms kernel and 10 steps reads as 10 % slower launches."""
    import torch

    from kernels.grouped_gemm import launch_grouped
    from utils.metrics import gemm_bytes, gemm_flops

    workspace = _workspace(projection, parallel_type, m, seed, model)

    def step():
        launch_grouped(workspace, config=pinned, autotune=pinned is None, b_stream=b_stream)

    step()  # autotune (untimed) on a cache miss
    for c in workspace.c:
        c.fill_(float("nan"))
    step()
    torch.cuda.synchronize()
    error = _check_sample(workspace)

    cold_ms, _ = _timed(step, steps, warmup)  # straight after the idle check, no settle period
    timed_steps = max(steps, math.ceil(min_timed_ms / cold_ms)) if cold_ms > 0 else steps
    ms, wall_ms = _timed(step, timed_steps, warmup, settle_s)
    # Device time per launch from hipGraph replays (the reference's timing method): for kernels
    # shorter than the Python launch path the eager loop above measures the host, not the kernel.
    from utils.benchmark import time_cuda

    graph_ms = time_cuda(lambda _i: step(), warmup, max(steps, 20), 200.0).median_ms
    flops = sum(gemm_flops(*s) for s in workspace.shapes)
    nbytes = sum(gemm_bytes(*s, 2) for s in workspace.shapes)
    tflops = flops / (ms * 1e9)
    gbs = nbytes / (ms * 1e6)
    bound = "mfma" if flops / (PEAK_BF16_TFLOPS * 1e12) >= nbytes / (PEAK_HBM_GBS * 1e9) else "hbm"
    row = {
        "case": f"{model}_{projection.lower()}_{parallel_type.lower()}_me{m}",
        "experts": workspace.problem_count, "shape_mkn": list(workspace.shapes[0]),
        "ms": ms, "wall_ms": wall_ms, "cold_ms": cold_ms, "graph_ms": graph_ms, "settle_s": settle_s,
        "timed_steps": timed_steps,
        "tflops": tflops, "gbs": gbs, "bound": bound,
        "frac": tflops / PEAK_BF16_TFLOPS if bound == "mfma" else gbs / PEAK_HBM_GBS,
        "config": workspace.config.as_dict(), "scheduler": workspace.scheduler,
        "tile_schedule": workspace.tile_schedule, "split_k": workspace.split_k, "b_stream": workspace.b_stream,
        "normwise_error_sampled": error, "correct": bool(error <= (2e-3 if MODELS[model][4] == "fp16" else 1e-2)),
        "flops": flops, "ideal_bytes": nbytes,
    }
    del workspace
    torch.cuda.empty_cache()
    return row


def _swiglu_case(m: int, steps: int, warmup: int, seed: int = 1234, settle_s: float = 0.0) -> dict:
    """DSV3 EP W13 with the SwiGLU activation fused into the epilogue (labelled variant)."""
    import torch

    from kernels.grouped_gemm import launch_gate_up_swiglu
    from utils.metrics import gemm_flops

    workspace = _workspace("W1", "EP", m, seed)
    outputs = launch_gate_up_swiglu(workspace)  # autotune (untimed) on a cache miss
    for h in outputs:
        h.fill_(float("nan"))
    launch_gate_up_swiglu(workspace, workspace.swiglu_config, autotune=False)
    torch.cuda.synchronize()
    f = workspace.shapes[0][2] // 2
    worst = 0.0
    for index in (0, -1):
        a, b = workspace.a[index].float(), workspace.b[index].float()
        ref = torch.nn.functional.silu(a @ b[:, :f]) * (a @ b[:, f:])
        worst = max(worst, _normwise(outputs[index], ref))
    from kernels.grouped_gemm import launch_grouped

    cfg = workspace.swiglu_config

    def fused_step():
        launch_gate_up_swiglu(workspace)

    def plain_step():
        launch_grouped(workspace, config=cfg, autotune=False, split_k=1, tile_schedule="static",
                       b_stream=workspace.swiglu_b_stream)

    # SwiGLU and the plain W13 GEMM with the same tile, interleaved (three rounds each) after one
    # settle period, so the gap is measured under one clock state rather than against a case timed
    # minutes earlier.
    _settle(fused_step, settle_s)
    fused, plain = [], []
    for _ in range(3):
        fused.append(_timed(fused_step, steps, warmup)[0])
        plain.append(_timed(plain_step, steps, warmup)[0])
    ms, plain_ms = sorted(fused)[1], sorted(plain)[1]
    flops = sum(gemm_flops(*s) for s in workspace.shapes)
    nbytes = sum(2 * (mm * k + k * n + mm * n // 2) for mm, k, n in workspace.shapes)
    row = {
        "case": f"dsv3_w1_ep_me{m}_swiglu", "experts": workspace.problem_count,
        "shape_mkn": list(workspace.shapes[0]), "ms": ms, "tflops": flops / (ms * 1e9),
        "gbs": nbytes / (ms * 1e6), "bound": "mfma", "frac": flops / (ms * 1e9) / PEAK_BF16_TFLOPS,
        "config": workspace.swiglu_config.as_dict(), "scheduler": workspace.scheduler,
        "b_stream": workspace.swiglu_b_stream, "epilogue": "silu(gate)*up fused, H [M_e, F] stored",
        "plain_w13_ms_same_tile": plain_ms,
        "swiglu_over_plain": ms / plain_ms, "normwise_error_sampled": worst,
        "correct": bool(worst <= 1e-2), "flops": flops, "ideal_bytes": nbytes,
    }
    del workspace
    torch.cuda.empty_cache()
    return row


def _ragged_case(steps: int, warmup: int, seed: int = 1234, settle_s: float = 0.0, mean_rows: int = 512) -> dict:
    """DSV3 EP W13 over the expert-sorted layout with lognormal routing (32 experts, rows around
    ``mean_rows``, one empty and one single-row expert): each tile schedule timed with its own tuned
    config."""
    import numpy as np
    import torch

    from kernels.grouped_mm import build_offsets_workspace, grouped_mm, last_grouped_mm_b_stream, last_grouped_mm_config
    from utils.metrics import gemm_flops

    rng = np.random.default_rng(2024)
    sigma = 0.6
    sizes = [int(round(v)) for v in np.exp(rng.normal(math.log(mean_rows) - sigma * sigma / 2, sigma, size=32))]
    sizes[5], sizes[9] = 0, 1
    k, n = DSV3["hidden"], 2 * DSV3["ffn"]
    ws = build_offsets_workspace([(m, k, n) for m in sizes], torch.bfloat16, seed, operation="gate_up")
    flops = sum(gemm_flops(m, k, n) for m in sizes)
    name = "dsv3_w1_ep_lognormal_offsets" if mean_rows == 512 else f"dsv3_w1_ep_lognormal{mean_rows}_offsets"
    row = {"case": name, "experts": len(sizes), "rows": sum(sizes),
           "rows_min_max": [min(sizes), max(sizes)], "flops": flops, "schedules": {}}
    steps_by_schedule = {}
    for schedule in ("static", "stealing"):
        def step(schedule=schedule):
            grouped_mm(ws.mat_a, ws.mat_b, ws.offs, out=ws.output, tile_schedule=schedule)

        step()  # autotune (untimed) for this schedule
        steps_by_schedule[schedule] = (step, {**last_grouped_mm_config().as_dict(),
                                              "b_stream": last_grouped_mm_b_stream()})
    # One settle period, then the schedules interleaved (three rounds each, median), so both see
    # the same clock state.
    _settle(steps_by_schedule["static"][0], settle_s)
    rounds = {schedule: [] for schedule in steps_by_schedule}
    for _ in range(3):
        for schedule, (step, _) in steps_by_schedule.items():
            rounds[schedule].append(_timed(step, steps, warmup)[0])
    # Each schedule's own output is checked: C is NaN-filled, that schedule runs once, and three
    # experts are sampled against an fp32 torch product.
    for schedule, (step, config) in steps_by_schedule.items():
        ms = sorted(rounds[schedule])[1]
        ws.output.fill_(float("nan"))
        step()
        torch.cuda.synchronize()
        worst = 0.0
        begin = 0
        for e, m in enumerate(sizes):
            if e in (0, 13, 31) and m:
                a, b, c = ws.mat_a[begin:begin + m], ws.mat_b[e], ws.output[begin:begin + m]
                worst = max(worst, _normwise(c, a.float() @ b.float()))
            begin += m
        row["schedules"][schedule] = {"ms": ms, "tflops": flops / (ms * 1e9), "config": config,
                                      "normwise_error_sampled": worst, "correct": bool(worst <= 1e-2)}
    static, stealing = row["schedules"]["static"]["ms"], row["schedules"]["stealing"]["ms"]
    worst = max(v["normwise_error_sampled"] for v in row["schedules"].values())
    row.update(ms=min(static, stealing), tflops=flops / (min(static, stealing) * 1e9),
               stealing_speedup=static / stealing, normwise_error_sampled=worst,
               correct=all(v["correct"] for v in row["schedules"].values()))
    del ws
    torch.cuda.empty_cache()
    return row


def _mfma_busy_from_profiles(case: str):
    """MFMA busy fraction and GFX clock recorded by a committed rocprofv3 counter summary, if any."""
    path = REPO / "profiles" / f"{case}_mfma_busy.md"
    if not path.exists():
        return None
    text = path.read_text()
    busy = re.search(r"mfma_busy_frac:\s*([0-9.]+)", text)
    clock = re.search(r"gfx_clock_ghz:\s*([0-9.]+)", text)
    if not busy or not clock:
        return None
    return {"busy_frac": float(busy.group(1)), "gfx_clock_ghz": float(clock.group(1)),
            "source": f"profiles/{path.name}"}


def _traffic_from_profiles(case: str, b_stream: int = 0):
    """HBM bytes per launch recorded by a committed rocprofv3 counter summary, if any.

    A summary may give one figure per B copy policy (``traffic_bytes_per_launch_b_stream_1: ...``);
    the plain ``traffic_bytes_per_launch: ...`` line serves a policy without one."""
    path = REPO / "profiles" / f"{case}_hbm_traffic.md"
    if not path.exists():
        return None
    text = path.read_text()
    match = (re.search(rf"traffic_bytes_per_launch_b_stream_{b_stream}:\s*([0-9.eE+]+)", text)
             or re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text))
    return float(match.group(1)) if match else None


def _cpu_model() -> str:
    """CPU model name of the host (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_seconds(function, seconds_target: float, max_reps: int = 50) -> tuple[float, int]:
    """1 untimed warm-up call, then timed calls until ``seconds_target`` (at least 3); median."""
    function()
    times = []
    while len(times) < 3 or (sum(times) < seconds_target and len(times) < max_reps):
        t0 = time.perf_counter()
        function()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def _cpu_reference_path(seconds_per_method: float = 8.0) -> dict:
    """The reference's CPU torch path on the host cores, over the headline step itself.

    Step = the 32 DSV3 EP W13 expert products [512,7168]@[7168,4096] in bf16, timed two ways:
      * the per-expert ``torch.mm`` loop of the reference's correctness reference
        (benchmark_moe.py:258-266);
      * one ``torch.nn.functional.grouped_mm`` over the expert-sorted 2-D A / 3-D B / int32 offs
        layout with row strides padded to 16 bytes (kernels/torch_grouped_gemm.py:139-158, 162-174).
    Each is a median over whole steps; the faster is ``value``, both are reported.
    """
    import torch

    from kernels.torch_grouped_gemm import build_torch_grouped_workspace, launch_torch_grouped

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    experts, m, k, n = 32, 512, DSV3["hidden"], 2 * DSV3["ffn"]
    # The torch provider's own layout builder, on the host: padded 2-D A / 3-D B / int32 offs.
    workspace = build_torch_grouped_workspace([(m, k, n)] * experts, torch.bfloat16, seed=1234, device="cpu")
    flops = 2 * experts * m * k * n

    def per_expert_loop():
        for index in range(experts):
            torch.mm(workspace.mat_a[index * m:(index + 1) * m], workspace.mat_b[index])

    def grouped():
        launch_torch_grouped(workspace)

    loop_s, loop_reps = _median_seconds(per_expert_loop, seconds_per_method)
    rows = {"torch_mm_loop": {"value": flops / loop_s / 1e12, "reps": loop_reps, "seconds_per_step": loop_s}}
    try:
        grouped_s, grouped_reps = _median_seconds(grouped, seconds_per_method)
        rows["torch_grouped_mm"] = {"value": flops / grouped_s / 1e12, "reps": grouped_reps,
                                    "seconds_per_step": grouped_s}
    except RuntimeError as exc:  # a torch without a CPU grouped_mm kernel for this layout (incl. unavailable)
        rows["torch_grouped_mm"] = {"value": None, "error": str(exc)[:200]}
    best = max((r for r in rows.values() if r.get("value")), key=lambda r: r["value"])
    best_name = next(name for name, r in rows.items() if r is best)
    return {
        "value": best["value"],
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "reference",
        "cpu_model": _cpu_model(),
        "method": best_name,
        "methods": rows,
        "sample": f"the whole headline step (32 x [512,7168]@[7168,4096] bf16, {flops / 1e9:.1f} GFLOP) per "
                  f"timed call, median of >=3 calls (~{seconds_per_method:.0f} s per method); the reference's "
                  "own CPU torch computation (per-expert torch.mm and F.grouped_mm on the 16-byte padded "
                  "2-D/3-D + offs layout), torch.set_num_threads(cores)",
    }


def _cpu_oracle_port(seconds_target: float = 5.0) -> dict:
    """Extra: the oracle's blocked OpenMP fp32-accumulating C GEMM on the same host cores."""
    import numpy as np

    from oracle import oracle

    threads = len(os.sched_getaffinity(0))
    m, k, n = 512, DSV3["hidden"], 2 * DSV3["ffn"]
    rng = np.random.default_rng(1234)

    def bf16(shape):
        return oracle.to_bf16_bits(rng.standard_normal(shape, dtype=np.float32) * 0.1)

    a = bf16((m, k))
    cols = 256
    b = bf16((k, cols))
    oracle.gemm_fast_bf16(a[:16], b, threads)  # warm (thread pool, pages)
    done_flops, elapsed, slices = 0, 0.0, 0
    while elapsed < seconds_target and slices < 4096:
        t0 = time.perf_counter()
        oracle.gemm_fast_bf16(a, b, threads)
        elapsed += time.perf_counter() - t0
        done_flops += 2 * m * k * cols
        slices += 1
    return {
        "value": done_flops / elapsed / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"{slices} x [512,7168]@[7168,{cols}] bf16 slices ({elapsed:.1f} s)",
    }


def _progress(row: dict) -> dict:
    """One line per finished case on stderr (stdout carries only the JSON result line)."""
    print(f"bench: {row['case']} {row['ms'] * 1e3:.1f} us per step", file=sys.stderr, flush=True)
    return row


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--settle-seconds", type=float, default=3.0,
                        help="untimed back-to-back steps before the warmup steps, so the timed steps see "
                             "the power manager's steady state (the cases use half); 0 disables")
    parser.add_argument("--no-cases", action="store_true", help="only the headline case")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--kernel-config", metavar="BM,BN,BK,WARPS,STAGES,GROUP_M,MULT", default=None,
                        help="pin the headline kernel config instead of autotuning (counter passes)")
    parser.add_argument("--b-stream", type=int, choices=(0, 1), default=None,
                        help="pin the headline's B copy policy (1 non-temporal); with --kernel-config the "
                             "default is 0, else the tuner times both")
    parser.add_argument("--case", metavar="PROJ,PAR,M", default=None,
                        help="only time one case (e.g. W1,EP,8) of --model, print its row and exit (profiling); "
                             "--kernel-config pins its kernel")
    parser.add_argument("--model", choices=sorted(MODELS), default="dsv3", help="model of a --case run")
    parser.add_argument("--copy-calibration", type=int, metavar="MIB", default=0,
                        help="only run a plain device copy of MIB MiB (HBM counter calibration) and exit")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (every GPU box here has "
              "one GPU); run with --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0 or args.settle_seconds < 0:
        raise SystemExit("--steps must be >= 1, --warmup and --settle-seconds >= 0")
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm GPU")
    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.empty(args.copy_calibration << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel(), "launches": args.steps}))
        return 0
    pinned = None
    if args.kernel_config:
        from kernels.matmul import KernelConfig

        bm, bn, bk, warps, stages, group, mult = (int(v) for v in args.kernel_config.split(","))
        pinned = KernelConfig(bm, bn, bk, group, warps, stages, mult)
    if args.case:
        projection, parallel_type, m = args.case.split(",")
        if projection not in ("W1", "W2") or parallel_type not in ("EP", "TP"):
            raise SystemExit("--case takes PROJ,PAR,M with PROJ in W1/W2 and PAR in EP/TP")
        row = _case(projection, parallel_type, int(m), args.steps, args.warmup, pinned=pinned, model=args.model,
                    settle_s=args.settle_seconds, b_stream=args.b_stream)
        print(json.dumps(row))
        return 0 if row["correct"] else 1
    headline = _case("W1", "EP", 512, args.steps, args.warmup, pinned=pinned, settle_s=args.settle_seconds,
                     b_stream=args.b_stream)
    _progress(headline)
    case_settle = args.settle_seconds / 2
    cases = []
    if not args.no_cases:
        for projection, parallel_type, m in (("W1", "EP", 8), ("W1", "TP", 512), ("W1", "TP", 8),
                                            ("W2", "EP", 512), ("W2", "TP", 512), ("W2", "EP", 8),
                                            ("W2", "TP", 8)):
            cases.append(_progress(_case(projection, parallel_type, m, max(5, args.steps // 2), 2,
                                         settle_s=case_settle, min_timed_ms=10.0)))
        cases.append(_progress(_swiglu_case(512, max(5, args.steps // 2), 2, settle_s=case_settle)))
        for mean_rows in (512, 64):
            cases.append(_progress(_ragged_case(max(5, args.steps // 2), 2, settle_s=case_settle, mean_rows=mean_rows)))
    traffic = _traffic_from_profiles(headline["case"], headline["b_stream"])
    tp = next((c for c in cases if c["case"] == "dsv3_w1_tp_me512"), None)
    by_case = {c["case"]: c for c in cases + [headline]}
    # TP TFLOP/s over EP TFLOP/s at equal per-rank FLOPs (the reference's EP/TP comparison).
    ep_tp = {}
    for projection in ("w1", "w2"):
        for m in (8, 512):
            ep, tp_case = by_case.get(f"dsv3_{projection}_ep_me{m}"), by_case.get(f"dsv3_{projection}_tp_me{m}")
            if ep and tp_case:
                ep_tp[f"{'w13' if projection == 'w1' else 'w2'}_me{m}"] = tp_case["tflops"] / ep["tflops"]
    line = {
        "metric": METRIC,
        "value": headline["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": headline["ms"],
        "settle_s": args.settle_seconds,
        "cold_ms_per_step": headline["cold_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic normal*0.1 inputs and weights (no checkpoints), resident in HBM",
        "config": {
            "workload": "DeepSeek-V3 EP rank, W13 packed Gate+Up, 32 experts x [512,7168]@[7168,4096], bf16, fp32 acc",
            "model": "deepseek-v3 expert shapes (H=7168, F=2048, E=256, topk=8, P=8)",
            "tokens_per_expert": 512, "global_batch": 32 * 512, "seq_len": None, "parallelism": "ep8 (one rank)",
            "kernel_config": headline["config"], "scheduler": headline["scheduler"],
            "tile_schedule": headline["tile_schedule"], "b_stream": headline["b_stream"],
        },
        "roofline": {
            "bound": "mfma", "achieved": headline["tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": headline["tflops"] / PEAK_BF16_TFLOPS, "traffic": traffic,
        },
        "mfma_counters": _mfma_busy_from_profiles(headline["case"]),
        "correct": headline["correct"],
        "normwise_error_sampled": headline["normwise_error_sampled"],
        "ep_tp_ratio_w13_me512": (tp["tflops"] / headline["tflops"]) if tp else None,
        "ep_tp_ratios": ep_tp,
        "cases": cases,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = _cpu_reference_path()
        line["cpu_oracle_port"] = _cpu_oracle_port()
    print(json.dumps(line))
    return 0 if headline["correct"] and all(c["correct"] for c in cases) else 1


if __name__ == "__main__":
    raise SystemExit(main())
