"""``python -m harness.power``: sustained throughput next to board power and clock (amd-smi).

A GEMM that holds the board at its power cap runs at whatever clock the cap allows, so its rate
says as much about energy per FLOP as about its schedule.  Each workload runs back to back for
``--seconds`` while a thread samples ``amd-smi metric --power --clock``; the first ``--skip``
seconds (the power controller's boost and throttle transient) are dropped, and the table reports
per workload: microseconds per launch, TFLOP/s, mean SOCKET_POWER and mean GFX clock over XCDs.

Workloads (bf16, seeded inputs):

* ``grouped``: DSV3 EP W13 at M_e=512, 32 x [512,7168]@[7168,4096] (the bench.py headline);
* ``single``: one [16384,7168]@[7168,4096] GEMM with the same FLOPs, this project's kernel;
* ``hipblaslt``: the same single GEMM through ``torch.mm`` (hipBLASLt on ROCm);
* ``hipblaslt_batched``: the grouped workload itself through one ``torch.bmm`` on contiguous
  [32, 512, 7168] and [32, 7168, 4096] operands (hipBLASLt's batched GEMM: the same 32 B matrices
  and HBM bytes as ``grouped``);
* ``decode``: DSV3 EP W13 at M_e=8, 32 x [8,7168]@[7168,4096] (HBM-bound; its rate is reported in
  TFLOP/s like the others, and its bytes per launch are 2 B x 32 x (8*7168 + 7168*4096 + 8*4096)).

This project's launches use the autotuned config unless ``--kernel-config`` pins one.
"""

from __future__ import annotations

import argparse
import os
import re
import subprocess
import threading
import time

import torch

from kernels.grouped_gemm import build_grouped_workspace, launch_grouped
from kernels.matmul import KernelConfig, launch_matmul

WORKLOADS = ("grouped", "single", "hipblaslt", "hipblaslt_batched", "decode")
GROUPED_SHAPE = (512, 7168, 4096)  # (M_e, K, N) per expert
DECODE_SHAPE = (8, 7168, 4096)
EXPERTS = 32
SINGLE_SHAPE = (16384, 7168, 4096)


def parse_amd_smi(text: str) -> tuple[float | None, list[float]]:
    """SOCKET_POWER (W) and the GFX clock of every XCD (MHz) from ``amd-smi metric --power --clock``."""
    power = re.findall(r"SOCKET_POWER:\s*([\d.]+)", text)
    clocks = re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*([\d.]+)", text)
    return (float(power[0]) if power else None), [float(c) for c in clocks]


class Sampler:
    """Background amd-smi sampling; samples are (time, power, mean GFX clock)."""

    def __init__(self, every: float):
        self.every = every
        self.samples: list[tuple[float, float | None, float | None]] = []
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)

    def _run(self) -> None:
        # Under a profiler's preloaded library (rocprofv3) the tool would run under it too: no samples.
        if "rocprof" in os.environ.get("LD_PRELOAD", ""):
            return
        while not self._stop.is_set():
            try:
                out = subprocess.run(["amd-smi", "metric", "--power", "--clock"], capture_output=True,
                                     text=True, timeout=10, check=False).stdout
            except (OSError, subprocess.SubprocessError):
                return
            power, clocks = parse_amd_smi(out)
            self.samples.append((time.time(), power, sum(clocks) / len(clocks) if clocks else None))
            time.sleep(self.every)

    def start(self) -> "Sampler":
        self._thread.start()
        return self

    def stop(self) -> None:
        self._stop.set()

    def between(self, t0: float, t1: float) -> tuple[float | None, float | None, int]:
        window = [(p, c) for t, p, c in self.samples if t0 <= t <= t1]
        powers = [p for p, _ in window if p is not None]
        clocks = [c for _, c in window if c is not None]
        mean = lambda xs: sum(xs) / len(xs) if xs else None  # noqa: E731
        return mean(powers), mean(clocks), len(window)


def sustained(step, seconds: float, skip: float, chunk: int = 20) -> tuple[float, float, float]:
    """Mean ms per launch after `skip` seconds of back-to-back launches; returns (ms, t_skip, t_end)."""
    step()
    torch.cuda.synchronize()
    t0 = time.time()
    rates = []
    while time.time() < t0 + seconds:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(chunk):
            step()
        end.record()
        end.synchronize()
        rates.append((time.time(), start.elapsed_time(end) / chunk))
    late = [ms for t, ms in rates if t > t0 + skip] or [ms for _, ms in rates]  # all, if skip >= seconds
    return sum(late) / len(late), t0 + skip, time.time()


def parse_kernel_config(text: str | None) -> KernelConfig | None:
    """BM,BN,BK,WARPS,STAGES,GROUP_M,MULT (the bench.py --kernel-config order)."""
    if not text:
        return None
    bm, bn, bk, warps, stages, group_m, mult = (int(v) for v in text.split(","))
    return KernelConfig(bm, bn, bk, group_m, warps, stages, mult)


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(prog="python -m harness.power", description=__doc__.split("\n")[0])
    parser.add_argument("--seconds", type=float, default=8.0, help="back-to-back time per workload")
    parser.add_argument("--skip", type=float, default=3.0, help="leading seconds left out of every mean")
    parser.add_argument("--pause", type=float, default=3.0, help="idle seconds between workloads")
    parser.add_argument("--sample-every", type=float, default=0.2)
    parser.add_argument("--workloads", default="grouped,single,hipblaslt")
    parser.add_argument("--kernel-config", default=None, metavar="BM,BN,BK,WARPS,STAGES,GROUP_M,MULT")
    parser.add_argument("--b-stream", type=int, choices=(0, 1), default=None,
                        help="B copy policy of this project's launches (1 = non-temporal B copies); "
                             "default: the tuner's choice, or 0 with --kernel-config")
    args = parser.parse_args(argv)
    workloads = [w for w in args.workloads.split(",") if w]
    unknown = sorted(set(workloads) - set(WORKLOADS))
    if unknown:
        parser.error(f"unknown workloads {unknown}; choose from {WORKLOADS}")
    if not torch.cuda.is_available():
        parser.error("a ROCm GPU is required")
    pinned = parse_kernel_config(args.kernel_config)
    dtype = torch.bfloat16
    m, k, n = SINGLE_SHAPE
    flops = 2 * m * k * n
    assert flops == 2 * EXPERTS * GROUPED_SHAPE[0] * GROUPED_SHAPE[1] * GROUPED_SHAPE[2]

    steps = {}
    flops_of = {name: flops for name in WORKLOADS}
    if "decode" in workloads:
        dws = build_grouped_workspace([DECODE_SHAPE] * EXPERTS, dtype, seed=1234)
        flops_of["decode"] = 2 * EXPERTS * DECODE_SHAPE[0] * DECODE_SHAPE[1] * DECODE_SHAPE[2]
        if pinned is None:
            launch_grouped(dws, b_stream=args.b_stream)
            steps["decode"] = lambda: launch_grouped(dws, b_stream=args.b_stream)
        else:
            steps["decode"] = lambda: launch_grouped(dws, config=pinned, autotune=False, b_stream=args.b_stream)
    if "grouped" in workloads:
        ws = build_grouped_workspace([GROUPED_SHAPE] * EXPERTS, dtype, seed=1234)
        if pinned is None:
            launch_grouped(ws, b_stream=args.b_stream)  # autotune once, outside the measurement
            steps["grouped"] = lambda: launch_grouped(ws, b_stream=args.b_stream)
            print(f"grouped: autotuned {ws.config}, schedule {ws.tile_schedule}, b_stream {ws.b_stream}", flush=True)
        else:
            steps["grouped"] = lambda: launch_grouped(ws, config=pinned, autotune=False, b_stream=args.b_stream)
    if "hipblaslt_batched" in workloads:
        gen = torch.Generator(device="cuda").manual_seed(1234)
        gm, gk, gn = GROUPED_SHAPE
        a3 = (torch.randn(EXPERTS, gm, gk, device="cuda", generator=gen) * 0.1).to(dtype)
        b3 = (torch.randn(EXPERTS, gk, gn, device="cuda", generator=gen) * 0.1).to(dtype)  # contiguous, not a view
        c3 = torch.empty(EXPERTS, gm, gn, device="cuda", dtype=dtype)
        steps["hipblaslt_batched"] = lambda: torch.bmm(a3, b3, out=c3)
    if "single" in workloads or "hipblaslt" in workloads:
        gen = torch.Generator(device="cuda").manual_seed(1234)
        a = (torch.randn(m, k, device="cuda", generator=gen) * 0.1).to(dtype)
        b = (torch.randn(k, n, device="cuda", generator=gen) * 0.1).to(dtype)
        c = torch.empty(m, n, device="cuda", dtype=dtype)
        if "single" in workloads:
            if pinned is None:
                launch_matmul(a, b, c, b_stream=args.b_stream)
                steps["single"] = lambda: launch_matmul(a, b, c, b_stream=args.b_stream)
            else:
                steps["single"] = lambda: launch_matmul(a, b, c, config=pinned, autotune=False,
                                                        b_stream=args.b_stream)
        if "hipblaslt" in workloads:
            steps["hipblaslt"] = lambda: torch.mm(a, b, out=c)

    sampler = Sampler(args.sample_every).start()
    time.sleep(1.0)
    print("| workload | us per launch | TFLOP/s | SOCKET_POWER W | GFX clock MHz (mean of XCDs) | samples |")
    print("|---|---|---|---|---|---|")
    for name in workloads:
        ms, t_skip, t_end = sustained(steps[name], args.seconds, args.skip)
        power, clock, count = sampler.between(t_skip, t_end)
        fmt = lambda v: "n/a" if v is None else f"{v:.0f}"  # noqa: E731
        print(f"| {name} | {ms * 1e3:.1f} | {flops_of[name] / (ms * 1e9):.1f} | {fmt(power)} | {fmt(clock)} | {count} |",
              flush=True)
        time.sleep(args.pause)
    sampler.stop()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
