"""Run provenance (``environment.json``) on ROCm; importable without torch, a GPU or ROCm tools.

``collect_environment()`` / ``write_environment(path, extra)`` are the names the reference's
drivers import (reference utils/hardware.py:22-132).  Here the record is assembled from a list of
independent probes, each contributing a group of keys and none able to stop the others (a probe
that raises is recorded under ``probe_errors``):

* host      - Python, OS, CPU model and usable cores;
* runtime   - torch and its HIP runtime version (``cuda_version`` holds the HIP version: the CSV
              column keeps the reference's name);
* device    - the current device from torch: name, gfx architecture, compute units
              (``sm_count``), memory, and a finite 16 x 16 matmul per dtype;
* driver    - ``amd-smi version`` (driver / ROCm / amd-smi versions) and ``amd-smi static``'s
              board name when the tool answers;
* kernels   - the native library: its ABI version (``triton_version`` holds
              ``libmoegemm-abi<N>``: the kernel stack's identifier in the reference's column)
              and the number of compiled kernels per dtype.
"""

from __future__ import annotations

import json
import os
import platform
import re
import subprocess
import sys
from datetime import datetime, timezone
from pathlib import Path
from typing import Any


def _run(args: list[str]) -> str | None:
    """stdout of a short tool call, or None when the tool is absent, fails or hangs.  Skipped under a
    profiler's preloaded library (rocprofv3): the child would load it too, and profiling the tool
    is not wanted."""
    if "rocprof" in os.environ.get("LD_PRELOAD", ""):
        return None
    try:
        done = subprocess.run(args, capture_output=True, text=True, timeout=15, check=False)
    except (OSError, subprocess.SubprocessError):
        return None
    return done.stdout.strip() if done.returncode == 0 and done.stdout.strip() else None


def _host() -> dict[str, Any]:
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"python_version": platform.python_version(), "platform": platform.platform(),
            "host_cpu_model": model, "host_cpu_cores": cores}


def _runtime() -> dict[str, Any]:
    import torch

    return {"torch_version": torch.__version__, "cuda_version": getattr(torch.version, "hip", None),
            "hip_runtime_version": getattr(torch.version, "hip", None)}


def _device() -> dict[str, Any]:
    import torch

    if not torch.cuda.is_available():
        return {"gpu_available": False, "gpu_name": "unavailable"}
    index = torch.cuda.current_device()
    props = torch.cuda.get_device_properties(index)
    free, total = torch.cuda.mem_get_info(index)
    arch = str(getattr(props, "gcnArchName", "")).split(":")[0] or None
    probes = {}
    for name, dtype in (("fp16", torch.float16), ("bf16", torch.bfloat16), ("fp32", torch.float32)):
        try:
            square = torch.full((16, 16), 0.25, device="cuda", dtype=dtype)
            product = square @ square
            probes[name] = {"torch_matmul_ok": True, "result_dtype": str(product.dtype),
                            "finite": bool(torch.isfinite(product).all().item())}
        except Exception as exc:  # noqa: BLE001 - recorded, not raised
            probes[name] = {"torch_matmul_ok": False, "error": repr(exc)}
    return {
        "gpu_available": True,
        "gpu_name": props.name,
        "logical_cuda_device": f"cuda:{index}",
        "gfx_arch": arch,
        "compute_capability": f"{props.major}.{props.minor}",
        "sm_count": int(props.multi_processor_count),
        "total_memory_bytes": int(props.total_memory),
        "runtime_total_memory_bytes": int(total),
        "free_memory_bytes": int(free),
        "matrix_core_capability": "CDNA4 MFMA (fp16/bf16/fp8/fp6/fp4)" if arch == "gfx950" else "MFMA",
        "dtype_probes": probes,
        "fp16_supported": probes["fp16"].get("torch_matmul_ok", False),
        "bf16_supported": probes["bf16"].get("torch_matmul_ok", False),
        "fp32_supported": probes["fp32"].get("torch_matmul_ok", False),
        "tf32_supported": False,  # gfx950 has no XF32 MFMA; the library emulates TF32 by rounding
    }


def _driver() -> dict[str, Any]:
    out: dict[str, Any] = {}
    version = _run(["amd-smi", "version"])
    if version:
        for key, pattern in (("amdgpu_driver_version", r"amdgpu version:\s*([^|\s]+)"),
                             ("rocm_version", r"ROCm version:\s*([^|\s]+)"),
                             ("amd_smi_version", r"AMDSMI Tool:\s*([^|\s]+)")):
            match = re.search(pattern, version)
            if match:
                out[key] = match.group(1)
    static = _run(["amd-smi", "static", "--asic", "--json"])
    if static:
        try:
            parsed = json.loads(static)
            first = parsed[0] if isinstance(parsed, list) and parsed else parsed.get("gpu_data", [{}])[0]
            asic = first.get("asic", {})
            out["asic_market_name"] = asic.get("market_name")
            out["asic_target_graphics_version"] = asic.get("target_graphics_version")
        except (ValueError, AttributeError, IndexError, KeyError):
            pass
    return out


def _kernels() -> dict[str, Any]:
    from kernels import _native

    if not _native.available():
        return {"triton_version": None, "kernel_library": "libmoegemm unavailable"}
    lib = _native.library()
    counts = {name: int(lib.moegemm_kernel_count(code)) for code, name in _native.DTYPE_NAMES.items()}
    return {"triton_version": f"libmoegemm-abi{_native.ABI_VERSION}",
            "kernel_library": str(_native.LIBRARY_PATH.name), "compiled_kernels": counts}


_PROBES = (_host, _runtime, _device, _driver, _kernels)


def collect_environment() -> dict[str, Any]:
    env: dict[str, Any] = {
        "timestamp": datetime.now(timezone.utc).isoformat(),
        "gpu_available": False,
        "gpu_name": "unavailable",
        "cuda_version": None,
        "torch_version": None,
        "triton_version": None,
        "sm_count": None,
    }
    for probe in _PROBES:
        try:
            env.update(probe())
        except Exception as exc:  # noqa: BLE001 - one failed probe must not hide the others
            env.setdefault("probe_errors", {})[probe.__name__.lstrip("_")] = repr(exc)
    env["python_executable"] = Path(sys.executable).name
    return env


def write_environment(path: str | Path, extra: dict[str, Any] | None = None) -> dict[str, Any]:
    """Collect, merge ``extra`` over it, write it as JSON to ``path`` and return it."""
    env = {**collect_environment(), **(extra or {})}
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(env, indent=2, sort_keys=True, ensure_ascii=False) + "\n", encoding="utf-8")
    return env
