"""ROCm environment provenance for ``environment.json`` (importable without torch or a GPU).

Fills the same keys as the reference's utils/hardware.py:22-122 so downstream readers work
unchanged, from ROCm sources: torch's device properties (name, gfx arch, CU count, memory),
``torch.version.hip`` for the runtime, ``amd-smi``/``rocm-smi`` for the driver, a real 16x16
matmul per dtype, and the native library's ABI for the kernel stack.  ``sm_count`` is the
compute-unit count (256 on MI355X); ``compute_capability`` is torch's major.minor (9.5 on gfx950).
"""

from __future__ import annotations

import json
import platform
import re
import subprocess
import sys
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

_MATRIX_CORES = {
    "gfx950": "CDNA4 matrix cores (FP16/BF16/FP8/FP6/FP4 MFMA; no XF32)",
    "gfx942": "CDNA3 matrix cores (FP16/BF16/FP8/XF32 MFMA)",
    "gfx90a": "CDNA2 matrix cores (FP16/BF16 MFMA)",
}


def _command(args: list[str]) -> str | None:
    try:
        return subprocess.check_output(args, text=True, stderr=subprocess.STDOUT, timeout=10).strip()
    except Exception:
        return None


def _driver_version() -> str | None:
    text = _command(["amd-smi", "version"]) or _command(["rocm-smi", "--showdriverversion"])
    if not text:
        return None
    match = re.search(r"(?:amdgpu version|Driver version)\s*:?\s*([\w.\-]+)", text, re.I)
    return match.group(1) if match else text.splitlines()[0][:120]


def collect_environment() -> dict[str, Any]:
    env: dict[str, Any] = {
        "timestamp": datetime.now(timezone.utc).isoformat(),
        "python_version": sys.version.split()[0],
        "platform": platform.platform(),
        "gpu_available": False,
        "gpu_name": "unavailable",
        "gpu_arch": None,
        "logical_cuda_device": None,
        "cuda_driver_version": _driver_version(),
        "cuda_driver_api_version": None,
        "cuda_version": None,
        "nvcc_version": None,
        "hipcc_version": _command(["hipcc", "--version"]),
        "torch_version": None,
        "triton_version": None,
        "kernel_library": None,
        "compute_capability": None,
        "total_memory_bytes": None,
        "free_memory_bytes": None,
        "sm_count": None,
        "fp16_supported": False,
        "bf16_supported": False,
        "fp32_supported": False,
        "tf32_supported": False,
        "tensor_core_capability": "unknown",
        "dtype_probes": {},
    }
    try:
        from kernels import _native

        lib = _native.library()
        env["kernel_library"] = f"libmoegemm-abi{lib.moegemm_abi_version()}"
        env["triton_version"] = env["kernel_library"]
    except Exception as exc:
        env["kernel_library_error"] = repr(exc)
    try:
        import torch

        env["torch_version"] = torch.__version__
        hip = getattr(torch.version, "hip", None)
        env["cuda_version"] = f"hip-{hip}" if hip else None
        env["cuda_driver_api_version"] = hip
        if torch.cuda.is_available():
            index = torch.cuda.current_device()
            props = torch.cuda.get_device_properties(index)
            free, total = torch.cuda.mem_get_info(index)
            major, minor = torch.cuda.get_device_capability(index)
            arch = str(getattr(props, "gcnArchName", "")).split(":")[0] or None
            env.update(
                gpu_available=True,
                gpu_name=f"{props.name} ({arch})" if arch else props.name,
                gpu_arch=arch,
                logical_cuda_device=f"cuda:{index}",
                compute_capability=f"{major}.{minor}",
                total_memory_bytes=int(props.total_memory),
                runtime_total_memory_bytes=int(total),
                free_memory_bytes=int(free),
                sm_count=int(props.multi_processor_count),
                tf32_supported=False,  # emulated by operand rounding; no XF32 MFMA on gfx950
                tensor_core_capability=_MATRIX_CORES.get(arch or "", "matrix cores (unknown generation)"),
            )
            probes: dict[str, dict[str, Any]] = {}
            for name, dtype in (("fp16", torch.float16), ("bf16", torch.bfloat16), ("fp32", torch.float32)):
                try:
                    x = torch.ones((16, 16), device="cuda", dtype=dtype)
                    y = torch.mm(x, x)
                    torch.cuda.synchronize()
                    probes[name] = {"torch_matmul_ok": True, "result_dtype": str(y.dtype),
                                    "finite": bool(torch.isfinite(y).all().item())}
                except Exception as probe_exc:
                    probes[name] = {"torch_matmul_ok": False, "error": repr(probe_exc)}
            env["dtype_probes"] = probes
            for name in ("fp16", "bf16", "fp32"):
                env[f"{name}_supported"] = bool(probes[name].get("torch_matmul_ok"))
    except Exception as exc:
        env["torch_probe_error"] = repr(exc)
    return env


def write_environment(path: str | Path, extra: dict[str, Any] | None = None) -> dict[str, Any]:
    env = collect_environment()
    if extra:
        env.update(extra)
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(env, indent=2, ensure_ascii=False) + "\n", encoding="utf-8")
    return env
