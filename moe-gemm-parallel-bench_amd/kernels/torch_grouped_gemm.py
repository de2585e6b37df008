"""PyTorch ``grouped_mm`` comparison provider (ROCm) for homogeneous MoE experts.

Mirrors the reference's kernels/torch_grouped_gemm.py: a 2-D expert-sorted A [sum M_e, K], a 3-D B
[G, K, N] and int32 cumulative ``offs`` (row strides padded to 16 bytes), one public
``torch.nn.functional.grouped_mm`` call per iteration, and admission only after a profiler trace
proves that the call ran as one grouped compute kernel (plus allowed metadata-preparation
kernels) with no sequential ``mm`` fallback and no device copies (reference :67-118).  On ROCm
the grouped kernel is not a CUTLASS kernel, so ``inspect_grouped_trace`` recognises the ROCm
grouped-GEMM kernel names instead; anything unrecognised stays unverified (fail closed).
"""

from __future__ import annotations

from collections.abc import Iterator, Sequence
from dataclasses import dataclass
from itertools import accumulate

try:
    import torch
except ImportError:  # pragma: no cover
    torch = None


class TorchGroupedMMUnavailable(RuntimeError):
    """Raised when the public PyTorch grouped-GEMM API cannot be admitted as one grouped kernel."""


@dataclass
class TorchGroupedWorkspace:
    mat_a: object
    mat_b: object
    offs: object
    shapes: tuple[tuple[int, int, int], ...]
    output: object | None = None
    operation: str = "gemm"
    scheduler: str = "torch_grouped_mm"

    @property
    def problem_count(self) -> int:
        return len(self.shapes)

    @property
    def storage_bytes(self) -> int:
        tensors = (self.mat_a, self.mat_b, self.offs, self.output)
        return sum(t.untyped_storage().nbytes() for t in tensors if t is not None)

    def problem_tensors(self) -> Iterator[tuple[object, object, object]]:
        if self.output is None:
            raise RuntimeError("torch grouped_mm has not produced an output")
        row = 0
        for index, (m, _, _) in enumerate(self.shapes):
            yield self.mat_a[row:row + m], self.mat_b[index], self.output[row:row + m]
            row += m


def torch_grouped_mm_unavailable_reason(dtype=None, problem_count: int = 1) -> str:
    if torch is None:
        return "PyTorch unavailable"
    if not hasattr(torch.nn.functional, "grouped_mm"):
        return "torch.nn.functional.grouped_mm unavailable"
    if not torch.cuda.is_available():
        return "GPU unavailable"
    if dtype is not None and dtype != torch.bfloat16:
        return "grouped_mm is admitted for bf16 only; other dtypes take a sequential fallback"
    if problem_count >= 1024:
        return "grouped_mm requires fewer than 1024 groups"
    return ""


# Substrings of device kernels that prepare grouped-GEMM metadata (counted as launches, not GEMMs).
_METADATA_KERNELS = ("prepare_grouped_gemm_data", "fill", "offsets")


def _is_metadata(name: str) -> bool:
    return any(tag in name for tag in _METADATA_KERNELS)


def _is_grouped_compute(name: str) -> bool:
    lowered = name.lower()
    if _is_metadata(lowered):
        return False
    return "group" in lowered and ("gemm" in lowered or "_mm" in lowered or "matmul" in lowered)


def inspect_grouped_trace(cpu_ops: Sequence[str], gpu_events: Sequence[str]) -> dict[str, int | bool]:
    """Fail closed unless the trace shows one native grouped_mm call and one grouped compute kernel."""
    if any(op in {"aten::mm", "aten::mm_out", "aten::bmm", "aten::matmul"} for op in cpu_ops):
        raise TorchGroupedMMUnavailable("profiler detected a sequential/batched matmul fallback")
    if list(cpu_ops).count("aten::_grouped_mm") != 1:
        raise TorchGroupedMMUnavailable("profiler did not observe exactly one native grouped_mm call")
    names = [n.lower() for n in gpu_events]
    if any("memcpy" in n or "copybuffer" in n for n in names):
        raise TorchGroupedMMUnavailable("grouped_mm probe contains a device transfer")
    kernels = [n for n in names if "memset" not in n]
    compute = [n for n in kernels if _is_grouped_compute(n)]
    others = [n for n in kernels if n not in compute]
    if len(compute) != 1 or any(not _is_metadata(n) for n in others):
        raise TorchGroupedMMUnavailable(f"device trace does not prove one grouped compute kernel: {kernels}")
    return {
        "execution_verified": True,
        "api_calls_per_iteration": 1,
        "launches_per_iteration": len(kernels),
        "grouped_compute_launches": 1,
    }


def verify_torch_grouped_execution(workspace: TorchGroupedWorkspace) -> dict[str, int | bool]:
    """Profile this exact shape/dtype (outside measurement) before admitting it."""
    activities = torch.profiler.supported_activities()
    if torch.profiler.ProfilerActivity.CUDA not in activities:
        raise TorchGroupedMMUnavailable("device profiler unavailable; grouped execution cannot be verified")
    try:
        launch_torch_grouped(workspace)
        torch.cuda.synchronize()
        with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU,
                                                torch.profiler.ProfilerActivity.CUDA]) as prof:
            launch_torch_grouped(workspace)
            torch.cuda.synchronize()
        events = prof.events()
        return inspect_grouped_trace(
            [e.name for e in events if e.device_type == torch.autograd.DeviceType.CPU],
            [e.name for e in events if e.device_type == torch.autograd.DeviceType.CUDA],
        )
    except TorchGroupedMMUnavailable:
        raise
    except RuntimeError as exc:
        raise TorchGroupedMMUnavailable(f"grouped execution probe failed: {exc}") from exc


def build_torch_grouped_workspace(
    shapes: Sequence[tuple[int, int, int]],
    dtype,
    seed: int = 0,
    *,
    operation: str = "gemm",
    device: str = "cuda",
) -> TorchGroupedWorkspace:
    if device != "cpu":
        reason = torch_grouped_mm_unavailable_reason(dtype, len(shapes))
        if reason:
            raise TorchGroupedMMUnavailable(reason)
    if not shapes:
        raise ValueError("torch grouped GEMM requires at least one problem")
    normalized = tuple(tuple(int(v) for v in s) for s in shapes)
    if any(len(s) != 3 or any(v <= 0 for v in s) for s in normalized):
        raise ValueError("every torch grouped shape must be a positive (M, K, N) triple")
    _, k, n = normalized[0]
    if any(kk != k or nn != n for _, kk, nn in normalized):
        raise ValueError("torch grouped_mm 2D/3D mode requires shared K and N dimensions")
    ends = tuple(accumulate(m for m, _, _ in normalized))
    if ends[-1] > 2**31 - 1:
        raise ValueError("torch grouped_mm offsets exceed int32 range")
    elements_per_16_bytes = max(1, 16 // torch.empty((), dtype=dtype).element_size())

    def padded(extent: int) -> int:
        return -(-extent // elements_per_16_bytes) * elements_per_16_bytes

    generator = torch.Generator(device=device).manual_seed(seed)
    mat_a = torch.empty((ends[-1], padded(k)), device=device, dtype=dtype)[:, :k]
    mat_b = torch.empty((len(normalized), k, padded(n)), device=device, dtype=dtype)[:, :, :n]
    mat_a.normal_(generator=generator).mul_(0.1)
    mat_b.normal_(generator=generator).mul_(0.1)
    offs = torch.tensor(ends, device=device, dtype=torch.int32)
    return TorchGroupedWorkspace(mat_a, mat_b, offs, normalized, operation=operation)


def launch_torch_grouped(workspace: TorchGroupedWorkspace) -> None:
    """One public grouped_mm call; the previous output is released first so the allocator reuses it."""
    if workspace.mat_a.device.type == "cuda":
        reason = torch_grouped_mm_unavailable_reason(workspace.mat_a.dtype, workspace.problem_count)
        if reason:
            raise TorchGroupedMMUnavailable(reason)
    workspace.output = None
    workspace.output = torch.nn.functional.grouped_mm(workspace.mat_a, workspace.mat_b, offs=workspace.offs)
    workspace.scheduler = "torch_grouped_mm"
