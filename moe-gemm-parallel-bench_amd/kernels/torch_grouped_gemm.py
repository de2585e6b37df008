"""PyTorch ``grouped_mm`` as a comparison provider on ROCm, admitted only on trace evidence.

The reference compares its kernel against one public ``torch.nn.functional.grouped_mm`` call over
the expert-sorted layout (2-D A [sum M_e, K], 3-D B [G, K, N], int32 cumulative ``offs``, row
strides padded to 16 bytes: reference kernels/torch_grouped_gemm.py:121-174).  The same public
names live here - ``TorchGroupedWorkspace`` (its fields are the interface),
``build_torch_grouped_workspace``, ``launch_torch_grouped``,
``torch_grouped_mm_unavailable_reason``, ``inspect_grouped_trace``,
``verify_torch_grouped_execution`` and ``TorchGroupedMMUnavailable`` - with this project's own
admission rule:

A call is admitted as "one grouped kernel" only if a profiler trace of exactly that shape and
dtype shows it.  Every device activity of the traced call is classified:

  copy        a memcpy (host/device transfer or device copy)   -> never allowed
  fill        memset / fill kernels                            -> allowed, not counted
  metadata    grouped-GEMM argument preparation                -> allowed, counted as a launch
  grouped     a grouped-GEMM compute kernel (CK/hipBLASLt/...) -> exactly one required
  other       anything else (a plain GEMM, an unknown kernel)  -> never allowed

and the host side must show exactly one ``aten::_grouped_mm`` and no ``aten::mm`` / ``bmm`` /
``matmul`` / ``addmm`` (those are the sequential fallback).  Anything the classifier does not
recognise fails the check: the provider is skipped rather than mislabelled.
"""

from __future__ import annotations

from collections.abc import Iterator, Sequence
from dataclasses import dataclass

try:
    import torch
except ImportError:  # pragma: no cover - the module stays importable for CPU tooling
    torch = None


class TorchGroupedMMUnavailable(RuntimeError):
    """torch's grouped_mm cannot be admitted (missing API/GPU, or a trace that proves no grouped kernel)."""


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
        held = [t for t in (self.mat_a, self.mat_b, self.offs, self.output) if t is not None]
        return sum(t.untyped_storage().nbytes() for t in held)

    def problem_tensors(self) -> Iterator[tuple[object, object, object]]:
        """(A_e, B_e, C_e) views per expert of the last output."""
        if self.output is None:
            raise RuntimeError("torch grouped_mm has not produced an output yet")
        begin = 0
        for index, (rows, _, _) in enumerate(self.shapes):
            yield self.mat_a[begin:begin + rows], self.mat_b[index], self.output[begin:begin + rows]
            begin += rows


_GROUP_LIMIT = 1024  # torch's grouped_mm checks the group count against this bound


def torch_grouped_mm_unavailable_reason(dtype=None, problem_count: int = 1) -> str:
    """Why the provider cannot run at all ("" when a trace check is worth attempting)."""
    if torch is None:
        return "PyTorch unavailable"
    if not hasattr(torch.nn.functional, "grouped_mm"):
        return "torch.nn.functional.grouped_mm unavailable in this PyTorch"
    if not torch.cuda.is_available():
        return "GPU unavailable"
    if dtype is not None and dtype != torch.bfloat16:
        return "grouped_mm is only trace-checked for bf16; other dtypes take torch's sequential path"
    if problem_count >= _GROUP_LIMIT:
        return f"grouped_mm takes fewer than {_GROUP_LIMIT} groups"
    return ""


_FALLBACK_OPS = frozenset({"aten::mm", "aten::mm_out", "aten::bmm", "aten::matmul", "aten::addmm"})


def _classify(kernel_name: str) -> str:
    name = kernel_name.lower()
    if "memcpy" in name or "copybuffer" in name:
        return "copy"
    if "memset" in name or "fill" in name or "zero" in name:
        return "fill"
    if "prepare" in name and "group" in name:
        return "metadata"
    if "group" in name and ("gemm" in name or "_mm" in name or "matmul" in name):
        return "grouped"
    return "other"


def inspect_grouped_trace(cpu_ops: Sequence[str], cuda_events: Sequence[str]) -> dict[str, int | bool]:
    """Execution evidence of one traced call, or TorchGroupedMMUnavailable (fail closed)."""
    fallback = sorted(set(cpu_ops) & _FALLBACK_OPS)
    if fallback:
        raise TorchGroupedMMUnavailable(f"profiler saw the sequential fallback ({', '.join(fallback)})")
    grouped_calls = sum(op == "aten::_grouped_mm" for op in cpu_ops)
    if grouped_calls != 1:
        raise TorchGroupedMMUnavailable(f"expected one aten::_grouped_mm call, the profiler saw {grouped_calls}")
    classes: dict[str, list[str]] = {}
    for event in cuda_events:
        classes.setdefault(_classify(event), []).append(event)
    if classes.get("copy"):
        raise TorchGroupedMMUnavailable("the traced call moved data (memcpy); not a device-resident grouped GEMM")
    if classes.get("other"):
        raise TorchGroupedMMUnavailable(f"unrecognised device kernels in the trace: {classes['other'][:3]}")
    if len(classes.get("grouped", [])) != 1:
        raise TorchGroupedMMUnavailable(
            f"expected exactly one grouped compute kernel, found {len(classes.get('grouped', []))}")
    return {
        "execution_verified": True,
        "api_calls_per_iteration": 1,
        "launches_per_iteration": 1 + len(classes.get("metadata", [])),
        "grouped_compute_launches": 1,
    }


def verify_torch_grouped_execution(workspace: TorchGroupedWorkspace) -> dict[str, int | bool]:
    """Trace one call on this workspace (after an untimed warm call) and inspect it."""
    activities = torch.profiler.supported_activities()
    if torch.profiler.ProfilerActivity.CUDA not in activities:
        raise TorchGroupedMMUnavailable("device profiling (roctracer) unavailable; execution cannot be verified")
    try:
        launch_torch_grouped(workspace)
        torch.cuda.synchronize()
        with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU,
                                                torch.profiler.ProfilerActivity.CUDA]) as trace:
            launch_torch_grouped(workspace)
            torch.cuda.synchronize()
    except TorchGroupedMMUnavailable:
        raise
    except RuntimeError as exc:
        raise TorchGroupedMMUnavailable(f"grouped_mm probe failed: {exc}") from exc
    host = [e.name for e in trace.events() if e.device_type == torch.autograd.DeviceType.CPU]
    device = [e.name for e in trace.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    return inspect_grouped_trace(host, device)


def _padded_columns(columns: int, element_size: int) -> int:
    per_16_bytes = max(1, 16 // element_size)
    return -(-columns // per_16_bytes) * per_16_bytes


def build_torch_grouped_workspace(
    shapes: Sequence[tuple[int, int, int]],
    dtype,
    seed: int = 0,
    *,
    operation: str = "gemm",
    device: str = "cuda",
) -> TorchGroupedWorkspace:
    """Expert-sorted operands with 16-byte row pitches and seeded ``normal_() * 0.1`` values.

    Groups share K and N (the 2-D x 3-D form of grouped_mm); ``offs`` holds the cumulative end
    row of each group as int32.  ``device="cpu"`` builds the same layout on the host (for the CPU
    baseline and layout tests); launching requires a GPU.
    """
    if device != "cpu":
        reason = torch_grouped_mm_unavailable_reason(dtype, len(shapes))
        if reason:
            raise TorchGroupedMMUnavailable(reason)
    problems = tuple(tuple(int(v) for v in shape) for shape in shapes)
    if not problems or any(len(p) != 3 or min(p) <= 0 for p in problems):
        raise ValueError("torch grouped GEMM needs at least one positive (M, K, N) problem")
    ks, ns = {k for _, k, _ in problems}, {n for _, _, n in problems}
    if len(ks) != 1 or len(ns) != 1:
        raise ValueError("torch grouped_mm's 2-D x 3-D form needs one shared K and one shared N")
    k, n = ks.pop(), ns.pop()
    ends, total = [], 0
    for m, _, _ in problems:
        total += m
        ends.append(total)
    if total >= 2**31:
        raise ValueError("grouped_mm offsets must fit int32")
    element_size = torch.empty((), dtype=dtype).element_size()
    generator = torch.Generator(device=device).manual_seed(seed)
    a_store = torch.empty((total, _padded_columns(k, element_size)), device=device, dtype=dtype)
    b_store = torch.empty((len(problems), k, _padded_columns(n, element_size)), device=device, dtype=dtype)
    mat_a, mat_b = a_store[:, :k], b_store[:, :, :n]
    mat_a.normal_(generator=generator).mul_(0.1)
    mat_b.normal_(generator=generator).mul_(0.1)
    offs = torch.tensor(ends, device=device, dtype=torch.int32)
    return TorchGroupedWorkspace(mat_a, mat_b, offs, problems, operation=operation)


def launch_torch_grouped(workspace: TorchGroupedWorkspace) -> None:
    """One ``torch.nn.functional.grouped_mm`` call.  The previous output is released first so
    the caching allocator hands the same block back (grouped_mm has no ``out=``)."""
    if workspace.mat_a.device.type == "cpu":  # host operands: torch's CPU kernel (layout checks, CPU timing)
        reason = "" if hasattr(torch.nn.functional, "grouped_mm") else "torch.nn.functional.grouped_mm unavailable"
    else:
        reason = torch_grouped_mm_unavailable_reason(workspace.mat_a.dtype, workspace.problem_count)
    if reason:
        raise TorchGroupedMMUnavailable(reason)
    workspace.output = None
    workspace.output = torch.nn.functional.grouped_mm(workspace.mat_a, workspace.mat_b, offs=workspace.offs)
    workspace.scheduler = "torch_grouped_mm"
