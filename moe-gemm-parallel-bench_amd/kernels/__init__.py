"""gfx950 HIP grouped/single GEMM kernels and the PyTorch grouped_mm comparison provider."""

from .grouped_gemm import (
    GroupedWorkspace,
    build_fused_gate_up_workspace,
    build_grouped_workspace,
    grouped_candidate_configs,
    launch_gate_up_swiglu,
    launch_grouped,
)
from .grouped_mm import (
    OffsetsWorkspace,
    build_offsets_workspace,
    grouped_mm,
    grouped_mm_swiglu,
    last_grouped_mm_config,
    last_grouped_mm_schedule,
    launch_grouped_offsets,
)
from .matmul import (
    KernelConfig,
    last_matmul_config,
    launch_matmul,
    matmul_candidate_configs,
    select_config,
)
from .torch_grouped_gemm import (
    TorchGroupedMMUnavailable,
    TorchGroupedWorkspace,
    build_torch_grouped_workspace,
    launch_torch_grouped,
    torch_grouped_mm_unavailable_reason,
)

__all__ = [
    "GroupedWorkspace",
    "KernelConfig",
    "OffsetsWorkspace",
    "TorchGroupedMMUnavailable",
    "TorchGroupedWorkspace",
    "build_fused_gate_up_workspace",
    "build_grouped_workspace",
    "build_offsets_workspace",
    "build_torch_grouped_workspace",
    "grouped_candidate_configs",
    "grouped_mm",
    "grouped_mm_swiglu",
    "last_grouped_mm_config",
    "last_grouped_mm_schedule",
    "last_matmul_config",
    "launch_gate_up_swiglu",
    "launch_grouped",
    "launch_grouped_offsets",
    "launch_matmul",
    "launch_torch_grouped",
    "matmul_candidate_configs",
    "select_config",
    "torch_grouped_mm_unavailable_reason",
]
