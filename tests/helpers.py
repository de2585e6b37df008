"""Conversions between torch tensors and the oracle's numpy encodings (test infrastructure)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle

DTYPE_NAME = {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}
TORCH_DTYPE = {name: dtype for dtype, name in DTYPE_NAME.items()}


def to_oracle(t: torch.Tensor) -> np.ndarray:
    """Copy a (possibly strided) tensor to host memory in the oracle's encoding, keeping strides."""
    host = t.detach().cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        storage = host.as_strided((host.untyped_storage().nbytes() // 2,), (1,), 0)
        flat = storage.view(torch.int16).numpy().view(np.uint16)
        es = 2
    else:
        storage = host.as_strided((host.untyped_storage().nbytes() // 4,), (1,), 0)
        flat = storage.numpy()
        es = 4
    base = flat[host.storage_offset():]
    return np.lib.stride_tricks.as_strided(base, shape=tuple(host.shape),
                                           strides=tuple(s * es for s in host.stride()))


def from_oracle(c: np.ndarray, dtype_name: str) -> torch.Tensor:
    """Oracle output (bit patterns or float32) -> float64 torch tensor of the represented values."""
    return torch.from_numpy(oracle.to_float(np.ascontiguousarray(c), dtype_name).astype(np.float64))


def oracle_product(a: torch.Tensor, b: torch.Tensor, *, tf32: bool = False, accum: str = "f64") -> torch.Tensor:
    """Oracle C = A @ B for device or host tensors, as float64 values of the rounded output."""
    name = DTYPE_NAME[a.dtype]
    c = oracle.gemm(to_oracle(a), to_oracle(b), name, tf32=tf32, accum=accum)
    return from_oracle(c, name)


def normwise(actual: torch.Tensor, reference: torch.Tensor) -> float:
    diff = (actual.double().cpu() - reference.double().cpu()).abs()
    scale = float(reference.double().abs().max()) if reference.numel() else 0.0
    return float(diff.max()) / scale if scale > 0 else float(diff.max()) if diff.numel() else 0.0
