"""Generate the golden GEMM fixtures in this directory with torch on the CPU (float64 products).

The vectors are independent of the oracle: inputs are drawn with a seeded torch CPU generator
(``normal_() * 0.1`` like the reference builders, kernels/grouped_gemm.py:522-527), rounded to
the operand dtype by torch, and the expected values are torch's float64 matmul of those rounded
operands plus torch's cast of that product to the operand dtype.  Shapes follow the reference's
own GPU tests (tests/test_gpu.py:74, :89, :100, :178) plus a BASELINE.json plumbing-case sample.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def case(gen: torch.Generator, m: int, k: int, n: int, dtype: torch.dtype, scale: float = 0.1):
    a = (torch.empty((m, k), dtype=torch.float64).normal_(generator=gen) * scale).to(dtype)
    b = (torch.empty((k, n), dtype=torch.float64).normal_(generator=gen) * scale).to(dtype)
    exact = a.double() @ b.double()
    rounded = exact.to(dtype)
    return bits(a), bits(b), exact.numpy(), bits(rounded)


def main() -> None:
    gen = torch.Generator(device="cpu").manual_seed(20260601)
    arrays: dict[str, np.ndarray] = {}
    names = []
    shapes = [(1, 5, 3), (17, 13, 31), (33, 70, 65), (9, 70, 65), (16, 64, 128)]
    plan = [(d, s) for d in DTYPES for s in shapes] + [("bf16", (40, 256, 320))]
    for dname, (m, k, n) in plan:
        key = f"{dname}_{m}x{k}x{n}"
        a, b, exact, rounded = case(gen, m, k, n, DTYPES[dname])
        arrays[f"{key}_a"], arrays[f"{key}_b"] = a, b
        arrays[f"{key}_exact"], arrays[f"{key}_out"] = exact, rounded
        names.append(key)
    # Packed W13 (gate | up along N): reference tests/test_gpu.py:176-188 shape.
    a, b, exact, rounded = case(gen, 17, 13, 62, torch.float16)
    arrays["w13_fp16_a"], arrays["w13_fp16_b"], arrays["w13_fp16_exact"], arrays["w13_fp16_out"] = a, b, exact, rounded
    # Plumbing case sample: one expert of [64, 512] @ [512, 1024], bf16,
    # N(0,1)/sqrt(K) inputs; the exact product is kept only for 64 sampled entries.
    k = 512
    a = (torch.empty((64, k), dtype=torch.float64).normal_(generator=gen) / math.sqrt(k)).to(torch.bfloat16)
    b = (torch.empty((k, 1024), dtype=torch.float64).normal_(generator=gen) / math.sqrt(k)).to(torch.bfloat16)
    exact = a.double() @ b.double()
    rows = torch.randint(0, 64, (64,), generator=gen)
    cols = torch.randint(0, 1024, (64,), generator=gen)
    arrays["plumbing_a"], arrays["plumbing_b_cols"] = bits(a), bits(b[:, cols])
    arrays["plumbing_rows"], arrays["plumbing_cols"] = rows.numpy(), cols.numpy()
    arrays["plumbing_exact"] = exact[rows, cols].numpy()
    arrays["plumbing_out"] = bits(exact.to(torch.bfloat16)[rows, cols])
    # Rounding vectors: float32 values and torch's bf16/fp16 casts, including ties and edges.
    edge = torch.tensor(
        [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, -65520.0, 1e-8, -1e-8, 6.1e-5, 5.96e-8,
         2.98e-8, 3.0e38, float("inf"), float("-inf")], dtype=torch.float32)
    ties = torch.tensor([1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11], dtype=torch.float32)
    rnd = torch.empty(4096, dtype=torch.float64).normal_(generator=gen).mul_(3.0).exp_().float()
    rnd[::2] *= -1
    values = torch.cat([edge, ties, rnd])
    arrays["round_values"] = values.numpy()
    arrays["round_bf16"] = bits(values.to(torch.bfloat16))
    arrays["round_fp16"] = bits(values.to(torch.float16))
    arrays["case_names"] = np.array(names)
    np.savez_compressed(HERE / "gemm_golden.npz", **arrays)
    print(f"wrote {len(names)} GEMM cases, W13, plumbing sample and {values.numel()} rounding vectors")


if __name__ == "__main__":
    main()
