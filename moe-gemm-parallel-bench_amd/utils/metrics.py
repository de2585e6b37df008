"""Workload arithmetic: FLOPs, ideal bytes, tile/wave metrics and per-rank EP/TP expert shapes.

Restates the reference's utils/metrics.py:9-80.  Shapes are (M, K, N) triples: one expert GEMM
[M, K] @ [K, N].  Everything here is exact integer arithmetic except the ratios.
"""

from __future__ import annotations

import math
from collections.abc import Iterable


def gemm_flops(m: int, k: int, n: int) -> int:
    """Useful FLOPs of one [m, k] @ [k, n] product (one multiply + one add per term)."""
    return 2 * m * k * n


def gemm_bytes(m: int, k: int, n: int, element_size: int) -> int:
    """Ideal traffic: read A and B once, write C once."""
    return element_size * (m * k + k * n + m * n)


def arithmetic_intensity(m: int, k: int, n: int, element_size: int) -> float:
    """FLOPs per ideal byte (reference utils/metrics.py:13-16); not measured traffic."""
    traffic = gemm_bytes(m, k, n, element_size)
    return gemm_flops(m, k, n) / traffic if traffic else 0.0


def tile_metrics(
    shapes: Iterable[tuple[int, int, int]], block_m: int, block_n: int, block_k: int, sm_count: int
) -> dict[str, float | int]:
    """Tile counts, waves over ``sm_count`` compute units, and padding efficiencies."""
    shapes = list(shapes)
    out_tiles = 0
    mac_tiles = 0
    useful = 0
    useful_out = 0
    for m, k, n in shapes:
        tiles = math.ceil(m / block_m) * math.ceil(n / block_n)
        out_tiles += tiles
        mac_tiles += tiles * math.ceil(k / block_k)
        useful += gemm_flops(m, k, n)
        useful_out += m * n
    padded = mac_tiles * 2 * block_m * block_n * block_k
    padded_out = out_tiles * block_m * block_n
    return {
        "output_tiles_per_gemm": out_tiles / len(shapes) if shapes else 0.0,
        "total_output_tiles_per_rank": out_tiles,
        "dot_tiles": mac_tiles,
        "tiles_per_sm": out_tiles / sm_count if sm_count else 0.0,
        "estimated_waves": math.ceil(out_tiles / sm_count) if sm_count and out_tiles else 0,
        "tile_efficiency": useful / padded if padded else 0.0,
        "output_tile_efficiency": useful_out / padded_out if padded_out else 0.0,
    }


def moe_shapes(
    projection: str,
    parallel_type: str,
    m: int,
    hidden: int,
    ffn: int,
    experts: int,
    parallel_size: int,
) -> list[tuple[int, int, int]]:
    """One rank's expert GEMMs after uniform top-k routing (no router is executed).

    ``m`` is the number of top-k-expanded rows per expert.  EP ranks own ``experts / P`` whole
    experts; TP ranks own every expert with ``ffn / P`` columns.  W1 is the packed Gate+Up (W13)
    projection with output width ``2 * F_local``; W2 is Down with contraction ``F_local``.
    """
    if experts % parallel_size:
        raise ValueError("num_experts must be divisible by parallel_size")
    if ffn % parallel_size:
        raise ValueError("ffn_size must be divisible by parallel_size")
    if parallel_type not in ("EP", "TP"):
        raise ValueError(f"unknown parallel type {parallel_type}")
    expert_parallel = parallel_type == "EP"
    count = experts // parallel_size if expert_parallel else experts
    local_ffn = ffn if expert_parallel else ffn // parallel_size
    if projection == "W1":
        shape = (m, hidden, 2 * local_ffn)
    elif projection == "W2":
        shape = (m, local_ffn, hidden)
    else:
        raise ValueError(f"unknown projection {projection}")
    return [shape] * count


def verify_ep_tp_flops(projection: str, m: int, hidden: int, ffn: int, experts: int, p: int) -> int:
    """Per-rank FLOPs of the projection; raises unless EP and TP are exactly equal."""
    totals = {
        kind: sum(gemm_flops(*shape) for shape in moe_shapes(projection, kind, m, hidden, ffn, experts, p))
        for kind in ("EP", "TP")
    }
    if totals["EP"] != totals["TP"]:
        raise ValueError(f"per-rank FLOPs differ: EP={totals['EP']}, TP={totals['TP']}")
    return totals["EP"]
