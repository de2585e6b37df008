"""Workload cases: the per-rank MoE EP/TP GEMMs, the single-GEMM shape sweep and the heatmap.

A ``Case`` is one group of GEMM problems (M, K, N) that one provider launch computes, plus the
labels its CSV row carries.  Case generators turn the run settings into an ordered list; they do
all argument checks that do not need a GPU, so a bad sweep fails before any allocation.

MoE cases follow the reference's per-rank construction (reference benchmark_moe.py:341-372 and
utils/metrics.py:40-80): M is the top-k-expanded row count per expert, T = M * E / topk must be
integral, and EP and TP ranks do exactly equal FLOPs.  The heatmap extends the reference's
G = 1 grid (benchmark_shapes.py:321-335) with group counts and K values.
"""

from __future__ import annotations

from collections.abc import Iterator
from dataclasses import dataclass, field

from utils.metrics import gemm_flops, moe_shapes, verify_ep_tp_flops

DEFAULT_MOE_MS = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024)
DEFAULT_SHAPE_MS = (8192, 4096, 2048, 1024, 512, 256, 128, 64, 32, 16)
DEFAULT_HEATMAP_MS = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024)
DEFAULT_HEATMAP_NS = (256, 512, 1024, 2048, 4096, 8192, 14336)

_PROJECTION_LABELS = {
    # projection -> (operation, fused projections, output layout)
    "W1": ("gate_up", 2, "gate_then_up"),
    "W2": ("down", 1, "down"),
}


@dataclass(frozen=True)
class Case:
    experiment: str                                   # "moe" | "shapes" | "heatmap"
    shapes: tuple[tuple[int, int, int], ...]          # (M, K, N) per problem
    projection: str = ""                              # "W1" | "W2" for MoE cases
    parallel_type: str = ""                           # "EP" | "TP" for MoE cases
    tokens: int | None = None                         # pre-routing tokens T (MoE)
    skip_reason: str = ""                             # set when the case cannot be formed
    labels: dict = field(default_factory=dict, compare=False, hash=False)

    @property
    def m(self) -> int:
        return self.shapes[0][0]

    @property
    def k(self) -> int:
        return self.shapes[0][1]

    @property
    def n(self) -> int:
        return self.shapes[0][2]

    @property
    def problem_count(self) -> int:
        return len(self.shapes)

    @property
    def total_flops(self) -> int:
        return sum(gemm_flops(*shape) for shape in self.shapes)

    @property
    def projection_labels(self) -> tuple[str, object, str]:
        return _PROJECTION_LABELS.get(self.projection, ("", "", ""))

    @property
    def name(self) -> str:
        if self.experiment == "moe":
            return f"{self.projection} {self.parallel_type} M={self.m}"
        return f"{self.experiment} G={self.problem_count} M={self.m} K={self.k} N={self.n}"


def _positive(values, option: str) -> tuple[int, ...]:
    values = tuple(int(v) for v in values)
    if not values or min(values) <= 0:
        raise ValueError(f"{option} must list positive integers")
    return values


def moe_token_counts(settings) -> tuple[int, ...]:
    """Rows per expert to sweep: ``--tokens`` T gives the single M = T * topk / E."""
    experts, topk = settings.num_experts, settings.topk
    if experts % settings.parallel_size:
        raise ValueError(f"num_experts ({experts}) must be divisible by parallel_size ({settings.parallel_size})")
    if settings.ffn_size % settings.parallel_size:
        raise ValueError(f"ffn_size ({settings.ffn_size}) must be divisible by parallel_size ({settings.parallel_size})")
    if settings.tokens is not None:
        if settings.tokens <= 0:
            raise ValueError("--tokens must be positive")
        if (settings.tokens * topk) % experts:
            raise ValueError("tokens * topk must be divisible by num_experts (uniform routing needs whole rows)")
        return ((settings.tokens * topk) // experts,)
    ms = _positive(settings.moe_ms or DEFAULT_MOE_MS, "--moe-ms")
    uneven = [m for m in ms if (m * experts) % topk]
    if uneven:
        raise ValueError("every M * num_experts must be divisible by topk so that T is integral; offending M: "
                         + ",".join(map(str, uneven)))
    return ms


def moe_cases(settings, projection: str) -> list[Case]:
    """EP and TP cases of one projection, M ascending, EP before TP at each M."""
    cases = []
    for m in moe_token_counts(settings):
        verify_ep_tp_flops(projection, m, settings.hidden_size, settings.ffn_size, settings.num_experts,
                           settings.parallel_size)
        for parallel_type in ("EP", "TP"):
            shapes = moe_shapes(projection, parallel_type, m, settings.hidden_size, settings.ffn_size,
                                settings.num_experts, settings.parallel_size)
            cases.append(Case("moe", tuple(shapes), projection, parallel_type,
                              tokens=m * settings.num_experts // settings.topk))
    return cases


def shape_cases(settings) -> list[Case]:
    """Single GEMMs [M, shape_k] @ [shape_k, product / M]; an M that does not divide the product
    yields a case carrying its skip reason (a row is still written for it)."""
    product = settings.shape_product
    cases = []
    for m in _positive(settings.shape_ms or DEFAULT_SHAPE_MS, "--shape-ms"):
        if product % m:
            cases.append(Case("shapes", ((m, settings.shape_k, 0),), skip_reason="M does not divide shape product"))
        else:
            cases.append(Case("shapes", ((m, settings.shape_k, product // m),)))
    return cases


def heatmap_cases(settings) -> list[Case]:
    """G x K x M x N grid of G equal problems; G defaults to 1 and K to ``heatmap_k``."""
    groups = _positive(getattr(settings, "heatmap_gs", None) or (1,), "--heatmap-gs")
    ks = _positive(getattr(settings, "heatmap_ks", None) or (settings.heatmap_k,), "--heatmap-ks")
    ms = _positive(settings.heatmap_ms or DEFAULT_HEATMAP_MS, "--heatmap-ms")
    ns = _positive(settings.heatmap_ns or DEFAULT_HEATMAP_NS, "--heatmap-ns")
    return [Case("heatmap", ((m, k, n),) * g) for g in groups for k in ks for m in ms for n in ns]


def iter_experiments(settings) -> Iterator[tuple[str, list[Case]]]:
    """(CSV stem, cases) per output file of the selected experiments, in run order."""
    selected = {"shapes", "moe", "heatmap"} if settings.experiment == "all" else {settings.experiment}
    if "shapes" in selected:
        yield "gemm_shape_sweep", shape_cases(settings)
    if "moe" in selected:
        yield "moe_w1", moe_cases(settings, "W1")
        yield "moe_w2", moe_cases(settings, "W2")
    if "heatmap" in selected:
        yield "gemm_heatmap", heatmap_cases(settings)
