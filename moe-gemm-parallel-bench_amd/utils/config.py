"""Expert dimensions from a Hugging Face style MoE ``config.json``.

``load_model_defaults(path) -> ModelDefaults`` is the loader the reference's drivers call
(reference utils/config.py:11-66; the dataclass fields are that interface).  The published
configs of MoE families name the same four quantities differently, so each field is read through
an ordered alias list; the first alias present wins:

=============  ============================================================================
field          aliases (families that use them)
=============  ============================================================================
hidden_size    hidden_size (all)
ffn_size       moe_intermediate_size (DeepSeek, GLM, Kimi, Qwen3), then intermediate_size
               (Mixtral, GPT-OSS, Llama 4, where it is the routed expert's width)
num_experts    n_routed_experts (DeepSeek, GLM, Kimi), num_local_experts (Mixtral, GPT-OSS,
               Llama 4), num_experts (Qwen3)
topk           num_experts_per_tok (most), num_experts_per_token, router_top_k
=============  ============================================================================

Multimodal configs (Llama 4) keep the language model under ``text_config``; that block is the
scope for every field when present.  A dense ``intermediate_size`` next to a
``moe_intermediate_size`` is the shared/dense MLP and is ignored.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any


@dataclass(frozen=True)
class ModelDefaults:
    model_path: str
    model_type: str
    hidden_size: int
    ffn_size: int
    num_experts: int
    topk: int
    dtype: str
    config_ep_size: int
    quantization: dict[str, Any] | None


_ALIASES: dict[str, tuple[str, ...]] = {
    "hidden_size": ("hidden_size",),
    "ffn_size": ("moe_intermediate_size", "intermediate_size"),
    "num_experts": ("n_routed_experts", "num_local_experts", "num_experts"),
    "topk": ("num_experts_per_tok", "num_experts_per_token", "router_top_k"),
}
_DTYPE_NAMES = {"float16": "fp16", "bfloat16": "bf16", "float32": "fp32"}


def _resolve(scopes: list[dict[str, Any]], aliases: tuple[str, ...]) -> Any:
    """First non-null value of the aliases, trying every alias in the innermost scope first."""
    for scope in scopes:
        for alias in aliases:
            if scope.get(alias) is not None:
                return scope[alias]
    return None


def load_model_defaults(path: str | Path) -> ModelDefaults:
    """Read one config file; ValueError names every dimension the schema does not provide."""
    path = Path(path)
    raw = json.loads(path.read_text(encoding="utf-8"))
    nested = raw.get("text_config")
    inner = nested if isinstance(nested, dict) else raw
    dims = {field: _resolve([inner], aliases) for field, aliases in _ALIASES.items()}
    absent = sorted(field for field, value in dims.items() if value is None)
    if absent:
        raise ValueError(f"{path}: not a supported MoE config schema; missing {', '.join(absent)} "
                         f"(looked for {', '.join(a for f in absent for a in _ALIASES[f])})")
    declared = _resolve([inner, raw], ("torch_dtype", "dtype"))
    return ModelDefaults(
        model_path=str(path),
        model_type=str(_resolve([raw, inner], ("model_type",)) or path.stem),
        hidden_size=int(dims["hidden_size"]),
        ffn_size=int(dims["ffn_size"]),
        num_experts=int(dims["num_experts"]),
        topk=int(dims["topk"]),
        dtype=_DTYPE_NAMES.get(str(declared), "bf16"),
        config_ep_size=int(_resolve([inner, raw], ("ep_size",)) or 1),
        quantization=_resolve([inner, raw], ("quantization_config",)),
    )
