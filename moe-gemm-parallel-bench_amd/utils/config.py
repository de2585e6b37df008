"""Model configuration loading: maps Hugging Face ``config.json`` schemas to MoE GEMM dimensions.

Same contract as the reference's utils/config.py:32-66: hidden size H, routed-expert FFN width F,
expert count E and top-k are read from the first matching key of each schema family; multimodal
configs keep the language model under ``text_config``; a missing field is a ValueError naming it.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any

# Key preference per field.  A dedicated MoE width wins over ``intermediate_size``, which some
# schemas use for the dense MLP and others for the expert MLP.
_FIELD_KEYS = {
    "hidden_size": ("hidden_size",),
    "ffn_size": ("moe_intermediate_size", "intermediate_size"),
    "num_experts": ("n_routed_experts", "num_local_experts", "num_experts"),
    "topk": ("num_experts_per_tok", "num_experts_per_token", "router_top_k"),
}
_DTYPE_NAMES = {"float16": "fp16", "bfloat16": "bf16", "float32": "fp32"}


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


def _lookup(mapping: dict[str, Any], keys: tuple[str, ...]) -> Any:
    return next((mapping[key] for key in keys if mapping.get(key) is not None), None)


def load_model_defaults(path: str | Path) -> ModelDefaults:
    path = Path(path)
    raw = json.loads(path.read_text(encoding="utf-8"))
    scope = raw["text_config"] if isinstance(raw.get("text_config"), dict) else raw
    values = {field: _lookup(scope, keys) for field, keys in _FIELD_KEYS.items()}
    missing = [field for field, value in values.items() if value is None]
    if missing:
        raise ValueError(f"unsupported MoE config schema in {path}: missing " + ", ".join(missing))
    declared = _lookup(scope, ("torch_dtype", "dtype")) or _lookup(raw, ("torch_dtype", "dtype")) or "bfloat16"
    return ModelDefaults(
        model_path=str(path),
        model_type=str(raw.get("model_type", scope.get("model_type", path.stem))),
        hidden_size=int(values["hidden_size"]),
        ffn_size=int(values["ffn_size"]),
        num_experts=int(values["num_experts"]),
        topk=int(values["topk"]),
        dtype=_DTYPE_NAMES.get(str(declared), "bf16"),
        config_ep_size=int(scope.get("ep_size", raw.get("ep_size", 1))),
        quantization=scope.get("quantization_config") or raw.get("quantization_config"),
    )
