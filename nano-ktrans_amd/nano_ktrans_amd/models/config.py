"""Per-architecture routing flags and expert key layouts.

Restates the MoE-relevant fields of nano_ktrans/models/config.py:9-75 and the
``norm_topk_prob`` override of config.py:126, 181 (Qwen3-30B-A3B ships
``norm_topk_prob = true``, which overrides the spec default).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional


@dataclass
class ModelArchitectureSpec:
    name: str
    expert_key_template: str
    expert_proj_names: dict
    router_prefix: str
    experts_prefix: str
    router_use_softmax: bool = False
    normalize_topk_prob: bool = True
    has_shared_expert: bool = False
    shared_expert_key_template: Optional[str] = None
    shared_expert_prefix: Optional[str] = None
    shared_expert_gate_prefix: Optional[str] = None
    use_qk_norm: bool = False
    experts_are_packed: bool = False


MIXTRAL_SPEC = ModelArchitectureSpec(
    name="mixtral",
    expert_key_template="model.layers.{layer}.block_sparse_moe.experts.{expert}.{proj}.weight",
    expert_proj_names={"gate": "w1", "up": "w3", "down": "w2"},
    router_prefix="block_sparse_moe.gate",
    experts_prefix="block_sparse_moe.experts",
    router_use_softmax=False,
    normalize_topk_prob=True,
)

QWEN2_MOE_SPEC = ModelArchitectureSpec(
    name="qwen2_moe",
    expert_key_template="model.layers.{layer}.mlp.experts.{expert}.{proj}_proj.weight",
    expert_proj_names={"gate": "gate", "up": "up", "down": "down"},
    router_prefix="mlp.gate",
    experts_prefix="mlp.experts",
    router_use_softmax=True,
    normalize_topk_prob=False,
    has_shared_expert=True,
    shared_expert_key_template="model.layers.{layer}.mlp.shared_expert.{proj}_proj.weight",
    shared_expert_prefix="mlp.shared_expert",
    shared_expert_gate_prefix="mlp.shared_expert_gate",
)

QWEN3_MOE_SPEC = ModelArchitectureSpec(
    name="qwen3_moe",
    expert_key_template="model.layers.{layer}.mlp.experts.{expert}.{proj}.weight",
    expert_proj_names={"gate_up": "gate_up_proj", "down": "down_proj"},
    router_prefix="mlp.gate",
    experts_prefix="mlp.experts",
    router_use_softmax=True,
    normalize_topk_prob=False,
    use_qk_norm=True,
    experts_are_packed=True,
)

QWEN3_MOE_UNPACKED_SPEC = ModelArchitectureSpec(
    name="qwen3_moe",
    expert_key_template="model.layers.{layer}.mlp.experts.{expert}.{proj}.weight",
    expert_proj_names={"gate": "gate_proj", "up": "up_proj", "down": "down_proj"},
    router_prefix="mlp.gate",
    experts_prefix="mlp.experts",
    router_use_softmax=True,
    normalize_topk_prob=False,
    use_qk_norm=True,
    experts_are_packed=False,
)


def infer_architecture(hf_config) -> ModelArchitectureSpec:
    """Pick the spec from an HF-style config (config.py:204-220)."""
    model_type = getattr(hf_config, "model_type", "")
    architectures = [a.lower() for a in getattr(hf_config, "architectures", []) or []]
    if model_type == "mixtral":
        return MIXTRAL_SPEC
    if model_type == "qwen2_moe" or any("qwen2moe" in a for a in architectures):
        return QWEN2_MOE_SPEC
    if model_type == "qwen3_moe" or any("qwen3moe" in a for a in architectures):
        return QWEN3_MOE_SPEC
    if getattr(hf_config, "shared_expert_intermediate_size", None) is not None:
        return QWEN2_MOE_SPEC
    return MIXTRAL_SPEC


def routing_flags(hf_config) -> dict:
    """HybridMoE routing kwargs for an HF-style config (spec flags + norm_topk_prob override)."""
    arch = infer_architecture(hf_config)
    norm = getattr(hf_config, "norm_topk_prob", None)
    return {
        "router_use_softmax": arch.router_use_softmax,
        "normalize_topk_prob": arch.normalize_topk_prob if norm is None else bool(norm),
        "experts_are_packed": arch.experts_are_packed,
        "expert_key_template": arch.expert_key_template,
        "expert_proj_names": dict(arch.expert_proj_names),
    }
