"""Expert weight containers with the reference's module names and parameter layout.

``SparseExpertMLP`` (w1 gate [I, H], w3 up [I, H], w2 down [H, I]) and
``PackedSparseExpertMLP`` (gate_up_proj [2I, H] = cat([gate; up]), down_proj
[H, I]) match nano_ktrans/layers/expert_mlp.py:9-41 so that a caller's
``gpu_experts`` ModuleDict and checkpoint names load unchanged.  ``HybridMoE``
only reads their parameters; its expert math runs in the HIP kernels.  Each
module keeps a plain torch ``forward`` (expert_mlp.py:20-23, 37-41) so that a
caller's own per-expert loop can still call ``gpu_experts[str(e)](x)``.
"""
from __future__ import annotations

from typing import Dict

import torch
from torch import nn


class SparseExpertMLP(nn.Module):
    def __init__(self, hidden_size: int, intermediate_size: int, hidden_act: str = "silu"):
        super().__init__()
        self.hidden_dim = hidden_size
        self.ffn_dim = intermediate_size
        self.hidden_act = hidden_act
        self.w1 = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.w2 = nn.Linear(intermediate_size, hidden_size, bias=False)
        self.w3 = nn.Linear(hidden_size, intermediate_size, bias=False)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """act(w1 x) * (w3 x), then w2; in the parameters' dtype."""
        act = getattr(nn.functional, self.hidden_act)
        return self.w2(act(self.w1(hidden_states)) * self.w3(hidden_states))

    def projections(self) -> Dict[str, torch.Tensor]:
        return {"gate": self.w1.weight, "up": self.w3.weight, "down": self.w2.weight}


class PackedSparseExpertMLP(nn.Module):
    def __init__(self, hidden_size: int, intermediate_size: int, hidden_act: str = "silu"):
        super().__init__()
        self.hidden_dim = hidden_size
        self.intermediate_size = intermediate_size
        self.hidden_act = hidden_act
        self.gate_up_proj = nn.Parameter(torch.empty(2 * intermediate_size, hidden_size))
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """One product with the packed [2I, H] weight, split into gate (first I
        outputs) and up (last I), then act(gate) * up through down_proj."""
        act = getattr(nn.functional, self.hidden_act)
        gate_up = nn.functional.linear(hidden_states, self.gate_up_proj)
        gate, up = gate_up[..., : self.intermediate_size], gate_up[..., self.intermediate_size:]
        return self.down_proj(act(gate) * up)

    def projections(self) -> Dict[str, torch.Tensor]:
        gate, up = self.gate_up_proj.chunk(2, dim=0)
        return {"gate": gate, "up": up, "down": self.down_proj.weight}


def build_expert_module(*, hidden_size: int, intermediate_size: int, hidden_act: str,
                        experts_are_packed: bool) -> nn.Module:
    if experts_are_packed:
        return PackedSparseExpertMLP(hidden_size, intermediate_size, hidden_act)
    return SparseExpertMLP(hidden_size, intermediate_size, hidden_act)


def load_expert_weights(module: nn.Module, weights: Dict[str, torch.Tensor]) -> None:
    """Copy {"gate", "up", "down"} tensors into an expert module (expert_mlp.py:56-85)."""
    with torch.no_grad():
        if isinstance(module, PackedSparseExpertMLP):
            gate_up = torch.cat([weights["gate"], weights["up"]], dim=0)
            module.gate_up_proj.copy_(gate_up.to(module.gate_up_proj.device, module.gate_up_proj.dtype))
            module.down_proj.weight.copy_(weights["down"].to(module.down_proj.weight.device,
                                                             module.down_proj.weight.dtype))
            return
        if not isinstance(module, SparseExpertMLP):
            raise TypeError(f"Unsupported expert module type: {type(module)!r}")
        module.w1.weight.copy_(weights["gate"].to(module.w1.weight.device, module.w1.weight.dtype))
        module.w2.weight.copy_(weights["down"].to(module.w2.weight.device, module.w2.weight.dtype))
        module.w3.weight.copy_(weights["up"].to(module.w3.weight.device, module.w3.weight.dtype))


def load_shared_expert_modules(weight_path: str, layer_idx: int, spec, *, hidden_size: int,
                               shared_intermediate_size: int, dtype: torch.dtype = torch.bfloat16):
    """The Qwen2-MoE shared expert and its gate from a safetensors checkpoint.

    Keys follow the architecture spec (nano_ktrans/models/config.py:37-49):
    ``spec.shared_expert_key_template`` with proj in {gate, up, down} for the
    dense shared MLP, read into a ``SparseExpertMLP`` (gate -> w1, up -> w3,
    down -> w2: the renames of nano_ktrans/models/mixtral.py:418-422), and
    ``model.layers.{layer}.{spec.shared_expert_gate_prefix}.weight`` [1, H] for
    ``shared_expert_gate`` = nn.Linear(H, 1, bias=False).  Returns
    (shared_expert, shared_expert_gate) in ``dtype``, on the CPU."""
    from ..kernels.weight_loader import ExpertWeightLoader

    if not spec.has_shared_expert:
        raise ValueError(f"architecture {spec.name!r} has no shared expert")
    loader = ExpertWeightLoader(weight_path)
    tpl = spec.shared_expert_key_template
    weights = {p: loader.load_tensor(tpl.format(layer=layer_idx, proj=p)) for p in ("gate", "up", "down")}
    expert = SparseExpertMLP(hidden_size, shared_intermediate_size)
    if tuple(weights["gate"].shape) != (shared_intermediate_size, hidden_size):
        raise ValueError(f"shared expert gate_proj is {tuple(weights['gate'].shape)}, expected "
                         f"{(shared_intermediate_size, hidden_size)}")
    load_expert_weights(expert, weights)
    gate = nn.Linear(hidden_size, 1, bias=False)
    gw = loader.load_tensor(f"model.layers.{layer_idx}.{spec.shared_expert_gate_prefix}.weight")
    with torch.no_grad():
        gate.weight.copy_(gw.reshape(1, hidden_size).to(gate.weight.dtype))
    return expert.to(dtype), gate.to(dtype)
