"""Expert weight containers with the reference's module names and parameter layout.

``SparseExpertMLP`` (w1 gate [I, H], w3 up [I, H], w2 down [H, I]) and
``PackedSparseExpertMLP`` (gate_up_proj [2I, H] = cat([gate; up]), down_proj
[H, I]) match nano_ktrans/layers/expert_mlp.py:9-41 so that a caller's
``gpu_experts`` ModuleDict and checkpoint names load unchanged.  ``HybridMoE``
only reads their parameters; the expert math runs in the HIP kernels.
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
