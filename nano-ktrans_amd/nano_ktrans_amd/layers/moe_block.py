"""The MoE half of a decoder layer as one fused call.

nano_ktrans/models/mixtral.py:206-223 runs, after attention:

    residual = hidden_states
    hidden_states = self.post_attention_layernorm(hidden_states)   # norm.py:11-17
    router_logits = self.gate(hidden_states)
    hidden_states = self.hybrid_moe(hidden_states, router_logits) (+ shared expert)
    hidden_states = residual + hidden_states

``FusedMoEBlock(norm, moe)(hidden_states)`` computes the same with the RMSNorm,
router GEMV, routing, experts, shared expert, combine and residual add in
the library's launches (``nkt_moe_forward_block``): no bf16 round trip of the
MoE output before the residual add, and no separate normalisation or gate
launches.  ``moe`` is a HybridMoE built with ``gate=``; bf16 activations.
"""
from __future__ import annotations

import torch
from torch import nn

from .hybrid_moe import HybridMoE


class FusedMoEBlock(nn.Module):
    def __init__(self, post_attention_layernorm: nn.Module, moe: HybridMoE):
        super().__init__()
        if moe.gate is None:
            raise ValueError("FusedMoEBlock needs a HybridMoE built with gate=")
        if moe.offload_backend is not None:
            raise ValueError("the fused block runs every expert in HBM (no offload backend)")
        self.norm = post_attention_layernorm
        self.moe = moe

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.dtype != torch.bfloat16:
            raise ValueError("FusedMoEBlock needs bf16 hidden states")
        native = self.moe._ensure(hidden_states)
        shape = hidden_states.shape
        out = native.forward_block(hidden_states.reshape(-1, self.moe.hidden_size), self.norm.weight.detach(),
                                   float(self.norm.eps))
        return out.view(shape)
