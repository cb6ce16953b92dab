"""The reference's CPU expert loop in torch, for the timed CPU baseline.
TEST INFRASTRUCTURE ONLY: ``bench.py``'s ``cpu_baseline`` leg and ``tests/``
use it; the product package never imports it.

A torch restatement (torch's CPU kernels on the host's threads, as the
reference runs it) of:

* ``matvec_grouped``  nano_ktrans/kernels/quantized_ops.py:86-124: per group
                      g of the packed words, unpack, ``(q - zero) * scale``,
                      ``out += linear(x[:, g], w_g)`` in fp32, groups ascending
* ``expert_gptq``     nano_ktrans/kernels/cpu_moe.py:419-450:
                      ``down(silu(gate(x)) * up(x))`` in fp32
* ``moe_loop``        nano_ktrans/kernels/cpu_moe.py:491-539: experts in
                      ascending id, each on the tokens that picked it,
                      ``index_add_`` of ``y * w`` into an fp32 output; dense
                      (unquantized fp32) experts through ``linear`` as
                      nano_ktrans/layers/expert_mlp.py:20-23 computes them

Routing comes from the oracle (``oracle.route``), the same ids and weights
the GPU path is checked against.  ``tests/test_oracle.py`` pins ``moe_loop``
against ``oracle.moe_forward``.
"""
from __future__ import annotations

from typing import List, Optional

import numpy as np
import torch
import torch.nn.functional as F

import oracle as O


class TorchQWeight:
    """A GPTQ-layout weight as torch tensors: qweight int32 [out, in*bits/32],
    scales fp32 [out, groups]."""

    def __init__(self, qw: "O.QWeight"):
        self.qweight = torch.from_numpy(np.ascontiguousarray(qw.qweight))
        self.scales = torch.from_numpy(np.ascontiguousarray(qw.scales, dtype=np.float32))
        self.bits = qw.bits
        self.group_size = qw.group_size
        self.per_word = 32 // qw.bits
        self.out_dim = self.qweight.shape[0]
        self.in_dim = self.qweight.shape[1] * self.per_word
        self.shifts = torch.arange(self.per_word, dtype=torch.int32) * self.bits


def matvec_grouped(x: torch.Tensor, w: TorchQWeight) -> torch.Tensor:
    out = torch.zeros(x.shape[0], w.out_dim, dtype=torch.float32)
    zero = float(1 << (w.bits - 1))
    mask = (1 << w.bits) - 1
    for g in range(w.scales.shape[1]):
        s, e = g * w.group_size, min((g + 1) * w.group_size, w.in_dim)
        words = w.qweight[:, s // w.per_word:(e + w.per_word - 1) // w.per_word]
        q = ((words.unsqueeze(-1) >> w.shifts) & mask).reshape(w.out_dim, -1).to(torch.float32)
        out += F.linear(x[:, s:e], (q - zero) * w.scales[:, g:g + 1])
    return out


def _lin(x: torch.Tensor, w) -> torch.Tensor:
    if isinstance(w, TorchQWeight):
        return matvec_grouped(x, w)
    return F.linear(x, w)


def to_torch_expert(ex: "O.Expert"):
    conv = lambda w: TorchQWeight(w) if isinstance(w, O.QWeight) else torch.from_numpy(
        np.ascontiguousarray(w, dtype=np.float32))
    return conv(ex.gate), conv(ex.up), conv(ex.down)


def expert_gptq(x: torch.Tensor, ex) -> torch.Tensor:
    gate, up, down = ex
    return _lin(F.silu(_lin(x, gate)) * _lin(x, up), down)


def moe_loop(x: np.ndarray, ids: np.ndarray, weights: np.ndarray, experts: List[Optional[tuple]]) -> np.ndarray:
    """fp32 output [T, H] of the routed experts (experts[e] from ``to_torch_expert``;
    None for an expert no token picked)."""
    xt = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    idt = torch.from_numpy(np.ascontiguousarray(ids)).to(torch.long)
    wt = torch.from_numpy(np.ascontiguousarray(weights, dtype=np.float32))
    out = torch.zeros_like(xt)
    for e in range(len(experts)):
        match = idt == e
        tokens = torch.where(match.any(dim=1))[0]
        if tokens.numel() == 0:
            continue
        y = expert_gptq(xt[tokens], experts[e])
        r, c = torch.where(match[tokens])
        out.index_add_(0, tokens[r], y[r] * wt[tokens[r], c].unsqueeze(1))
    return out.numpy()
