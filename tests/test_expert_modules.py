"""The expert modules' plain torch forward (nano_ktrans/layers/expert_mlp.py:
20-23, 37-41) against the oracle's SwiGLU expert, on the CPU.

HybridMoE never calls these forwards (its expert math runs in the HIP
kernels); they exist so that a ``gpu_experts`` ModuleDict built from them can
be called expert by expert, as the reference's per-expert loop does
(nano_ktrans/layers/hybrid_moe.py:3501-3533)."""
import numpy as np
import pytest
import torch

import oracle as O
from nano_ktrans_amd.layers.expert_mlp import (PackedSparseExpertMLP, SparseExpertMLP, build_expert_module,
                                               load_expert_weights)


def _weights(H, I, seed):
    g = torch.Generator().manual_seed(seed)
    return {"gate": torch.randn(I, H, generator=g) * 0.05, "up": torch.randn(I, H, generator=g) * 0.05,
            "down": torch.randn(H, I, generator=g) * 0.05}


@pytest.mark.parametrize("packed", [False, True])
def test_expert_forward_matches_oracle(packed):
    H, I = 256, 384
    w = _weights(H, I, 5)
    m = build_expert_module(hidden_size=H, intermediate_size=I, hidden_act="silu", experts_are_packed=packed)
    assert isinstance(m, PackedSparseExpertMLP if packed else SparseExpertMLP)
    load_expert_weights(m, w)
    x = torch.randn(7, H, generator=torch.Generator().manual_seed(6))
    with torch.no_grad():
        got = m(x).numpy()
    ref = O.expert_forward(x.numpy(), O.Expert(w["gate"].numpy(), w["up"].numpy(), w["down"].numpy()))
    assert O.rel_l2(got, ref) <= 1e-5
    # the packed module's gate rows come first: swapping gate and up changes the result
    if packed:
        m2 = build_expert_module(hidden_size=H, intermediate_size=I, hidden_act="silu", experts_are_packed=True)
        load_expert_weights(m2, {"gate": w["up"], "up": w["gate"], "down": w["down"]})
        with torch.no_grad():
            assert O.rel_l2(m2(x).numpy(), ref) > 1e-2


def test_packed_and_unpacked_agree_and_keep_leading_dims():
    H, I = 128, 256
    w = _weights(H, I, 8)
    a = SparseExpertMLP(H, I)
    b = PackedSparseExpertMLP(H, I)
    load_expert_weights(a, w)
    load_expert_weights(b, w)
    x = torch.randn(2, 3, H, generator=torch.Generator().manual_seed(9))
    with torch.no_grad():
        ya, yb = a(x), b(x)
    assert ya.shape == (2, 3, H)
    assert np.allclose(ya.numpy(), yb.numpy(), rtol=1e-5, atol=1e-6)
