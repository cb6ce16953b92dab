"""nkt_moe_forward_noalloc: the layer with the library's static per-GPU
scratch as its workspace (no allocation in the call) against
nkt_moe_forward on the same inputs, two calls in a row with the second
smaller, and the oracle; a batch whose workspace exceeds the scratch is
rejected with a message."""
import sys

import numpy as np
import pytest
import torch

from moe_cases import CONFIGS, build_inputs, build_layer, compare, native_layer, oracle_forward

pytestmark = pytest.mark.gpu


def announce(msg):
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


@pytest.mark.parametrize("name,E", [("qwen3_int4", 32), ("small_int8_shared", None)])
def test_noalloc_matches_forward(gpu_device, name, E):
    layer = build_layer(CONFIGS[name], device="cuda", num_experts=E)
    native = native_layer(layer, torch.device("cuda"), max_tokens=64)
    for T, seed in ((16, 51), (5, 52)):
        announce(f"noalloc {name} T={T}")
        x, logits = build_inputs(layer, T, seed=seed, device="cuda")
        ref = native.forward(x, logits).clone()
        out = torch.full_like(ref, float("nan"))
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        native.forward_noalloc(x, logits, out)
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        assert torch.equal(out, ref)
        compare(out.float().cpu().numpy(), oracle_forward(layer, x, logits), layer.cfg)


def test_noalloc_rejects_batches_beyond_the_scratch(gpu_device):
    from nano_ktrans_amd import _native as N

    announce("noalloc rejects a batch larger than the scratch")
    layer = build_layer(CONFIGS["qwen3_int4"], device="cuda", num_experts=32)
    native = native_layer(layer, torch.device("cuda"), max_tokens=2048)
    T = 2048
    assert native.workspace_bytes(T) > N.NOALLOC_SCRATCH_BYTES
    x, logits = build_inputs(layer, T, seed=53, device="cuda")
    out = torch.empty(T, layer.cfg.H, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(N.NativeError, match="static scratch"):
        native.forward_noalloc(x, logits, out)
    # a batch that fits still runs after the rejection
    x, logits = build_inputs(layer, 8, seed=54, device="cuda")
    out = torch.empty(8, layer.cfg.H, dtype=torch.bfloat16, device="cuda")
    assert torch.equal(native.forward_noalloc(x, logits, out), native.forward(x, logits))
