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


@pytest.mark.parametrize("name,E,T1,T2", [("qwen3_int4", 32, 16, 5), ("small_int8_shared", None, 16, 5),
                                          # the second call: the self-routing gate_up (3 tokens, 128 experts)
                                          ("qwen3_int4", None, 16, 3),
                                          # 17 .. 64 tokens: the several-workgroup routing launch, whose
                                          # counters and published masks live in the scratch's sync area
                                          ("qwen3_int4", None, 40, 24)])
def test_noalloc_matches_forward(gpu_device, name, E, T1, T2):
    layer = build_layer(CONFIGS[name], device="cuda", num_experts=E)
    native = native_layer(layer, torch.device("cuda"), max_tokens=64)
    for T, seed in ((T1, 51), (T2, 52)):
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


@pytest.mark.parametrize("name,E,T", [("qwen3_int4", 32, 16), ("small_int8_shared", None, 1), ("qwen3_int4", None, 40)])
def test_noalloc_captures_in_a_graph(gpu_device, name, E, T):
    """The call is capture-safe: captured in a HIP graph in global capture
    mode (where a hipMalloc, hipFree or stream creation anywhere in the
    process fails the capture), it replays bit for bit like the eager call,
    replay after replay, with eager calls of other inputs on the shared
    scratch in between; and the device's free memory (hipMemGetInfo, which
    sees the library's own allocations, unlike torch's allocator counters)
    is the same before and after eager calls."""
    announce(f"noalloc graph capture {name} T={T}")
    layer = build_layer(CONFIGS[name], device="cuda", num_experts=E)
    native = native_layer(layer, torch.device("cuda"), max_tokens=64)
    x, logits = build_inputs(layer, T, seed=55, device="cuda")
    x2, l2 = build_inputs(layer, T, seed=56, device="cuda")
    ref = native.forward(x, logits).clone()
    ref2 = native.forward(x2, l2).clone()
    out = torch.empty_like(ref)
    out2 = torch.empty_like(ref)
    native.forward_noalloc(x, logits, out)  # first call on the device: the scratch address lookup
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        native.forward_noalloc(x2, l2, out2)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free_before
    assert torch.equal(out2, ref2)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="global"):
        native.forward_noalloc(x, logits, out)
    for r in range(3):
        out.zero_()
        native.forward_noalloc(x2, l2, out2)  # eager work on the same scratch
        torch.cuda.synchronize()
        assert torch.equal(out2, ref2)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r}"


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
