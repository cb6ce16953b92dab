"""K1 + K2 on the GPU against the oracle: routing ids and weights, per-expert counts,
offsets and the permutation must be bit-exact."""
import sys

import numpy as np
import pytest
import torch

import oracle as O
from moe_cases import CONFIGS, build_inputs, build_layer, check_router_logits

pytestmark = pytest.mark.gpu


def announce(msg):
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _router_only(E, k, softmax, renorm, act_dtype, device, max_tokens=8192, hidden=128):
    from nano_ktrans_amd.native_moe import NativeMoE

    wfmt = "f32" if act_dtype == torch.float32 else "bf16"
    return NativeMoE(num_experts=E, top_k=k, hidden_size=hidden, intermediate_size=128, weight_format=wfmt,
                     act_dtype=act_dtype, use_softmax=softmax, renorm=renorm, max_tokens=max_tokens,
                     device=device)



def _check_route(native, logits, k, softmax, renorm, bf16):
    E = logits.shape[1]
    ids, w, counts, offsets, perm, inv = native.route(logits)
    torch.cuda.synchronize()
    oids, ow = O.route(logits.float().cpu().numpy(), k, softmax, renorm, bf16)
    ocounts, ooffsets, operm, oinv = O.group(oids, E)
    g_ids = ids.cpu().numpy()
    g_w = w.cpu().numpy()
    bad = np.argwhere(g_ids != oids)
    assert bad.size == 0, f"ids differ at {bad[:5].tolist()}: gpu {g_ids[bad[0][0]]} oracle {oids[bad[0][0]]}"
    assert np.array_equal(g_w.view(np.uint32), ow.view(np.uint32)), \
        f"weights differ: max |d| = {np.max(np.abs(g_w - ow))}"
    assert np.array_equal(counts.cpu().numpy(), ocounts)
    assert np.array_equal(offsets.cpu().numpy(), ooffsets)
    assert np.array_equal(perm.cpu().numpy(), operm)
    assert np.array_equal(inv.cpu().numpy(), oinv)


@pytest.mark.parametrize("name,T", [
    ("tiny_mixtral_fp32", 16), ("tiny_mixtral_fp32", 1),
    ("qwen3_int4", 1), ("qwen3_int4", 4), ("qwen3_int4", 16),
    ("qwen3_int8", 512), ("qwen3_int8", 4096),
    ("mixtral_int4", 1), ("mixtral_int4", 16), ("mixtral_int4", 2048),
    ("qwen15_int8_shared", 1), ("qwen15_int8_shared", 16), ("qwen15_int8_shared", 1024),
])
def test_route_matches_oracle_on_benchmark_configs(gpu_device, name, T):
    cfg = CONFIGS[name]
    announce(f"route {name} T={T}")
    # the router weights are all routing needs: build them alone
    g = torch.Generator().manual_seed(cfg.seed)
    router = torch.randn(cfg.E, cfg.H, generator=g) * 0.02
    from moe_cases import Layer
    layer = Layer(cfg, router, [])
    x, logits = build_inputs(layer, T, seed=100 + T)
    native = _router_only(cfg.E, cfg.k, cfg.softmax, cfg.renorm, cfg.act_dtype, gpu_device)
    _check_route(native, logits.to(gpu_device), cfg.k, cfg.softmax, cfg.renorm, cfg.act == "bf16")


@pytest.mark.parametrize("E,k", [(8, 1), (8, 2), (60, 4), (64, 8), (100, 6), (128, 8), (128, 16), (256, 8)])
@pytest.mark.parametrize("softmax,renorm", [(True, True), (True, False), (False, True)])
@pytest.mark.parametrize("act_dtype", [torch.bfloat16, torch.float32])
def test_route_ties_and_edges(gpu_device, E, k, softmax, renorm, act_dtype):
    announce(f"route edges E={E} k={k} softmax={softmax} renorm={renorm} {act_dtype}")
    rng = np.random.default_rng(E * 100 + k)
    T = 97
    cases = []
    # heavy ties: logits on a coarse grid
    cases.append(np.round(rng.standard_normal((T, E)) * 2) / 2)
    # all equal
    cases.append(np.zeros((5, E)))
    # one hot
    oh = np.zeros((min(E, 40), E))
    oh[np.arange(oh.shape[0]), np.arange(oh.shape[0])] = 5.0
    cases.append(oh)
    # very wide spread: exp underflows to subnormals and zero
    cases.append(rng.standard_normal((T, E)) * 60.0)
    # signed zeros and negatives
    z = np.zeros((3, E))
    z[:, ::2] = -0.0
    z[:, 1] = -1.0
    cases.append(z)
    native = _router_only(E, k, softmax, renorm, act_dtype, gpu_device)
    for c in cases:
        logits = torch.from_numpy(c.astype(np.float32)).to(act_dtype).to(gpu_device)
        _check_route(native, logits, k, softmax, renorm, act_dtype == torch.bfloat16)


@pytest.mark.parametrize("E,k", [(256, 16), (128, 16), (60, 4), (8, 2)])
@pytest.mark.parametrize("T", [63, 64, 65])
def test_route_fused_limits(gpu_device, E, k, T):
    """The one-workgroup route + group at its limits (T = 64 tokens, T k up to
    1024 pairs, E up to 256) and the first size past it, on tie-heavy logits."""
    announce(f"route fused limits E={E} k={k} T={T}")
    rng = np.random.default_rng(E + 7 * k + T)
    native = _router_only(E, k, True, True, torch.bfloat16, gpu_device)
    for c in (np.round(rng.standard_normal((T, E)) * 2) / 2, rng.standard_normal((T, E))):
        logits = torch.from_numpy(c.astype(np.float32)).to(torch.bfloat16).to(gpu_device)
        _check_route(native, logits, k, True, True, True)


def test_route_repeatable(gpu_device):
    announce("route repeatable")
    native = _router_only(128, 8, True, True, torch.bfloat16, gpu_device)
    logits = (torch.randn(4096, 128, generator=torch.Generator().manual_seed(5)) * 0.9).to(torch.bfloat16)
    logits = logits.to(gpu_device)
    first = [t.clone() for t in native.route(logits)]
    for _ in range(3):
        again = native.route(logits)
        for a, b in zip(first, again):
            assert torch.equal(a, b)


@pytest.mark.parametrize("name,T", [
    ("qwen3_int4", 1), ("qwen3_int4", 16), ("qwen3_int4", 64), ("qwen3_int4", 100), ("qwen3_int8", 1024),
    ("mixtral_int4", 16), ("qwen15_int8_shared", 1), ("qwen15_int8_shared", 64), ("qwen15_int8_shared", 300),
])
def test_route_hidden_matches_oracle(gpu_device, name, T):
    """Router GEMV fused with K1 + K2 (one launch up to 64 tokens, three past
    it): bf16 logits against the oracle's single rounding of the exact dot
    products (check_router_logits), and routing / grouping of those logits
    bit-exact; the workspace's whole sync area (status words and the single
    launch's counters and published masks) is left zero."""
    from nano_ktrans_amd import _native as N
    cfg = CONFIGS[name]
    announce(f"route_hidden {name} T={T}")
    g = torch.Generator().manual_seed(cfg.seed + 50)
    gate = (torch.randn(cfg.E, cfg.H, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(T, cfg.H, generator=g).to(torch.bfloat16)
    native = _router_only(cfg.E, cfg.k, cfg.softmax, cfg.renorm, torch.bfloat16, gpu_device, hidden=cfg.H)
    native.load_router(gate)
    logits, ids, w, counts, offsets, perm, inv = native.route_hidden(x.to(gpu_device))
    torch.cuda.synchronize()
    g_logits = logits.float().cpu().numpy()
    check_router_logits(g_logits, x.float().numpy(), gate.float().numpy())
    oids, ow = O.route(g_logits, cfg.k, cfg.softmax, cfg.renorm, True)
    ocounts, ooffsets, operm, oinv = O.group(oids, cfg.E)
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), ow.view(np.uint32))
    assert np.array_equal(counts.cpu().numpy(), ocounts)
    assert np.array_equal(offsets.cpu().numpy(), ooffsets)
    assert np.array_equal(perm.cpu().numpy(), operm)
    assert np.array_equal(inv.cpu().numpy(), oinv)
    # the whole sync area (the single launch's counters and published masks,
    # the status word) is left zero
    assert not native.workspace(T)[:N.SYNC_AREA_BYTES].any()
    native.check_status()


def test_route_hidden_single_launch_replays(gpu_device):
    """The single-launch router + route + group captured in a HIP graph: every
    replay (its counters reset by the call before, as every call leaves them) routes its own logits --
    eager calls with other inputs on the same workspace run between replays --
    and equals the eager result bit for bit."""
    from nano_ktrans_amd import _native as N
    announce("route_hidden graph replays")
    cfg = CONFIGS["qwen3_int4"]
    T = 16
    g = torch.Generator().manual_seed(77)
    gate = (torch.randn(cfg.E, cfg.H, generator=g) * 0.02).to(torch.bfloat16)
    xa = torch.randn(T, cfg.H, generator=g).to(torch.bfloat16).to(gpu_device)
    xb = torch.randn(T, cfg.H, generator=g).to(torch.bfloat16).to(gpu_device)
    native = _router_only(cfg.E, cfg.k, cfg.softmax, cfg.renorm, torch.bfloat16, gpu_device, hidden=cfg.H)
    native.load_router(gate)
    ref_a = [t.clone() for t in native.route_hidden(xa)]
    ref_b = [t.clone() for t in native.route_hidden(xb)]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        native.route_hidden(xa)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        views = native.route_hidden(xa)
    for r in range(4):
        got_b = [t.clone() for t in native.route_hidden(xb)]
        torch.cuda.synchronize()
        for a, b in zip(got_b, ref_b):
            assert torch.equal(a, b)
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(views, ref_a):
            assert torch.equal(a, b), f"replay {r}"
    assert not native.workspace(T)[:N.SYNC_AREA_BYTES].any()
    native.check_status()


def test_route_hidden_rejects_missing_router_and_fp32(gpu_device):
    from nano_ktrans_amd._native import NativeError

    native = _router_only(8, 2, True, True, torch.bfloat16, gpu_device, hidden=256)
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(NativeError, match="router weight not bound"):
        native.route_hidden(x)
    f32 = _router_only(8, 2, True, True, torch.float32, gpu_device, hidden=256)
    with pytest.raises(ValueError, match="bf16 activations"):
        f32.load_router(torch.zeros(8, 256))


@pytest.mark.parametrize("T", [4, 40])
def test_rejected_forward_hidden_launches_nothing(gpu_device, T):
    """nkt_moe_forward_hidden called with a null output is rejected before
    any launch (a batch of up to 16 tokens would otherwise start with the
    router's own launch): the error names the output and the router-logits
    region keeps its contents."""
    from nano_ktrans_amd import _native as N

    announce(f"forward_hidden rejected before launching T={T}")
    native = _router_only(16, 2, True, True, torch.bfloat16, gpu_device, max_tokens=64, hidden=256)
    native.load_router((torch.randn(16, 256, generator=torch.Generator().manual_seed(5)) * 0.02).to(torch.bfloat16))
    ws = native.workspace(T)
    region = native.region(T, N.WS_ROUTER_LOGITS, torch.int16, (T, 16))
    region.fill_(0x1234)
    torch.cuda.synchronize()
    x = torch.randn(T, 256, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(gpu_device)
    with pytest.raises(N.NativeError, match="null .*output"):
        native.err.check(native.lib.nkt_moe_forward_hidden(native.handle, x.data_ptr(), T, None, ws.data_ptr(),
                                                           ws.numel(), native._stream(), native.err.buf,
                                                           native.err.size), "nkt_moe_forward_hidden")
    torch.cuda.synchronize()
    assert bool((region == 0x1234).all())
