"""Expert compute on routing the caller supplies (nkt_moe_route_given /
nkt_moe_forward_routed), the provider side of the reference's offload
contract (nano_ktrans/kernels/offload_backend.py:40-52; kt-kernel's
forward_task, nano_ktrans/kernels/cpu_moe.py:570-592), against the oracle's
expert loop on the same routing (oracle.moe_forward_given, restating
cpu_moe.py:491-539).

Routing comes from torch.topk over tie-heavy softmax probabilities (logits
rounded to a coarse grid, so many experts share a value and torch's own tie
order decides), renormalised, in fp32.  Tolerances as moe_cases.compare; the
ids, counts and permutation the library derives are bit-exact."""
import sys

import numpy as np
import pytest
import torch

import oracle as O
from moe_cases import CONFIGS, _to_oracle, build_inputs, build_layer, compare, native_layer

pytestmark = pytest.mark.gpu


def announce(msg):
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


_LAYERS = {}


def _layer(name, E=None, I=None):
    key = (name, E, I)
    if key not in _LAYERS:
        cfg = CONFIGS[name]
        if I is not None:
            from dataclasses import replace
            cfg = replace(cfg, I=I)
        _LAYERS.clear()
        layer = build_layer(cfg, device="cuda", num_experts=E)
        _LAYERS[key] = (layer, native_layer(layer, torch.device("cuda")))
    return _LAYERS[key]


def _topk_routing(logits, k, grid=0.5):
    """ids int64 [T, k] and renormalised fp32 weights from torch.topk over the
    softmax of logits snapped to multiples of ``grid`` (tie-heavy)."""
    snapped = torch.round(logits.float() / grid) * grid
    p = torch.softmax(snapped, dim=-1)
    w, ids = torch.topk(p, k, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return ids, w.float()


def _oracle_given(layer, x, ids, w):
    experts = [O.Expert(_to_oracle(e["gate"]), _to_oracle(e["up"]), _to_oracle(e["down"])) for e in layer.experts]
    shared = None
    if layer.shared is not None:
        shared = O.Expert(_to_oracle(layer.shared["gate"]), _to_oracle(layer.shared["up"]),
                          _to_oracle(layer.shared["down"]))
    return O.moe_forward_given(x.float().cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), experts, shared=shared,
                               shared_gate=None if layer.shared_gate is None else layer.shared_gate.cpu().numpy())


@pytest.mark.parametrize("name,E,I,T", [
    ("qwen3_int4", None, None, 1), ("qwen3_int4", None, None, 4), ("qwen3_int4", None, None, 16),
    ("qwen3_int4", 32, None, 300),                 # int4 prefill form, the large-batch grouping
    ("qwen3_int8", 32, None, 512),                 # int8 prefill pipeline (fp16 copy made by gate_up's pre-pass)
    ("mixtral_int4", None, None, 1), ("mixtral_int4", None, 1024, 200),
    ("qwen15_int8_shared", None, None, 1),         # shared expert as chunks of the single-token launches
    ("qwen15_int8_shared", None, None, 16),        # ... of the routed decode launches
    ("qwen15_int8_shared", None, None, 200),       # shared expert on the side stream
    ("tiny_mixtral_fp32", None, None, 16),
])
def test_forward_routed_matches_oracle(gpu_device, name, E, I, T):
    from nano_ktrans_amd import _native as N
    announce(f"forward_routed {name} E={E} I={I} T={T}")
    layer, native = _layer(name, E, I)
    cfg = layer.cfg
    x, logits = build_inputs(layer, T, seed=81, device="cuda")
    ids, w = _topk_routing(logits, cfg.k)
    out = native.forward_routed(x, ids, w)
    torch.cuda.synchronize()
    got_ids = native.region(T, N.WS_TOPK_IDS, torch.int32, (T, cfg.k)).cpu()
    assert torch.equal(got_ids, ids.to(torch.int32).cpu())
    assert np.array_equal(native.region(T, N.WS_PERM, torch.int32, (T * cfg.k,)).cpu().numpy(),
                          O.group(ids.cpu().numpy(), cfg.E)[2])
    ref = _oracle_given(layer, x, ids, w)
    err_abs, err_rel = compare(out.float().cpu().numpy(), ref, cfg)
    announce(f"  max_abs={err_abs:.3e} rel_l2={err_rel:.3e}")
    assert native.status() == {"bad_routing": 0}


@pytest.mark.parametrize("name,E,T", [("qwen3_int4", None, 1), ("qwen3_int4", None, 16), ("qwen3_int8", 32, 512),
                                      ("qwen15_int8_shared", None, 16), ("mixtral_int4", None, 1)])
def test_forward_routed_on_own_routing_equals_forward(gpu_device, name, E, T):
    """Given the routing the library itself computes from the logits, the
    routed layer is the logits layer bit for bit; and the slots of a token may
    come in any order (the combine adds experts in ascending id)."""
    announce(f"forward_routed vs forward {name} E={E} T={T}")
    layer, native = _layer(name, E)
    x, logits = build_inputs(layer, T, seed=83, device="cuda")
    a = native.forward(x, logits).clone()
    ids, w, *_ = native.route(logits)
    ids, w = ids.to(torch.int64).clone(), w.clone()
    b = native.forward_routed(x, ids, w).clone()
    g = torch.Generator().manual_seed(5)
    perm = torch.stack([torch.randperm(layer.cfg.k, generator=g) for _ in range(T)]).to(ids.device)
    c = native.forward_routed(x, torch.gather(ids, 1, perm), torch.gather(w, 1, perm))
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(a, c)


@pytest.mark.parametrize("T", [3, 100])
def test_route_given_drops_bad_slots(gpu_device, T):
    """Ids outside [0, E) and a repeated id within a token: each such slot
    adds nothing (it takes the smallest id its token leaves unused, weight 0),
    the status word says so, check_status raises and clears it, and a clean
    call leaves it clear.  T = 3: the one-workgroup grouping; T = 100: the
    many-workgroup one."""
    from nano_ktrans_amd import _native as N
    announce(f"route_given bad slots qwen3_int4 E=32 T={T}")
    layer, native = _layer("qwen3_int4", 32)
    cfg = layer.cfg
    x, logits = build_inputs(layer, T, seed=85, device="cuda")
    ids, w = _topk_routing(logits, cfg.k)
    bad = ids.clone()
    bad[0, 2] = cfg.E          # out of range
    bad[1, 0] = -1             # negative
    bad[2, 5] = bad[2, 1]      # repeats slot 1 of the same token
    bad[2, 7] = 1 << 40        # far out of range (int64)
    out = native.forward_routed(x, bad, w)
    torch.cuda.synchronize()
    assert native.status()["bad_routing"] == 1
    # the sanitised routing the library used
    want = bad.cpu().numpy().copy()
    ww = w.cpu().numpy().copy()
    for t in range(T):
        kept = set()
        drop = []
        for j in range(cfg.k):
            e = int(want[t, j])
            if 0 <= e < cfg.E and e not in kept:
                kept.add(e)
            else:
                drop.append(j)
        for j in drop:
            f = min(set(range(cfg.E)) - kept)
            kept.add(f)
            want[t, j], ww[t, j] = f, 0.0
    got_ids = native.region(T, N.WS_TOPK_IDS, torch.int32, (T, cfg.k)).cpu().numpy()
    got_w = native.region(T, N.WS_TOPK_WEIGHTS, torch.float32, (T, cfg.k)).cpu().numpy()
    assert np.array_equal(got_ids, want) and np.array_equal(got_w, ww)
    ref = _oracle_given(layer, x, torch.from_numpy(want), torch.from_numpy(ww))
    compare(out.float().cpu().numpy(), ref, cfg)
    with pytest.raises(N.NativeError, match="bad_routing"):
        native.check_status()
    assert native.status()["bad_routing"] == 0
    native.forward_routed(x, ids, w)
    native.check_status()


@pytest.mark.parametrize("T", [1, 16, 300])
def test_hbm_offload_backend_serves_hybrid_moe(gpu_device, T):
    """HbmExpertBackend behind HybridMoE(offload_backend_impl=...): the
    experts with gpu_experts_mask False run in the backend's own layer from
    the routing HybridMoE submits (submit_forward / sync_forward on the
    caller's stream), the resident ones in HybridMoE's, and the sum matches
    the oracle's all-expert forward."""
    from torch import nn

    from moe_cases import Layer, MoEConfig, oracle_forward
    from nano_ktrans_amd.kernels.offload_backend import HbmExpertBackend
    from nano_ktrans_amd.layers.expert_mlp import SparseExpertMLP
    from nano_ktrans_amd.layers.hybrid_moe import HybridMoE
    from nano_ktrans_amd.models.config import MIXTRAL_SPEC
    from nano_ktrans_amd.native_moe import NativeMoE

    announce(f"HybridMoE + HbmExpertBackend T={T}")
    E, k, H, I = 16, 4, 2048, 768
    g = torch.Generator().manual_seed(600)
    experts = nn.ModuleDict()
    for e in range(E):
        m = SparseExpertMLP(H, I)
        with torch.no_grad():
            for p in m.parameters():
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
        experts[str(e)] = m.to(gpu_device, torch.bfloat16)
    mask = torch.tensor([e % 3 != 1 for e in range(E)])
    served = NativeMoE(num_experts=E, top_k=k, hidden_size=H, intermediate_size=I, weight_format="bf16",
                       act_dtype=torch.bfloat16, use_softmax=True, renorm=True, max_tokens=512, device=gpu_device)
    for e in range(E):
        if not mask[e]:
            served.load_expert(e, experts[str(e)].w1.weight, experts[str(e)].w3.weight, experts[str(e)].w2.weight)
    backend = HbmExpertBackend(served, mask)
    moe = HybridMoE(E, k, H, I, experts, mask, 0, "", router_use_softmax=True, normalize_topk_prob=True,
                    expert_key_template=MIXTRAL_SPEC.expert_key_template,
                    expert_proj_names=MIXTRAL_SPEC.expert_proj_names, offload_backend_impl=backend)
    gx = torch.Generator().manual_seed(7)
    x = torch.randn(T, H, generator=gx).to(torch.bfloat16)
    router = torch.randn(E, H, generator=gx) * 0.02
    logits = (x.float() @ router.T).to(torch.bfloat16)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    torch.cuda.synchronize()
    assert backend.submit_calls == 1 and backend.sync_calls == 1
    bf = lambda t: t.detach().to(torch.bfloat16).to(torch.float32).cpu()
    layer = Layer(MoEConfig("m", H, E, k, I, 0, True, True, "bf16", "bf16"), torch.zeros(E, H), [
        {"gate": bf(experts[str(e)].w1.weight), "up": bf(experts[str(e)].w3.weight),
         "down": bf(experts[str(e)].w2.weight)} for e in range(E)])
    err_abs, err_rel = compare(out.float().cpu().numpy(), oracle_forward(layer, x, logits), layer.cfg)
    announce(f"  max_abs={err_abs:.3e} rel_l2={err_rel:.3e}")
    served.check_status()
