"""The decode gate_up launch that routes its own tokens (2 .. 4 tokens from
given bf16 logits, int4 weights, Qwen3's 128 experts: every gate_up
workgroup selects the tokens' experts itself, one workgroup writes K1's and
K2's outputs); the int8 layer of the same shape, which keeps the routing
launch, through the same checks.

Checked per case: the routing outputs the layer leaves (ids, weights,
counts, offsets, perm, inv) bit-exact against the oracle's route + group
(nano_ktrans/layers/hybrid_moe.py:3321-3329, 3512-3526); the output bit for
bit against the stage entry points, whose routing is a launch of its own; and
the output against the oracle's expert loop (moe_cases.compare tolerances).
Cases: plain logits, logits snapped to a coarse grid (many equal
probabilities, so the lower-id tie rule decides, one token with every logit
equal), and half of the experts marked non-resident (their pairs keep their
positions but get no GPU compute and add nothing)."""
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


def _layer(name):
    if name not in _LAYERS:
        _LAYERS.clear()
        layer = build_layer(CONFIGS[name], device="cuda")
        _LAYERS[name] = (layer, native_layer(layer, torch.device("cuda")))
    return _LAYERS[name]


def _oracle_given(layer, x, ids, w):
    experts = [O.Expert(_to_oracle(e["gate"]), _to_oracle(e["up"]), _to_oracle(e["down"])) for e in layer.experts]
    return O.moe_forward_given(x.float().cpu().numpy(), ids, w, experts)


@pytest.mark.parametrize("name", ["qwen3_int4", "qwen3_int8"])
@pytest.mark.parametrize("T", [2, 3, 4])
@pytest.mark.parametrize("case", ["plain", "ties", "residency"])
def test_self_routing_gate_up(gpu_device, name, T, case):
    from nano_ktrans_amd import _native as N

    announce(f"self-routing gate_up {name} T={T} {case}")
    layer, native = _layer(name)
    cfg = layer.cfg
    E, k = cfg.E, cfg.k
    x, logits = build_inputs(layer, T, seed=300 + T, device="cuda")
    if case == "ties":
        logits = (torch.round(logits.float() * 2.0) / 2.0).to(logits.dtype)
        logits[0] = 0.25  # every probability equal: the k lowest ids
    resident = None
    if case == "residency":
        g = torch.Generator().manual_seed(7 + T)
        resident = torch.rand(E, generator=g) < 0.5
        native.set_residency(resident)
    try:
        out = native.forward(x, logits).clone()
        torch.cuda.synchronize()
        oids, ow = O.route(logits.float().cpu().numpy(), k, cfg.softmax, cfg.renorm, True)
        ocounts, ooffsets, operm, oinv = O.group(oids, E)
        regions = [(N.WS_TOPK_IDS, torch.int32, (T, k), oids), (N.WS_TOPK_WEIGHTS, torch.float32, (T, k), ow),
                   (N.WS_COUNTS, torch.int32, (E,), ocounts), (N.WS_OFFSETS, torch.int32, (E + 1,), ooffsets),
                   (N.WS_PERM, torch.int32, (T * k,), operm), (N.WS_INV, torch.int32, (T * k,), oinv)]
        for r, dt, shp, want in regions:
            got = native.region(T, r, dt, shp).cpu().numpy()
            if dt == torch.float32:
                assert np.array_equal(got.view(np.uint32), np.asarray(want, np.float32).view(np.uint32)), r
            else:
                assert np.array_equal(got, want), r
        if case == "ties":
            assert np.array_equal(np.sort(oids[0]), np.arange(k))
        # the stage entry points: a routing launch of its own, then the experts and the combine
        native.route(logits)
        native.experts(x)
        b = native.combine(T)
        torch.cuda.synchronize()
        assert torch.equal(out, b)
        w_eff = ow.copy()
        if resident is not None:
            w_eff = np.where(resident.numpy()[oids], ow, np.float32(0.0)).astype(np.float32)
        ref = _oracle_given(layer, x, oids, w_eff)
        err_abs, err_rel = compare(out.float().cpu().numpy(), ref, cfg)
        announce(f"  max_abs={err_abs:.3e} rel_l2={err_rel:.3e}")
    finally:
        if resident is not None:
            native.set_residency(None)


# (E, k, T, renorm, half the experts non-resident): E in (64, 128] and not
# always a multiple of 64, k from 1 to 16, both sides of 4 T k <= E
_SHAPES = [(72, 6, 4, True, False), (128, 16, 2, True, True), (127, 2, 4, False, False), (65, 8, 3, True, True),
           (100, 1, 4, False, False), (96, 4, 4, True, True), (128, 16, 4, False, False)]


@pytest.mark.parametrize("case", range(len(_SHAPES)))
def test_self_routing_other_shapes(gpu_device, case):
    """The self-routing gate_up over other shapes it takes (_SHAPES, I = 256,
    the Qwen3 hidden size): routing outputs bit-exact against the oracle, the
    output bit for bit against the stage entry points and within the bf16
    tolerance of the oracle."""
    from dataclasses import replace

    from nano_ktrans_amd import _native as N

    E, k, T, renorm, partial = _SHAPES[case]
    cfg = replace(CONFIGS["qwen3_int4"], name=f"sr_shape{case}", E=E, k=k, I=256, renorm=renorm, seed=20 + case)
    announce(f"self-routing shape {case}: E={E} k={k} T={T} renorm={renorm} partial residency={partial}")
    _LAYERS.clear()
    layer = build_layer(cfg, device="cuda")
    native = native_layer(layer, torch.device("cuda"))
    x, logits = build_inputs(layer, T, seed=400 + case, device="cuda")
    resident = None
    if partial:
        resident = torch.from_numpy(np.random.default_rng(1000 + case).random(E) < 0.5)
        native.set_residency(resident)
    out = native.forward(x, logits).clone()
    torch.cuda.synchronize()
    oids, ow = O.route(logits.float().cpu().numpy(), k, cfg.softmax, cfg.renorm, True)
    ocounts, ooffsets, operm, oinv = O.group(oids, E)
    for r, dt, shp, want in [(N.WS_TOPK_IDS, torch.int32, (T, k), oids), (N.WS_COUNTS, torch.int32, (E,), ocounts),
                             (N.WS_OFFSETS, torch.int32, (E + 1,), ooffsets), (N.WS_PERM, torch.int32, (T * k,), operm),
                             (N.WS_INV, torch.int32, (T * k,), oinv)]:
        assert np.array_equal(native.region(T, r, dt, shp).cpu().numpy(), want), r
    got_w = native.region(T, N.WS_TOPK_WEIGHTS, torch.float32, (T, k)).cpu().numpy()
    assert np.array_equal(got_w.view(np.uint32), np.asarray(ow, np.float32).view(np.uint32))
    native.route(logits)
    native.experts(x)
    b = native.combine(T)
    torch.cuda.synchronize()
    assert torch.equal(out, b)
    w_eff = ow if resident is None else np.where(resident.numpy()[oids], ow, np.float32(0.0)).astype(np.float32)
    err_abs, err_rel = compare(out.float().cpu().numpy(), _oracle_given(layer, x, oids, w_eff), cfg)
    announce(f"  max_abs={err_abs:.3e} rel_l2={err_rel:.3e}")
