"""The MoE layer on the GPU (K1..K5 through nkt_moe_forward) against the oracle.

Tolerances (moe_cases.compare): bf16 activations: every element within
max(2e-2, one bf16 ulp of the oracle value) and rel-L2 <= 1e-2; fp32 activations
with dense fp32 weights: rel-L2 <= 1e-4.  Routing,
counts and the permutation inside the forward are checked bit-exact."""
import sys

import numpy as np
import pytest
import torch

import oracle as O
from moe_cases import CONFIGS, build_inputs, build_layer, compare, native_layer, oracle_forward

pytestmark = pytest.mark.gpu


def announce(msg):
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


_LAYERS = {}


def _layer(name, E=None, I=None, device="cuda"):
    key = (name, E, I)
    if key not in _LAYERS:
        cfg = CONFIGS[name]
        if I is not None:
            from dataclasses import replace
            cfg = replace(cfg, I=I)
        _LAYERS.clear()  # keep at most one layer's weights alive
        layer = build_layer(cfg, device=device, num_experts=E)
        _LAYERS[key] = (layer, native_layer(layer, torch.device(device)))
    return _LAYERS[key]


def _check(layer, native, T, seed=7, bias=None):
    cfg = layer.cfg
    x, logits = build_inputs(layer, T, seed=seed, device="cuda")
    if bias is not None:  # skew the routing: bias [E] added to every token's logits
        logits = (logits.float() + bias.to(logits.device)).to(logits.dtype)
    out = native.forward(x, logits)
    torch.cuda.synchronize()
    ref, parts = oracle_forward(layer, x, logits, return_parts=True)
    # routing inside the forward is bit-exact
    ids = native.region(T, 0, torch.int32, (T, cfg.k)).cpu().numpy()
    assert np.array_equal(ids, parts["ids"])
    perm = native.region(T, 4, torch.int32, (T * cfg.k,)).cpu().numpy()
    assert np.array_equal(perm, parts["perm"])
    err_abs, err_rel = compare(out.float().cpu().numpy(), ref, cfg)
    announce(f"  {cfg.name} T={T}: max_abs={err_abs:.3e} rel_l2={err_rel:.3e}")
    return out


@pytest.mark.parametrize("T", [1, 16, 100])
def test_tiny_mixtral_fp32(gpu_device, T):
    announce(f"forward tiny_mixtral_fp32 T={T}")
    layer, native = _layer("tiny_mixtral_fp32")
    _check(layer, native, T)


@pytest.mark.parametrize("T", [1, 4, 16, 64, 300])
def test_qwen3_int4_cut_experts(gpu_device, T):
    announce(f"forward qwen3_int4 E=32 T={T}")
    layer, native = _layer("qwen3_int4", E=32)
    _check(layer, native, T)


@pytest.mark.parametrize("T", [17, 24, 32, 40, 64, 72])
def test_qwen3_int4_decode_form_multi_tile_experts(gpu_device, T):
    """Four experts picked by every token.  T = 17 .. 32: the decode form
    (T k <= 8 E for int4 weights): each hot expert holds T positions in
    ceil(T / 16) tiles, so the tile records past an expert's first tile and
    its tiles' source columns of rank >= 16 are used; T = 40 .. 72 are past
    that form (prefill tiles: a full one and a short one per hot expert
    from 64 on)."""
    announce(f"forward qwen3_int4 E=32 T={T} skewed")
    layer, native = _layer("qwen3_int4", E=32)
    assert layer.cfg.decode_form(T) == (T <= 32)
    bias = torch.zeros(32)
    bias[[3, 11, 20, 31]] = 30.0
    _check(layer, native, T, seed=9, bias=bias)


@pytest.mark.parametrize("max_tokens", [1, 48])
def test_empty_and_max_token_batches(gpu_device, max_tokens):
    """An empty batch returns an empty output without a launch; a batch of
    exactly max_tokens matches the oracle; one token more is rejected."""
    from nano_ktrans_amd import _native as N

    announce(f"empty / max_tokens={max_tokens} small_int8_shared")
    layer = build_layer(CONFIGS["small_int8_shared"], device="cuda")
    native = native_layer(layer, torch.device("cuda"), max_tokens=max_tokens)
    x, logits = build_inputs(layer, max_tokens + 1, seed=13, device="cuda")
    assert native.forward(x[:0], logits[:0]).shape == (0, layer.cfg.H)
    _check(layer, native, max_tokens, seed=13)
    with pytest.raises(N.NativeError, match="max_tokens"):
        native.forward(x, logits)


@pytest.mark.parametrize("T", [1, 2, 3, 4, 16])
def test_qwen3_int4_full(gpu_device, T):
    announce(f"forward qwen3_int4 full T={T}")
    layer, native = _layer("qwen3_int4")
    _check(layer, native, T)


@pytest.mark.parametrize("name,E,T", [("qwen3_int4", None, 300), ("qwen3_int4", 32, 90),
                                      ("qwen3_int8", 32, 40), ("qwen3_int8", 32, 100)])
def test_prefill_short_tile_copies(gpu_device, name, E, T):
    """Prefill tiles of at most 16 / 32 positions (an expert's last or only
    tile) run pipeline copies over their first 1 / 2 column tiles: int8
    always (the Zipf-skewed qwen3_int8 routing gives tiles of every size),
    int4 where the experts average at most 24 positions (T k <= 24 E: 18.75
    and 22.5 per expert here, tiles of 5 - 40 positions)."""
    announce(f"forward {name} E={E} T={T} (short prefill tiles)")
    layer, native = _layer(name, E=E)
    assert not layer.cfg.decode_form(T)
    _check(layer, native, T, seed=41)


@pytest.mark.parametrize("T", [16, 200, 512])
def test_qwen3_int8_cut_experts(gpu_device, T):
    announce(f"forward qwen3_int8 E=32 T={T}")
    layer, native = _layer("qwen3_int8", E=32)
    _check(layer, native, T)


def test_qwen3_int8_prefill_row_scales(gpu_device):
    """The int8 prefill gate_up multiplies power-of-two-scaled fp16 copies of
    the token rows: rows scaled by 2^-40 .. 2^40, a zero row and rows whose
    entries span 2^20 must each match the oracle to the bf16 tolerance of
    their own magnitude (routing from the unscaled rows); so must rows whose
    entries span 2^40 and 2^64."""
    announce("forward qwen3_int8 E=32 T=320 scaled rows")
    layer, native = _layer("qwen3_int8", E=32)
    T = 320
    x, logits = build_inputs(layer, T, seed=11, device="cuda")
    xf = x.float()
    exps = torch.tensor([-40, -20, 0, 20, 40], dtype=torch.float32, device="cuda")
    scale = torch.pow(2.0, exps[torch.arange(T, device="cuda") % 5])
    xf = xf * scale[:, None]
    xf[7] = 0.0
    xf[9, ::97] *= 2.0 ** 20  # one row spanning 2^20 (plus the N(0,1) spread)
    # rows spanning 2^40 and 2^64: entries below 2^-32 of the row's largest
    # fall out of the fp16 copy; their share of the output is below the
    # bf16 tolerance of the row's own magnitude
    xf[11, ::97] *= 2.0 ** 20
    xf[11, 1::97] *= 2.0 ** -20
    xf[13, ::53] *= 2.0 ** 32
    xf[13, 5::53] *= 2.0 ** -32
    xs = xf.to(torch.bfloat16)
    out = native.forward(xs, logits)
    torch.cuda.synchronize()
    ref = oracle_forward(layer, xs, logits)
    got = out.float().cpu().numpy().astype(np.float64)
    assert np.all(got[7] == 0.0)
    for t in range(T):
        if t == 7:
            continue
        r = ref[t].astype(np.float64)
        rel = np.linalg.norm(got[t] - r) / np.linalg.norm(r)
        assert rel <= 1e-2, f"row {t}: rel-L2 {rel}"
        assert np.max(np.abs(got[t] - r)) <= 2e-2 * np.max(np.abs(r)), f"row {t}: max-abs"


@pytest.mark.parametrize("T", [16, 100, 256])
def test_qwen3_shape_bf16_weights(gpu_device, T):
    """Dense bf16 experts at the Qwen3 shape (E cut to 16): T=16 decode form,
    T=100 the 64-position prefill form, T=256 the 128-position form."""
    announce(f"forward qwen3 shape bf16 weights E=16 T={T}")
    from dataclasses import replace
    cfg = replace(CONFIGS["qwen3_int4"], name="qwen3_bf16", wfmt="bf16")
    _LAYERS.clear()
    layer = build_layer(cfg, device="cuda", num_experts=16)
    _check(layer, native_layer(layer, torch.device("cuda")), T)


@pytest.mark.parametrize("T", [512, 2048, 4096])
def test_qwen3_int8_full_prefill(gpu_device, T):
    """The Qwen3-30B-A3B int8 prefill layer at its full shape (E = 128) and
    Zipf(1.1)-skewed routing, every row of every token count against the
    oracle: at T = 4096 that is all 32768 positions, the last tiles of every
    expert and the far end of the XCD work order included."""
    announce(f"forward qwen3_int8 full T={T}")
    layer, native = _layer("qwen3_int8")
    _check(layer, native, T)


def test_qwen3_int8_batch_invariance_at_4096(gpu_device):
    """Full-size property: a token's output does not depend on the other tokens in the batch.

    Within one kernel regime (tiled prefill GEMM at T=4096 and T=2048, decode GEMV at T=16
    and T=5) every output element accumulates over K in the same order whatever the tile, so
    the outputs are bit-identical; across regimes (T=4096 vs T=97) the K split differs, and
    both agree with the oracle within tolerance."""
    announce("forward qwen3_int8 full T=4096 batch invariance")
    layer, native = _layer("qwen3_int8")
    x, logits = build_inputs(layer, 4096, seed=21, device="cuda")
    full = native.forward(x, logits).clone()
    half = native.forward(x[:2048].contiguous(), logits[:2048].contiguous()).clone()
    small = native.forward(x[:16].contiguous(), logits[:16].contiguous()).clone()
    tiny = native.forward(x[:5].contiguous(), logits[:5].contiguous()).clone()
    part = native.forward(x[:97].contiguous(), logits[:97].contiguous()).clone()
    torch.cuda.synchronize()
    assert torch.equal(full[:2048], half)
    assert torch.equal(small[:5], tiny)
    ref = oracle_forward(layer, x[:97], logits[:97])
    compare(part.float().cpu().numpy(), ref, layer.cfg)
    compare(full[:97].float().cpu().numpy(), ref, layer.cfg)


@pytest.mark.parametrize("T", [1, 16, 24, 28])
def test_mixtral_int4_full(gpu_device, T):
    """T = 24: 6 positions per expert, the decode form's last count for
    experts of I >= 8192; T = 28 the prefill form's short-tile instance
    (tiles of about 7 positions: the one-column-tile copies)."""
    announce(f"forward mixtral_int4 full T={T}")
    layer, native = _layer("mixtral_int4")
    assert layer.cfg.decode_form(T) == (T <= 24)
    _check(layer, native, T)


def test_mixtral_int4_cut_intermediate_prefill(gpu_device):
    announce("forward mixtral_int4 I=1024 T=300")
    layer, native = _layer("mixtral_int4", I=1024)
    _check(layer, native, 300)


@pytest.mark.parametrize("T", [20, 40, 64, 600])
def test_small_int8_short_k(gpu_device, T):
    """T = 20 / 40 / 64: the prefill form at a token count the one-launch
    routing would take; with a shared expert the routing launch that makes
    the fp16 input copy runs instead, and the shared expert forks beside
    the routed experts."""
    announce(f"forward small_int8_shared T={T}")
    layer, native = _layer("small_int8_shared")
    _check(layer, native, T)


@pytest.mark.parametrize("wfmt,T", [("int4_g128", 1), ("int4_g128", 2), ("int4_g128", 3), ("int4_g128", 16),
                                    ("bf16", 1), ("bf16", 16)])
def test_shared_chunks_int4_and_bf16(gpu_device, wfmt, T):
    """The shared expert as chunks of the routed launches for every weight
    format: Qwen1.5-MoE's shape (E = 60, k = 4, I = 1408, shared 5632 = 4 x
    1408) with int4 g128 and bf16 weights.  One token: the chunks ride in the
    routing gate_up and the down + combine launch; int4 at T = 2 and 3
    (4 T k <= E): the few-token down + combine launch with chunk items (the
    int4 chunk scale addressing of gate_up and down); T = 16: chunk tiles of
    the routed decode launches.  Against the oracle, and the chunk gate and h
    against the shared stage's bit for bit."""
    from dataclasses import replace

    from nano_ktrans_amd import _native as N
    announce(f"shared chunks qwen15 shape {wfmt} T={T}")
    key = ("qwen15_" + wfmt, None, None)
    if key not in _LAYERS:
        cfg = replace(CONFIGS["qwen15_int8_shared"], name="qwen15_" + wfmt, wfmt=wfmt)
        _LAYERS.clear()
        layer = build_layer(cfg, device="cuda")
        _LAYERS[key] = (layer, native_layer(layer, torch.device("cuda")))
    layer, native = _LAYERS[key]
    assert layer.cfg.shared_in_routed_launches(T)
    out = _check(layer, native, T, seed=73).clone()
    Is = layer.cfg.Is
    gate_layer = native.region(T, N.WS_SHARED_GATE, torch.float32, (T,)).clone()
    h_layer = native.region(T, N.WS_SHARED_H, torch.bfloat16, (T, Is)).clone()
    x, _ = build_inputs(layer, T, seed=73, device="cuda")
    gate_stage, _ = native.shared(x)
    h_stage = native.region(T, N.WS_SHARED_H, torch.bfloat16, (T, Is))
    torch.cuda.synchronize()
    assert torch.equal(gate_layer, gate_stage)
    assert torch.equal(h_layer, h_stage)


@pytest.mark.parametrize("T", [1, 16, 48, 52, 53, 200])
def test_qwen15_shared_full(gpu_device, T):
    """T = 48 / 52: 3.2 / 3.47 positions per expert, the int8 decode form's
    last token counts in a layer with a shared expert (which rides as 4
    chunk tiles per chunk in the routed launches); T = 53 the first in the
    prefill form, the shared expert forked beside the routed experts."""
    announce(f"forward qwen15_int8_shared full T={T}")
    layer, native = _layer("qwen15_int8_shared")
    assert layer.cfg.decode_form(T) == (T <= 52)
    _check(layer, native, T)


@pytest.mark.parametrize("name,T", [("qwen15_int8_shared", 1), ("qwen15_int8_shared", 5),
                                    ("qwen15_int8_shared", 16), ("qwen15_int8_shared", 52),
                                    ("small_int8_shared", 1), ("small_int8_shared", 12)])
def test_shared_expert_in_routed_launches(gpu_device, name, T):
    """A decode-form batch and a shared expert whose intermediate size is a
    multiple of the routed one's (Qwen1.5-MoE: 4 chunks of 1408, the small
    case: 1 chunk): the shared expert runs as Is / I chunks inside the routed
    gate_up and down launches (one token: the routing gate_up and the down +
    combine launch).  The gate and h they leave equal the shared stage's (K4,
    then the shared expert's gate_up) bit for bit, and the output matches the
    oracle."""
    from nano_ktrans_amd import _native as N

    layer, native = _layer(name)
    assert layer.cfg.shared_in_routed_launches(T)
    Is = layer.cfg.Is
    for seed in (71, 72):
        announce(f"shared chunks in the routed launches {name} T={T} seed={seed}")
        x, logits = build_inputs(layer, T, seed=seed, device="cuda")
        out = native.forward(x, logits).clone()
        torch.cuda.synchronize()
        gate_layer = native.region(T, N.WS_SHARED_GATE, torch.float32, (T,)).clone()
        h_layer = native.region(T, N.WS_SHARED_H, torch.bfloat16, (T, Is)).clone()
        gate_stage, _ = native.shared(x)
        h_stage = native.region(T, N.WS_SHARED_H, torch.bfloat16, (T, Is))
        torch.cuda.synchronize()
        assert torch.equal(gate_layer, gate_stage)
        assert torch.equal(h_layer, h_stage)
        compare(out.float().cpu().numpy(), oracle_forward(layer, x, logits), layer.cfg)


def test_forward_deterministic(gpu_device):
    announce("forward determinism qwen3_int4 E=32 T=64")
    layer, native = _layer("qwen3_int4", E=32)
    x, logits = build_inputs(layer, 64, seed=3, device="cuda")
    a = native.forward(x, logits).clone()
    for _ in range(3):
        b = native.forward(x, logits)
        assert torch.equal(a, b)


def test_stages_match_forward(gpu_device):
    """route -> experts -> shared -> combine through the separate entry points
    equals forward, up to the order of the shared expert's down sums (the
    layer adds its Is / I chunks one by one): within 2^-12 of the largest
    |y_shared| plus one bf16 step."""
    announce("stages vs forward qwen15_int8_shared T=16")
    layer, native = _layer("qwen15_int8_shared")
    x, logits = build_inputs(layer, 16, seed=9, device="cuda")
    a = native.forward(x, logits).clone()
    native.route(logits)
    h, y = native.experts(x)
    gate, ysh = native.shared(x)
    b = native.combine(16)
    torch.cuda.synchronize()
    bound = 2.0 ** -12 * ysh.abs().max().item() + 2.0 ** -7 * torch.maximum(a.float().abs(), b.float().abs())
    assert bool(((a.float() - b.float()).abs() <= bound).all())
    # K4 alone: sigmoid(x . g)
    ref_gate = torch.sigmoid(x.float().cpu() @ layer.shared_gate.cpu())
    assert torch.allclose(gate.cpu(), ref_gate, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name,E,T", [("qwen15_int8_shared", None, 16), ("qwen15_int8_shared", None, 1),
                                      ("qwen3_int4", 32, 16), ("qwen3_int8", 32, 512), ("mixtral_int4", None, 300),
                                      ("qwen3_int4", None, 8), ("mixtral_int4", None, 16),
                                      ("qwen15_int8_shared", None, 1024), ("qwen15_int8_shared", None, 512),
                                      # 17 .. 64 tokens: the several-workgroup route + group launch
                                      ("qwen3_int4", None, 48), ("qwen15_int8_shared", None, 33),
                                      # 2 .. 4 tokens: the self-routing gate_up
                                      ("qwen3_int4", None, 3)])
def test_graph_replay_matches_eager(gpu_device, name, E, T):
    """The layer captured in a HIP graph (Qwen1.5-MoE at 1024 tokens: the
    prefill-form shared expert as a branch forked onto the handle's side
    stream after the routing launch) replays bit for bit like the eager call,
    replay after replay, with eager calls on the same workspace in between."""
    announce(f"graph replay {name} T={T}")
    layer, native = _layer(name, E=E)
    x, logits = build_inputs(layer, T, seed=21, device="cuda")
    eager = native.forward(x, logits).clone()
    out = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        native.forward(x, logits, out=out)  # warm the workspace outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        native.forward(x, logits, out=out)
    for _ in range(4):
        out.zero_()
        x2, l2 = build_inputs(layer, T, seed=22, device="cuda")
        native.forward(x2, l2)  # other eager work on the same workspace
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("name,T", [("qwen3_int4", 16), ("qwen3_int8", 512)])
def test_timed_phases_match_untimed(gpu_device, name, T):
    """The measurement entry point runs the same kernels: bitwise-equal h and y, and
    its dispatch-stamped events give a positive duration."""
    announce(f"timed phases {name} T={T}")
    layer, native = _layer(name, E=32)
    x, logits = build_inputs(layer, T, seed=11, device="cuda")
    native.route(logits)
    h0, y0 = (t.clone() for t in native.experts(x))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in ev:
        e.record()
    native.expert_phase_timed(0, x, T, ev[0], ev[1])
    native.expert_phase_timed(1, None, T, ev[2], ev[3])
    torch.cuda.synchronize()
    P = T * layer.cfg.k
    from nano_ktrans_amd import _native as N
    h1 = native.region(T, N.WS_H, torch.bfloat16, (P, layer.cfg.I))
    y1 = native.region(T, N.WS_Y, torch.float32, (P, layer.cfg.H))
    assert torch.equal(h0, h1)
    assert torch.equal(y0, y1)
    assert ev[0].elapsed_time(ev[1]) > 0 and ev[2].elapsed_time(ev[3]) > 0


@pytest.mark.parametrize("name,E,T", [("qwen3_int4", 32, 16), ("qwen3_int8", 32, 512), ("mixtral_int4", None, 1),
                                      ("qwen15_int8_shared", None, 16), ("qwen3_int4", None, 4),
                                      # router GEMV launch, then one token routed inside gate_up / the
                                      # self-routing gate_up; 17 .. 64 tokens: the single-launch router
                                      ("qwen3_int4", None, 1), ("qwen3_int4", None, 2), ("qwen3_int4", None, 40)])
def test_forward_hidden_fused_router(gpu_device, name, E, T):
    """The layer from hidden states alone (router GEMV fused): logits checked
    against the oracle's (check_router_logits), the output equal to the
    oracle's forward on the GPU's logits within the bf16 tolerance, and to
    nkt_moe_forward on them bit for bit; the sync area is left zero."""
    from nano_ktrans_amd import _native as N
    from moe_cases import check_router_logits
    announce(f"forward_hidden {name} E={E} T={T}")
    layer, native = _layer(name, E=E)
    gate = layer.router.to(torch.bfloat16)
    native.load_router(gate)
    x, _ = build_inputs(layer, T, seed=21, device="cuda")
    out = native.forward_hidden(x).clone()
    torch.cuda.synchronize()
    g_logits = native.region(T, N.WS_ROUTER_LOGITS, torch.bfloat16, (T, layer.cfg.E)).clone()
    check_router_logits(g_logits.float().cpu().numpy(), x.float().cpu().numpy(), gate.float().cpu().numpy())
    ref = oracle_forward(layer, x, g_logits)
    err_abs, err_rel = compare(out.float().cpu().numpy(), ref, layer.cfg)
    announce(f"  {name} T={T}: max_abs={err_abs:.3e} rel_l2={err_rel:.3e}")
    again = native.forward(x, g_logits)
    torch.cuda.synchronize()
    assert torch.equal(out, again)
    assert not native.workspace(T)[:N.SYNC_AREA_BYTES].any()
    native.check_status()


def _spread_rows(T, ids, n_edge=32, n_hot=16):
    """Rows to check against the oracle in a large batch: the first, middle and
    last n_edge (+1) rows -- they hold the first, middle and last positions of
    every expert, so the first, middle and last 64-position tiles -- plus up to
    n_hot rows routed to the most-used expert, spread over its segment."""
    mid = T // 2 - n_edge // 2
    rows = set(range(n_edge)) | set(range(mid, mid + n_edge)) | set(range(T - n_edge - 1, T))
    hot = np.bincount(ids.ravel()).argmax()
    hot_rows = np.nonzero((ids == hot).any(axis=1))[0]
    rows |= set(hot_rows[np.linspace(0, len(hot_rows) - 1, n_hot).astype(int)].tolist())
    return sorted(rows)


def _check_rows_and_prefix(layer, native, T, prefix, seed):
    """The full batch's routing and permutation bit-exact; >= 97 spread rows
    against the oracle; rows [0, prefix) bit-identical to a batch of prefix
    tokens (the same prefill regime: every output element sums over K in the
    same order whatever the tile)."""
    cfg = layer.cfg
    x, logits = build_inputs(layer, T, seed=seed, device="cuda")
    out = native.forward(x, logits).clone()
    torch.cuda.synchronize()
    ids = native.region(T, 0, torch.int32, (T, cfg.k)).cpu().numpy()
    perm = native.region(T, 4, torch.int32, (T * cfg.k,)).cpu().numpy()
    o_ids, _ = O.route(logits.float().cpu().numpy(), cfg.k, cfg.softmax, cfg.renorm, cfg.act == "bf16")
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(perm, O.group(o_ids, cfg.E)[2])
    rows = _spread_rows(T, ids)
    assert len(rows) >= 97
    idx = torch.tensor(rows, device="cuda")
    ref = oracle_forward(layer, x[idx], logits[idx])
    err_abs, err_rel = compare(out[idx].float().cpu().numpy(), ref, cfg)
    announce(f"  {cfg.name} T={T} ({len(rows)} rows): max_abs={err_abs:.3e} rel_l2={err_rel:.3e}")
    part = native.forward(x[:prefix].contiguous(), logits[:prefix].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(out[:prefix], part)


def test_mixtral_int4_full_prefill(gpu_device):
    """Mixtral-8x7B int4 at its full shape (I=14336) and T=2048: the int4
    prefill pipeline with down over K=14336 (112 stages) and experts of
    58.7 MB (gate_up) / 29.4 MB (down) that run in groups of 4 weight slabs."""
    announce("forward mixtral_int4 full T=2048 (rows) and T=1024 (prefix)")
    layer, native = _layer("mixtral_int4")
    _check_rows_and_prefix(layer, native, 2048, 1024, seed=31)


@pytest.mark.parametrize("T,prefix", [(1024, 896), (512, 320)])
def test_qwen15_shared_full_prefill(gpu_device, T, prefix):
    """Qwen1.5-MoE in the prefill form: the routed experts and the 23 MB
    shared gate_up (11264 x 2048 int8), the shared expert's weight slabs in
    groups of 4.  T=1024 (and its prefix 896): the shared down sums all of
    K = 5632 in one pass; T=512 (and 320): in 4 K parts of 1408 whose rows
    the combine adds in order -- each prefix in its batch's regime, so its
    rows are bit-identical."""
    announce(f"forward qwen15_int8_shared full T={T} (rows) and T={prefix} (prefix)")
    layer, native = _layer("qwen15_int8_shared")
    _check_rows_and_prefix(layer, native, T, prefix, seed=33)


@pytest.mark.parametrize("T", [1, 16])
@pytest.mark.parametrize("name,E", [("qwen3_int4", None), ("qwen15_int8_shared", None)])
def test_decode_outlier_channels(gpu_device, name, E, T):
    """The decode form feeds codes to the matrix cores as offset integers and
    removes offset x (group sum of x) afterwards; four activation channels
    scaled by 256 (the outlier channels of real activations) make those group
    sums large.  Routing from the unscaled rows."""
    announce(f"forward {name} T={T} outlier channels")
    layer, native = _layer(name, E=E)
    x, logits = build_inputs(layer, T, seed=41, device="cuda")
    xf = x.float()
    xf[:, [5, 700, 1500, 2047]] *= 256.0
    xs = xf.to(torch.bfloat16)
    out = native.forward(xs, logits)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    # (1) the fp32 oracle, at the bf16 tolerance scaled to each row's size: the
    # outputs grow with the inputs, and h is stored in bf16 on both the GPU and
    # the reference's bf16 path (an error of 2^-9 |h| per element that an
    # absolute bound does not scale with)
    ref = oracle_forward(layer, xs, logits)
    for t in range(T):
        r = ref[t].astype(np.float64)
        assert np.linalg.norm(got[t] - r) <= 1e-2 * np.linalg.norm(r), f"row {t}: rel-L2"
        assert np.max(np.abs(got[t] - r)) <= 2e-2 * np.max(np.abs(r)), f"row {t}: max-abs"
    # (2) the oracle with h rounded to bf16 like the GPU, at the absolute bf16
    # tolerance: what is left is the accumulation of the offset codes
    ref_h = oracle_forward(layer, xs, logits, h_bf16=True)
    err_abs, err_rel = compare(got, ref_h, layer.cfg)
    announce(f"  {name} T={T} outliers: max_abs={err_abs:.3e} rel_l2={err_rel:.3e} "
             f"max|ref|={np.abs(ref).max():.2f}")


@pytest.mark.parametrize("name,E,T", [("qwen3_int4", 32, 16), ("mixtral_int4", None, 1), ("qwen3_int4", 32, 64),
                                      ("qwen3_int4", None, 1), ("qwen15_int8_shared", None, 1),
                                      ("qwen3_int4", None, 16), ("qwen3_int4", None, 4), ("mixtral_int4", None, 16),
                                      ("qwen3_int8", 32, 16), ("qwen3_int8", 32, 512), ("qwen15_int8_shared", None, 1024),
                                      ("qwen15_int8_shared", None, 512),
                                      # 2 .. 16 tokens: the routing launch, then the decode launches
                                      # (2 Qwen3 int4 tokens: the self-routing gate_up, no routing
                                      # launch, then the down + combine launch)
                                      ("qwen3_int4", None, 2), ("qwen3_int4", None, 8), ("qwen3_int4", 32, 13),
                                      ("qwen15_int8_shared", None, 5), ("mixtral_int4", None, 3),
                                      ("qwen3_int8", 32, 7), ("small_int8_shared", None, 1)])
def test_forward_matches_stages_and_leaves_sync_area_zero(gpu_device, name, E, T):
    """The layer equals route -> experts -> shared -> combine through the
    separate entry points bit for bit (at T = 1, and at T = 2 / 4 for the
    int4 Qwen3 shape, the layer runs the down GEMV and the combine as one
    launch) in the decode form; in the prefill form
    the layer keeps y as fp16 with a power-of-two scale per position and
    256-column slab (the stages keep fp32 y), and the layer runs the shared
    expert's down in parts whose sums are added part by part (the decode
    form: Is / I chunks; the prefill form with up to 96 (token tile, weight
    slab) items, Qwen1.5-MoE at T = 512: 4 K parts) where the stage sums all
    of K at once, so there every output element is within 2^-11 of the
    largest |y| plus one bf16 step of the stages'.
    The layer leaves the workspace's sync area (the NKT_SYNC_AREA_BYTES
    before NKT_WS_TOPK_IDS) all zero."""
    import ctypes

    from nano_ktrans_amd import _native as N
    announce(f"forward vs stages {name} E={E} T={T}")
    layer, native = _layer(name, E=E)
    x, logits = build_inputs(layer, T, seed=61, device="cuda")
    a = native.forward(x, logits).clone()
    torch.cuda.synchronize()
    off = ctypes.c_size_t(0)
    native.err.check(native.lib.nkt_moe_workspace_region(native.handle, T, N.WS_TOPK_IDS, ctypes.byref(off),
                                                         native.err.buf, native.err.size), "region")
    assert off.value == N.SYNC_AREA_BYTES and not native.workspace(T)[: off.value].any()
    k, E = layer.cfg.k, layer.cfg.E
    regions = [(N.WS_TOPK_IDS, torch.int32, (T, k)), (N.WS_TOPK_WEIGHTS, torch.float32, (T, k)),
               (N.WS_COUNTS, torch.int32, (E,)), (N.WS_OFFSETS, torch.int32, (E + 1,)),
               (N.WS_PERM, torch.int32, (T * k,)), (N.WS_INV, torch.int32, (T * k,))]
    # the routing outputs the layer left (at T = 1 written by its gate_up launch)
    routed = [native.region(T, r, dt, shp).clone() for r, dt, shp in regions]
    for got, want in zip(routed, native.route(logits)):
        assert torch.equal(got, want)
    _, y = native.experts(x)
    ymax = y.abs().max().item()
    if layer.cfg.Is:
        _, ysh = native.shared(x)
        ymax = max(ymax, ysh.abs().max().item())
    b = native.combine(T)
    torch.cuda.synchronize()
    if layer.cfg.decode_form(T) and not layer.cfg.shared_in_routed_launches(T):
        assert torch.equal(a, b)
    else:
        # a compact row is within half an fp16 step of its value, 2^-11 of its
        # slab's largest |y| at most (that largest scaled into [2^14, 2^15)),
        # and the routing weights of a token sum to at most 1: the sums differ
        # by at most 2^-11 ymax (the chunk sums' reassociation is far below);
        # each is then rounded to bf16 (one step is at most 2^-7 of the value)
        bound = 2.0 ** -11 * ymax + 2.0 ** -7 * torch.maximum(a.float().abs(), b.float().abs())
        diff = (a.float() - b.float()).abs()
        announce(f"  compact y: max diff {diff.max().item():.3e}, largest |y| {ymax:.3e}")
        assert bool((diff <= bound).all())
