"""HybridMoE as a drop-in: the reference's constructor and forward(hidden_states,
router_logits), expert weights from gpu_experts modules (Mixtral w1/w2/w3, Qwen3
packed gate_up) or from safetensors checkpoints (dense and GPTQ), optional shared
expert.  Compared with the oracle at the bf16 tolerance of moe_cases.compare."""
import json
import sys
from dataclasses import replace

import numpy as np
import pytest
import torch
from torch import nn

import oracle as O
from moe_cases import Layer, MoEConfig, compare, oracle_forward
from nano_ktrans_amd.kernels.quantized_ops import (quantize_symmetric_int8_per_channel,
                                                   quantize_symmetric_w4a32, to_bf16_scales)
from nano_ktrans_amd.layers.expert_mlp import PackedSparseExpertMLP, SparseExpertMLP
from nano_ktrans_amd.layers.hybrid_moe import HybridMoE
from nano_ktrans_amd.models.config import MIXTRAL_SPEC, QWEN3_MOE_SPEC, QWEN3_MOE_UNPACKED_SPEC

pytestmark = pytest.mark.gpu


def announce(msg):
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _init(module, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in module.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    return module


def _check(out, ref):
    err_abs, err_rel = compare(out.float().cpu().numpy(), ref, MoEConfig("bf16", 1, 1, 1, 1))
    announce(f"  max_abs={err_abs:.3e} rel_l2={err_rel:.3e}")


def _inputs(T, H, E, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    router = torch.randn(E, H, generator=g) * 0.02
    logits = (x.float() @ router.T).to(torch.bfloat16)
    return x, logits


def _bf16(t):
    return t.detach().to(torch.bfloat16).to(torch.float32).cpu()


def test_mixtral_modules_dense_bf16(gpu_device):
    announce("HybridMoE mixtral modules dense bf16")
    E, k, H, I, T = 8, 2, 256, 512, 16
    experts = nn.ModuleDict({str(e): _init(SparseExpertMLP(H, I), e).to(gpu_device, torch.bfloat16)
                             for e in range(E)})
    moe = HybridMoE(E, k, H, I, experts, torch.ones(E, dtype=torch.bool), 0, "",
                    router_use_softmax=MIXTRAL_SPEC.router_use_softmax,
                    normalize_topk_prob=MIXTRAL_SPEC.normalize_topk_prob,
                    expert_key_template=MIXTRAL_SPEC.expert_key_template,
                    expert_proj_names=MIXTRAL_SPEC.expert_proj_names)
    x, logits = _inputs(T, H, E)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    assert out.shape == (T, H) and out.dtype == torch.bfloat16
    cfg = MoEConfig("m", H, E, k, I, 0, False, True, "bf16", "bf16")
    layer = Layer(cfg, torch.zeros(E, H), [
        {"gate": _bf16(experts[str(e)].w1.weight), "up": _bf16(experts[str(e)].w3.weight),
         "down": _bf16(experts[str(e)].w2.weight)} for e in range(E)])
    _check(out, oracle_forward(layer, x, logits))
    # the routing API returns the reference's (weights in logits dtype, int64 ids)
    w, ids = moe.route(logits.to(gpu_device))
    oids, ow = O.route(logits.float().numpy(), k, False, True, True)
    assert ids.dtype == torch.int64 and np.array_equal(ids.cpu().numpy(), oids)
    assert w.dtype == torch.bfloat16 and np.array_equal(w.float().cpu().numpy(), ow)


def test_qwen3_packed_modules_quantized_int4(gpu_device):
    announce("HybridMoE qwen3 packed modules int4 at ingest")
    E, k, H, I, T = 16, 8, 2048, 768, 12
    experts = nn.ModuleDict({str(e): _init(PackedSparseExpertMLP(H, I), 100 + e).to(gpu_device, torch.bfloat16)
                             for e in range(E)})
    moe = HybridMoE(E, k, H, I, experts, torch.ones(E, dtype=torch.bool), 0, "",
                    router_use_softmax=True, normalize_topk_prob=True, experts_are_packed=True,
                    expert_key_template=QWEN3_MOE_SPEC.expert_key_template,
                    expert_proj_names=QWEN3_MOE_SPEC.expert_proj_names, quantization="int4_g128")
    x, logits = _inputs(T, H, E, seed=1)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    q = lambda w: to_bf16_scales(quantize_symmetric_w4a32(w.detach().float(), group_size=128))
    layer = Layer(MoEConfig("q", H, E, k, I), torch.zeros(E, H), [
        {"gate": q(experts[str(e)].gate_up_proj[:I]), "up": q(experts[str(e)].gate_up_proj[I:]),
         "down": q(experts[str(e)].down_proj.weight)} for e in range(E)])
    _check(out, oracle_forward(layer, x, logits))


def test_qwen3_fused_router_gate_module(gpu_device):
    """HybridMoE(gate=nn.Linear): forward(x) without router_logits runs the router
    GEMV inside the path and equals forward(x, gate(x)) computed by the library's
    own logits; the logits match the oracle's gate(x)."""
    from moe_cases import check_router_logits
    from nano_ktrans_amd import _native as N
    announce("HybridMoE qwen3 fused router gate module")
    E, k, H, I, T = 16, 8, 2048, 768, 12
    experts = nn.ModuleDict({str(e): _init(PackedSparseExpertMLP(H, I), 300 + e).to(gpu_device, torch.bfloat16)
                             for e in range(E)})
    gate = nn.Linear(H, E, bias=False)
    with torch.no_grad():
        gate.weight.copy_(torch.randn(E, H, generator=torch.Generator().manual_seed(9)) * 0.02)
    gate = gate.to(gpu_device, torch.bfloat16)
    moe = HybridMoE(E, k, H, I, experts, torch.ones(E, dtype=torch.bool), 0, "",
                    router_use_softmax=True, normalize_topk_prob=True, experts_are_packed=True,
                    expert_key_template=QWEN3_MOE_SPEC.expert_key_template,
                    expert_proj_names=QWEN3_MOE_SPEC.expert_proj_names, quantization="int4_g128", gate=gate)
    x, _ = _inputs(T, H, E, seed=3)
    x = x.to(gpu_device)
    out = moe(x).clone()
    torch.cuda.synchronize()
    logits = moe._native.region(T, N.WS_ROUTER_LOGITS, torch.bfloat16, (T, E)).clone()
    check_router_logits(logits.float().cpu().numpy(), x.float().cpu().numpy(),
                        gate.weight.detach().float().cpu().numpy())
    assert torch.equal(out, moe(x, logits))
    with pytest.raises(ValueError, match="router_logits is required"):
        HybridMoE(E, k, H, I, experts, torch.ones(E, dtype=torch.bool), 0, "", router_use_softmax=True,
                  experts_are_packed=True, expert_key_template=QWEN3_MOE_SPEC.expert_key_template,
                  expert_proj_names=QWEN3_MOE_SPEC.expert_proj_names, quantization="int4_g128")(x)


def test_safetensors_dense_and_gptq_checkpoints(gpu_device, tmp_path):
    from safetensors.torch import save_file

    announce("HybridMoE from safetensors: dense mixtral + gptq int4 qwen3")
    E, k, H, I, T = 8, 2, 256, 256, 9
    g = torch.Generator().manual_seed(3)
    dense = {}
    weights = []
    for e in range(E):
        w = {p: (torch.randn(s, generator=g) * 0.02).to(torch.bfloat16)
             for p, s in (("w1", (I, H)), ("w3", (I, H)), ("w2", (H, I)))}
        weights.append(w)
        for p, t in w.items():
            dense[f"model.layers.0.block_sparse_moe.experts.{e}.{p}.weight"] = t
    d1 = tmp_path / "dense"
    d1.mkdir()
    save_file(dense, str(d1 / "model.safetensors"))
    mask = torch.zeros(E, dtype=torch.bool)  # nothing in gpu_experts: every expert comes from disk
    moe = HybridMoE(E, k, H, I, nn.ModuleDict(), mask, 0, str(d1), router_use_softmax=False)
    x, logits = _inputs(T, H, E, seed=2)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    layer = Layer(MoEConfig("d", H, E, k, I, 0, False, True, "bf16", "bf16"), torch.zeros(E, H), [
        {"gate": w["w1"].float(), "up": w["w3"].float(), "down": w["w2"].float()} for w in weights])
    _check(out, oracle_forward(layer, x, logits))

    # GPTQ int4 checkpoint in the on-disk layout: qweight [in/8, out], scales [groups, out]
    gptq = {}
    qlayers = []
    for e in range(E):
        qe = {}
        for p, s in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            qw = to_bf16_scales(quantize_symmetric_w4a32(torch.randn(s, generator=g) * 0.02, group_size=128))
            pre = f"model.layers.0.mlp.experts.{e}.{p}"
            gptq[f"{pre}.qweight"] = qw.qweight.T.contiguous()
            gptq[f"{pre}.scales"] = qw.scales.T.contiguous().to(torch.float16 if e % 2 else torch.float32)
            gptq[f"{pre}.g_idx"] = (torch.arange(qw.input_dim) // 128).to(torch.int32)
            # fp16 scales of bf16 values stay exact only when they are fp16-representable
            qe[p] = replace(qw, scales=gptq[f"{pre}.scales"].T.float())
        qlayers.append({"gate": qe["gate_proj"], "up": qe["up_proj"], "down": qe["down_proj"]})
    d2 = tmp_path / "gptq"
    d2.mkdir()
    save_file(gptq, str(d2 / "model.safetensors"))
    (d2 / "quantize_config.json").write_text(json.dumps({"bits": 4, "group_size": 128, "sym": True}))
    moe = HybridMoE(E, k, H, I, nn.ModuleDict(), mask, 0, str(d2), router_use_softmax=True,
                    normalize_topk_prob=True, expert_key_template=QWEN3_MOE_UNPACKED_SPEC.expert_key_template,
                    expert_proj_names=QWEN3_MOE_UNPACKED_SPEC.expert_proj_names)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    # the device keeps bf16 scales: the oracle sees the same rounding
    qlayers = [{p: to_bf16_scales(w) for p, w in q.items()} for q in qlayers]
    layer = Layer(MoEConfig("g", H, E, k, I), torch.zeros(E, H), qlayers)
    _check(out, oracle_forward(layer, x, logits))


def test_shared_expert_int8(gpu_device):
    announce("HybridMoE qwen2-moe shared expert int8")
    E, k, H, I, Is, T = 12, 4, 2048, 1408, 5632, 10
    experts = nn.ModuleDict({str(e): _init(SparseExpertMLP(H, I), 200 + e).to(gpu_device, torch.bfloat16)
                             for e in range(E)})
    shared = _init(SparseExpertMLP(H, Is), 7).to(gpu_device, torch.bfloat16)
    gate = _init(nn.Linear(H, 1, bias=False), 8).to(gpu_device, torch.bfloat16)
    moe = HybridMoE(E, k, H, I, experts, torch.ones(E, dtype=torch.bool), 0, "", router_use_softmax=True,
                    normalize_topk_prob=False, quantization="int8_per_channel",
                    shared_expert=shared, shared_expert_gate=gate)
    x, logits = _inputs(T, H, E, seed=4)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    q = lambda w: to_bf16_scales(quantize_symmetric_int8_per_channel(w.detach().float()))
    layer = Layer(MoEConfig("s", H, E, k, I, Is, True, False, "bf16", "int8_per_channel"), torch.zeros(E, H), [
        {"gate": q(experts[str(e)].w1.weight), "up": q(experts[str(e)].w3.weight),
         "down": q(experts[str(e)].w2.weight)} for e in range(E)],
        shared={"gate": q(shared.w1.weight), "up": q(shared.w3.weight), "down": q(shared.w2.weight)},
        shared_gate=gate.weight.detach().float().reshape(-1).cpu())
    _check(out, oracle_forward(layer, x, logits))


class _OracleOffload:
    """A stand-in offload backend with the reference's contract
    (nano_ktrans/kernels/offload_backend.py:40-52): the weighted sum of the
    non-resident experts' outputs, computed on the CPU by the oracle."""

    def __init__(self, experts, resident):
        self.experts, self.resident = experts, resident
        self.pending = None
        self.calls = 0

    def submit_forward(self, hidden_states, topk_ids, topk_weights, cuda_stream):
        assert topk_ids.dtype == torch.int64
        self.pending = (topk_ids.cpu().numpy(), topk_weights.float().cpu().numpy())

    def sync_forward(self, hidden_states, cuda_stream):
        ids, w = self.pending
        x = hidden_states.float().cpu().numpy()
        out = np.zeros_like(x)
        for t in range(x.shape[0]):
            for j in np.argsort(ids[t], kind="stable"):  # ascending expert id
                e = int(ids[t, j])
                if not self.resident[e]:
                    out[t] += w[t, j] * O.expert_forward(x[t:t + 1], self.experts[e])[0]
        self.calls += 1
        return torch.from_numpy(out).to(hidden_states.device, hidden_states.dtype)


@pytest.mark.parametrize("T", [5, 300])
def test_mixed_residency_with_offload_backend(gpu_device, T):
    """gpu_experts_mask False + an offload backend: non-resident experts get no GPU
    work, the backend's sum joins the combine, and the result matches the oracle's
    all-expert forward (decode and prefill forms)."""
    announce(f"HybridMoE mixed residency T={T}")
    E, k, H, I = 16, 4, 2048, 768
    experts = nn.ModuleDict({str(e): _init(SparseExpertMLP(H, I), 500 + e).to(gpu_device, torch.bfloat16)
                             for e in range(E)})
    mask = torch.tensor([e % 3 != 1 for e in range(E)])
    oracle_experts = [O.Expert(_bf16(experts[str(e)].w1.weight).numpy(), _bf16(experts[str(e)].w3.weight).numpy(),
                               _bf16(experts[str(e)].w2.weight).numpy()) for e in range(E)]
    backend = _OracleOffload(oracle_experts, mask.tolist())
    moe = HybridMoE(E, k, H, I, experts, mask, 0, "", router_use_softmax=True, normalize_topk_prob=True,
                    expert_key_template=MIXTRAL_SPEC.expert_key_template,
                    expert_proj_names=MIXTRAL_SPEC.expert_proj_names, offload_backend_impl=backend)
    x, logits = _inputs(T, H, E, seed=7)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    torch.cuda.synchronize()
    assert backend.calls == 1 and moe.diagnostics()["experts_resident"] == int(mask.sum())
    cfg = MoEConfig("m", H, E, k, I, 0, True, True, "bf16", "bf16")
    layer = Layer(cfg, torch.zeros(E, H), [
        {"gate": _bf16(experts[str(e)].w1.weight), "up": _bf16(experts[str(e)].w3.weight),
         "down": _bf16(experts[str(e)].w2.weight)} for e in range(E)])
    _check(out, oracle_forward(layer, x, logits))


class _RMSNorm(nn.Module):
    """The reference's RMSNorm parameters (nano_ktrans/layers/norm.py:5-9)."""

    def __init__(self, H, eps):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(H))


@pytest.mark.parametrize("T", [1, 16, 40, 300])
def test_fused_decoder_block(gpu_device, T):
    """FusedMoEBlock: hidden + MoE(RMSNorm(hidden)) with the fused router.  The
    RMSNorm output matches the oracle's within one bf16 step, the logits pass
    check_router_logits, and the block output matches hidden + the oracle's MoE
    forward on the GPU's normalised input and logits."""
    from moe_cases import bf16_steps, check_router_logits
    from nano_ktrans_amd import _native as N
    from nano_ktrans_amd.layers.moe_block import FusedMoEBlock
    announce(f"fused decoder block T={T}")
    E, k, H, I = 16, 4, 2048, 768
    experts = nn.ModuleDict({str(e): _init(SparseExpertMLP(H, I), 700 + e).to(gpu_device, torch.bfloat16)
                             for e in range(E)})
    gate = _init(nn.Linear(H, E, bias=False), 42).to(gpu_device, torch.bfloat16)
    norm = _RMSNorm(H, 1e-6)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(8)))
    norm = norm.to(gpu_device, torch.bfloat16)
    moe = HybridMoE(E, k, H, I, experts, torch.ones(E, dtype=torch.bool), 0, "", router_use_softmax=True,
                    normalize_topk_prob=True, expert_key_template=MIXTRAL_SPEC.expert_key_template,
                    expert_proj_names=MIXTRAL_SPEC.expert_proj_names, gate=gate)
    block = FusedMoEBlock(norm, moe)
    h = (torch.randn(T, H, generator=torch.Generator().manual_seed(T)) * 3.0).to(torch.bfloat16).to(gpu_device)
    out = block(h).clone()
    torch.cuda.synchronize()
    native = moe._native
    xg = native.region(T, N.WS_NORMED, torch.bfloat16, (T, H)).float().cpu().numpy()
    xo = O.rms_norm(h.float().cpu().numpy(), norm.weight.detach().float().cpu().numpy(), 1e-6)
    steps = bf16_steps(xg, xo)
    assert steps.max() <= 1 and (steps == 0).mean() > 0.99
    logits = native.region(T, N.WS_ROUTER_LOGITS, torch.bfloat16, (T, E)).clone()
    check_router_logits(logits.float().cpu().numpy(), xg, gate.weight.detach().float().cpu().numpy())
    cfg = MoEConfig("b", H, E, k, I, 0, True, True, "bf16", "bf16")
    layer = Layer(cfg, torch.zeros(E, H), [
        {"gate": _bf16(experts[str(e)].w1.weight), "up": _bf16(experts[str(e)].w3.weight),
         "down": _bf16(experts[str(e)].w2.weight)} for e in range(E)])
    moe_ref = oracle_forward(layer, torch.from_numpy(xg), logits.cpu())
    _check(out, h.float().cpu().numpy() + moe_ref)


def test_safetensors_qwen3_packed_dense(gpu_device, tmp_path):
    """Qwen3 checkpoint with packed dense experts: ``gate_up_proj.weight``
    [2I, H] split into gate (first I rows) and up by the loader
    (nano_ktrans/kernels/weight_loader.py:355-392), every expert read from disk."""
    from safetensors.torch import save_file

    announce("HybridMoE from safetensors: qwen3 packed gate_up (dense bf16)")
    E, k, H, I, T = 16, 8, 1024, 384, 11
    g = torch.Generator().manual_seed(21)
    ck, weights = {}, []
    for e in range(E):
        gu = (torch.randn(2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
        dn = (torch.randn(H, I, generator=g) * 0.02).to(torch.bfloat16)
        ck[f"model.layers.3.mlp.experts.{e}.gate_up_proj.weight"] = gu
        ck[f"model.layers.3.mlp.experts.{e}.down_proj.weight"] = dn
        weights.append({"gate": gu[:I].float(), "up": gu[I:].float(), "down": dn.float()})
    save_file(ck, str(tmp_path / "model.safetensors"))
    moe = HybridMoE(E, k, H, I, nn.ModuleDict(), torch.zeros(E, dtype=torch.bool), 3, str(tmp_path),
                    router_use_softmax=True, normalize_topk_prob=True, experts_are_packed=True,
                    expert_key_template=QWEN3_MOE_SPEC.expert_key_template,
                    expert_proj_names=QWEN3_MOE_SPEC.expert_proj_names)
    x, logits = _inputs(T, H, E, seed=22)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    assert moe._native.weight_format == "bf16"
    layer = Layer(MoEConfig("p", H, E, k, I, 0, True, True, "bf16", "bf16"), torch.zeros(E, H), weights)
    _check(out, oracle_forward(layer, x, logits))


def test_safetensors_qwen2_moe_with_shared_expert(gpu_device, tmp_path):
    """Qwen2-MoE checkpoint: routed experts under ``mlp.experts.{e}.{gate,up,down}_proj``,
    the shared expert under ``mlp.shared_expert.{gate,up,down}_proj`` and its gate
    ``mlp.shared_expert_gate.weight`` [1, H] (nano_ktrans/models/config.py:37-49,
    nano_ktrans/models/mixtral.py:404-426), quantized to int8 at ingest."""
    from safetensors.torch import save_file

    from nano_ktrans_amd.layers.expert_mlp import load_shared_expert_modules
    from nano_ktrans_amd.models.config import QWEN2_MOE_SPEC

    announce("HybridMoE from safetensors: qwen2-moe + shared expert (int8 at ingest)")
    E, k, H, I, Is, T = 12, 4, 2048, 256, 512, 10
    g = torch.Generator().manual_seed(23)
    ck, weights = {}, []
    for e in range(E):
        w = {p: (torch.randn(s, generator=g) * 0.02).to(torch.bfloat16)
             for p, s in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
        for p, t in w.items():
            ck[QWEN2_MOE_SPEC.expert_key_template.format(layer=0, expert=e, proj=p)] = t
        weights.append(w)
    shared = {p: (torch.randn(s, generator=g) * 0.02).to(torch.bfloat16)
              for p, s in (("gate", (Is, H)), ("up", (Is, H)), ("down", (H, Is)))}
    for p, t in shared.items():
        ck[QWEN2_MOE_SPEC.shared_expert_key_template.format(layer=0, proj=p)] = t
    sg = (torch.randn(1, H, generator=g) * 0.02).to(torch.bfloat16)
    ck["model.layers.0.mlp.shared_expert_gate.weight"] = sg
    save_file(ck, str(tmp_path / "model.safetensors"))
    sh_mod, sh_gate = load_shared_expert_modules(str(tmp_path), 0, QWEN2_MOE_SPEC, hidden_size=H,
                                                 shared_intermediate_size=Is)
    assert torch.equal(sh_mod.w1.weight, shared["gate"]) and torch.equal(sh_mod.w3.weight, shared["up"])
    assert torch.equal(sh_mod.w2.weight, shared["down"]) and torch.equal(sh_gate.weight, sg)
    moe = HybridMoE(E, k, H, I, nn.ModuleDict(), torch.zeros(E, dtype=torch.bool), 0, str(tmp_path),
                    router_use_softmax=QWEN2_MOE_SPEC.router_use_softmax,
                    normalize_topk_prob=QWEN2_MOE_SPEC.normalize_topk_prob,
                    expert_key_template=QWEN2_MOE_SPEC.expert_key_template,
                    expert_proj_names=QWEN2_MOE_SPEC.expert_proj_names, quantization="int8_per_channel",
                    shared_expert=sh_mod.to(gpu_device), shared_expert_gate=sh_gate.to(gpu_device))
    x, logits = _inputs(T, H, E, seed=24)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    q = lambda w: to_bf16_scales(quantize_symmetric_int8_per_channel(w.float()))
    layer = Layer(MoEConfig("s", H, E, k, I, Is, True, False, "bf16", "int8_per_channel"), torch.zeros(E, H),
                  [{p: q(w[p]) for p in ("gate", "up", "down")} for w in weights],
                  shared={p: q(shared[p]) for p in ("gate", "up", "down")},
                  shared_gate=sg.float().reshape(-1))
    _check(out, oracle_forward(layer, x, logits))


def test_safetensors_int8_per_channel_gptq(gpu_device, tmp_path):
    """int8 checkpoint in the GPTQ on-disk layout with ``group_size: -1`` (one
    scale per output row): qweight [in/4, out] int32 (byte j of a word = input
    row 4w + j, stored q + 128), scales [1, out] in fp16."""
    from safetensors.torch import save_file

    announce("HybridMoE from safetensors: int8 bits=8 group_size=-1")
    E, k, H, I, T = 8, 2, 512, 256, 13
    g = torch.Generator().manual_seed(25)
    ck, qlayers = {}, []
    for e in range(E):
        qe = {}
        for p, s in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            qw = to_bf16_scales(quantize_symmetric_int8_per_channel(torch.randn(s, generator=g) * 0.02))
            pre = f"model.layers.0.mlp.experts.{e}.{p}"
            ck[f"{pre}.qweight"] = qw.qweight.T.contiguous()
            # bf16 scales of these magnitudes are fp16-representable (exact round trip)
            ck[f"{pre}.scales"] = qw.scales.T.contiguous().to(torch.float16)
            assert torch.equal(ck[f"{pre}.scales"].float(), qw.scales.T.float())
            qe[p] = qw
        qlayers.append({"gate": qe["gate_proj"], "up": qe["up_proj"], "down": qe["down_proj"]})
    save_file(ck, str(tmp_path / "model.safetensors"))
    (tmp_path / "quantize_config.json").write_text(json.dumps({"bits": 8, "group_size": -1, "sym": True}))
    moe = HybridMoE(E, k, H, I, nn.ModuleDict(), torch.zeros(E, dtype=torch.bool), 0, str(tmp_path),
                    router_use_softmax=True, normalize_topk_prob=True,
                    expert_key_template=QWEN3_MOE_UNPACKED_SPEC.expert_key_template,
                    expert_proj_names=QWEN3_MOE_UNPACKED_SPEC.expert_proj_names)
    x, logits = _inputs(T, H, E, seed=26)
    out = moe(x.to(gpu_device), logits.to(gpu_device))
    assert moe._native.weight_format == "int8_per_channel"
    layer = Layer(MoEConfig("i8", H, E, k, I, 0, True, True, "bf16", "int8_per_channel"), torch.zeros(E, H),
                  qlayers)
    _check(out, oracle_forward(layer, x, logits))
