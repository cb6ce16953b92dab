"""Seeded MoE problems at the benchmark configurations.

Shapes and seeds:
  tiny_mixtral_fp32  H=256  E=8   k=2 I=512   fp32, softmax -> top-2 -> renorm, seed 0
  qwen3_int4         H=2048 E=128 k=8 I=768   bf16 act, int4 g128 bf16 scales, softmax+renorm, seed 1
  qwen3_int8         same fp32 weights as qwen3_int4, int8 per-channel, Zipf(1.1) logit bias, seed 1
  mixtral_int4       H=4096 E=8   k=2 I=14336 bf16 act, int4 g128, top-k on logits then softmax, seed 2
  qwen15_int8_shared H=2048 E=60  k=4 I=1408  shared I=5632 + sigmoid gate, int8 per-channel,
                     softmax without renorm, seed 3
  small_int8_shared  H=256  E=8   k=2 I=128   shared I=128, int8 per-channel, softmax+renorm, seed 4
                     (prefill-form K loops of 4 and 2 stages)
Activations ~N(0,1); router and expert weights ~N(0, 0.02); router logits are
x . router^T in fp32, then cast to the activation dtype.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import List, Optional

import numpy as np
import torch

import oracle as O
from nano_ktrans_amd.kernels.quantized_ops import (quantize_symmetric_int8_per_channel,
                                                   quantize_symmetric_w4a32, to_bf16_scales)
from nano_ktrans_amd.kernels.weight_loader import GPTQLinearWeight


@dataclass(frozen=True)
class MoEConfig:
    name: str
    H: int
    E: int
    k: int
    I: int
    Is: int = 0
    softmax: bool = True
    renorm: bool = True
    act: str = "bf16"          # "bf16" | "f32"
    wfmt: str = "int4_g128"    # "f32" | "bf16" | "int8_per_channel" | "int4_g128"
    seed: int = 0
    zipf: float = 0.0

    @property
    def act_dtype(self) -> torch.dtype:
        return torch.float32 if self.act == "f32" else torch.bfloat16

    def decode_form(self, T: int) -> bool:
        """Whether the library runs a batch of T tokens in its decode form:
        up to 4.5 tokens per expert (T k / E) for int8 weights (3.5 with a
        shared expert), 8 for int4 (6 where I >= 8192) and 12 for the others."""
        int8 = 3.5 if self.Is > 0 else 4.5
        int4 = 6 if self.I >= 8192 else 8
        return T * self.k <= {"int8_per_channel": int8, "int4_g128": int4}.get(self.wfmt, 12) * self.E

    def shared_in_routed_launches(self, T: int) -> bool:
        """Whether the layer runs the shared expert inside the routed experts'
        decode-form launches (as Is / I chunks of the routed shape) instead of
        launches of its own."""
        return (self.Is > 0 and self.Is % self.I == 0 and self.Is // self.I <= 8 and self.act == "bf16"
                and self.decode_form(T) and T <= 256)


CONFIGS = {
    "tiny_mixtral_fp32": MoEConfig("tiny_mixtral_fp32", 256, 8, 2, 512, 0, True, True, "f32", "f32", 0),
    "qwen3_int4": MoEConfig("qwen3_int4", 2048, 128, 8, 768, 0, True, True, "bf16", "int4_g128", 1),
    "qwen3_int8": MoEConfig("qwen3_int8", 2048, 128, 8, 768, 0, True, True, "bf16", "int8_per_channel", 1, 1.1),
    "mixtral_int4": MoEConfig("mixtral_int4", 4096, 8, 2, 14336, 0, False, True, "bf16", "int4_g128", 2),
    "qwen15_int8_shared": MoEConfig("qwen15_int8_shared", 2048, 60, 4, 1408, 5632, True, False, "bf16",
                                    "int8_per_channel", 3),
    # K of 256 / 128: the prefill form's K loop is only its last, partial round
    "small_int8_shared": MoEConfig("small_int8_shared", 256, 8, 2, 128, 128, True, True, "bf16",
                                   "int8_per_channel", 4),
}


@dataclass
class Layer:
    cfg: MoEConfig
    router: torch.Tensor                      # [E, H] fp32
    experts: List[dict]                       # {"gate","up","down"}: fp32 tensor or GPTQLinearWeight
    shared: Optional[dict] = None
    shared_gate: Optional[torch.Tensor] = None  # [H] fp32 (activation-dtype valued)


def _quantize(w: torch.Tensor, wfmt: str, act_dtype: torch.dtype):
    if wfmt == "int4_g128":
        return to_bf16_scales(quantize_symmetric_w4a32(w, group_size=128))
    if wfmt == "int8_per_channel":
        return to_bf16_scales(quantize_symmetric_int8_per_channel(w))
    if wfmt == "bf16":
        return w.to(torch.bfloat16).to(torch.float32)
    return w.to(torch.float32)


def build_layer(cfg: MoEConfig, device: str = "cpu", num_experts: Optional[int] = None) -> Layer:
    """Random-init weights of the config's architecture (``num_experts`` can cut E down)."""
    E = num_experts or cfg.E
    g = torch.Generator(device=device)
    g.manual_seed(cfg.seed)

    def randn(*shape):
        return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * 0.02)

    router = randn(E, cfg.H)
    experts = []
    for _ in range(E):
        gate_up = randn(2 * cfg.I, cfg.H)
        down = randn(cfg.H, cfg.I)
        experts.append({
            "gate": _quantize(gate_up[: cfg.I], cfg.wfmt, cfg.act_dtype),
            "up": _quantize(gate_up[cfg.I:], cfg.wfmt, cfg.act_dtype),
            "down": _quantize(down, cfg.wfmt, cfg.act_dtype),
        })
    shared = shared_gate = None
    if cfg.Is:
        shared = {
            "gate": _quantize(randn(cfg.Is, cfg.H), cfg.wfmt, cfg.act_dtype),
            "up": _quantize(randn(cfg.Is, cfg.H), cfg.wfmt, cfg.act_dtype),
            "down": _quantize(randn(cfg.H, cfg.Is), cfg.wfmt, cfg.act_dtype),
        }
        sg = randn(cfg.H)
        shared_gate = sg.to(cfg.act_dtype).to(torch.float32)
    return Layer(replace(cfg, E=E), router, experts, shared, shared_gate)


def build_inputs(layer: Layer, T: int, seed: int = 1234, device: str = "cpu"):
    """x [T, H] and router_logits [T, E] in the activation dtype."""
    cfg = layer.cfg
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    x = torch.randn(T, cfg.H, generator=g, device=device, dtype=torch.float32)
    x = x.to(cfg.act_dtype)
    logits = x.to(torch.float32) @ layer.router.to(device).T
    if cfg.zipf:
        e = torch.arange(cfg.E, device=device, dtype=torch.float32)
        logits = logits - cfg.zipf * torch.log(e + 1.0)
    return x, logits.to(cfg.act_dtype)


# ---------------------------------------------------------------- oracle bridge
def _to_oracle(w):
    if isinstance(w, GPTQLinearWeight):
        return O.QWeight(w.qweight.cpu().numpy(), w.scales.cpu().numpy().astype(np.float32), w.bits, w.group_size)
    return w.cpu().numpy().astype(np.float32)


def oracle_forward(layer: Layer, x: torch.Tensor, logits: torch.Tensor, return_parts: bool = False,
                   h_bf16: bool = False):
    cfg = layer.cfg
    experts = [O.Expert(_to_oracle(e["gate"]), _to_oracle(e["up"]), _to_oracle(e["down"])) for e in layer.experts]
    shared = None
    if layer.shared is not None:
        shared = O.Expert(_to_oracle(layer.shared["gate"]), _to_oracle(layer.shared["up"]),
                          _to_oracle(layer.shared["down"]))
    return O.moe_forward(
        x.float().cpu().numpy(), logits.float().cpu().numpy(), experts, cfg.k, cfg.softmax, cfg.renorm,
        cfg.act == "bf16", shared=shared,
        shared_gate=None if layer.shared_gate is None else layer.shared_gate.cpu().numpy(),
        return_parts=return_parts, h_bf16=h_bf16)


def native_layer(layer: Layer, device, max_tokens: int = 8192):
    from nano_ktrans_amd.native_moe import NativeMoE

    cfg = layer.cfg
    n = NativeMoE(num_experts=cfg.E, top_k=cfg.k, hidden_size=cfg.H, intermediate_size=cfg.I,
                  shared_intermediate_size=cfg.Is, weight_format=cfg.wfmt, act_dtype=cfg.act_dtype,
                  use_softmax=cfg.softmax, renorm=cfg.renorm, max_tokens=max_tokens, device=device)
    for e, ex in enumerate(layer.experts):
        n.load_expert(e, ex["gate"], ex["up"], ex["down"])
    if layer.shared is not None:
        n.load_shared_expert(layer.shared["gate"], layer.shared["up"], layer.shared["down"], layer.shared_gate)
    return n


def tolerances(cfg: MoEConfig):
    """(max-abs, rel-L2) bounds: bf16 activations 2e-2 / 1e-2, fp32 with dense weights - / 1e-4."""
    if cfg.act == "f32":
        return math.inf, 1e-4
    return 2e-2, 1e-2


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |x| (8 significant bits)."""
    _, ex = np.frexp(np.abs(np.asarray(x, dtype=np.float64)))
    return np.ldexp(1.0, ex - 8)


def bf16_steps(a, b) -> np.ndarray:
    """Elementwise distance in bf16 steps between two arrays of bf16 values (float32)."""
    ia = (np.ascontiguousarray(a, np.float32).view(np.int32) >> 16).astype(np.int64)
    ib = (np.ascontiguousarray(b, np.float32).view(np.int32) >> 16).astype(np.int64)
    # sign-magnitude -> a monotone integer line (+0 and -0 both map to 0)
    ia = np.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFF), ib)
    return np.abs(ia - ib)


def check_router_logits(got: np.ndarray, x: np.ndarray, gate: np.ndarray) -> None:
    """GPU bf16 logits against the oracle's single rounding of the exact dot
    products: each within one bf16 step, or, where cancellation leaves a value
    near zero, within fp32 summation error (2^-20 x sum |x_i w_i|, a bound far
    above a 2048-term fp32 sum's typical error); nearly all bit-equal."""
    ref = O.router_logits(x, gate)
    steps = bf16_steps(got, ref)
    absterm = np.abs(np.asarray(x, np.float64)) @ np.abs(np.asarray(gate, np.float64)).T
    near = np.abs(np.asarray(got, np.float64) - ref) <= 2.0 ** -20 * absterm
    bad = ~((steps <= 1) | near)
    assert not bad.any(), f"{bad.sum()} logits off: got {got[bad][:4]} want {ref[bad][:4]}"
    assert (steps == 0).mean() > 0.99


def compare(got: np.ndarray, ref: np.ndarray, cfg: MoEConfig):
    """Check a GPU output against the oracle's fp32 result.

    bf16 outputs: every element within max(2e-2, one bf16 ulp of the oracle value) of the
    oracle rounded to bf16 -- where |y| >= 4 one bf16 ulp exceeds 2e-2, so a single flip of
    the final rounding must be allowed there -- and rel-L2 <= 1e-2 against the fp32 oracle.
    fp32 outputs: rel-L2 <= 1e-4.  Returns (max-abs vs the rounded oracle, rel-L2)."""
    got = np.asarray(got, dtype=np.float32)
    if cfg.act == "f32":
        rel = O.rel_l2(got, ref)
        assert rel <= 1e-4, f"rel-L2 {rel} > 1e-4"
        return float(np.max(np.abs(got - ref))) if got.size else 0.0, rel
    ref_b = O.bf16_round(ref)
    d = np.abs(got.astype(np.float64) - ref_b)
    bound = np.maximum(2e-2, bf16_ulp(ref_b))
    worst = np.unravel_index(np.argmax(d - bound), d.shape) if d.size else None
    assert d.size == 0 or np.all(d <= bound), \
        f"|d|={d[worst]} > {bound[worst]} at {worst} (ref {ref_b[worst]}, got {got[worst]})"
    rel = O.rel_l2(got, ref)
    assert rel <= 1e-2, f"rel-L2 {rel} > 1e-2"
    return float(np.max(d)) if d.size else 0.0, rel
