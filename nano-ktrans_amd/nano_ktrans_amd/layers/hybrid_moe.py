"""HybridMoE: drop-in MoE layer whose expert path runs as HIP kernels on MI355X.

Same constructor keywords and ``forward(hidden_states, router_logits)`` as
nano_ktrans/layers/hybrid_moe.py:55-86, 3310-3570.  By default every expert
lives in HBM (an MI355X holds the experts of a whole Qwen3-30B-A3B or
Mixtral-8x7B model), so the CPU/PIM offload split of the reference collapses
to one device path: experts whose ``gpu_experts_mask`` entry is False are read
from ``weight_path`` (dense ``.weight`` or GPTQ ``.qweight``/``.scales``) into
HBM instead of being served by an offload backend (pass
``offload_backend_impl`` to keep them out of HBM).  The residency control plane
(migration, prefetch caches, scheduler, expert-map store) has nothing to do in
that arrangement; its keywords are accepted and ignored, and an enabled
dynamic scheduler is rejected.

Additions, keyword-only and off by default:
  quantization       None | "int4_g128" | "int8_per_channel": quantize dense
                     experts at ingest (symmetric, bf16 scales).
  quantized_experts  {expert: {"gate", "up", "down": GPTQLinearWeight}}.
  shared_expert, shared_expert_gate
                     the Qwen2-MoE shared expert (SparseExpertMLP) and its
                     nn.Linear(H, 1) gate; forward then adds
                     sigmoid(gate(x)) * shared_expert(x) as
                     nano_ktrans/models/mixtral.py:215-218 does.
  gate               the router nn.Linear(H, E, bias=False); forward(x) without
                     router_logits then runs the router GEMV inside the path.
  offload_backend_impl
                     an object with the reference's offload contract
                     (submit_forward(hidden_states, topk_ids, topk_weights,
                     cuda_stream), sync_forward(hidden_states, cuda_stream),
                     nano_ktrans/kernels/offload_backend.py:40-52).  With it,
                     experts whose gpu_experts_mask entry is False stay out of
                     HBM and the backend serves them: the routing goes to
                     submit_forward, the resident experts run on the GPU, and
                     sync_forward's sum joins the combine
                     (nano_ktrans/layers/hybrid_moe.py:3373-3378, 3563-3570).
  max_tokens         largest token count per call (default 65536).
"""
from __future__ import annotations

from typing import Dict, Optional

import torch
from torch import nn

from ..kernels.quantized_ops import quantize_symmetric_int8_per_channel, quantize_symmetric_w4a32
from ..kernels.weight_loader import ExpertWeightLoader, GPTQLinearWeight
from ..native_moe import NativeMoE, weight_format_of
from ..utils.context import get_context

_QUANTIZERS = {
    "int4_g128": lambda w: quantize_symmetric_w4a32(w, group_size=128),
    "int8_per_channel": quantize_symmetric_int8_per_channel,
}


def _module_projections(module: nn.Module) -> Dict[str, torch.Tensor]:
    if hasattr(module, "projections"):
        return module.projections()
    if hasattr(module, "gate_up_proj"):
        gate, up = module.gate_up_proj.chunk(2, dim=0)
        return {"gate": gate, "up": up, "down": module.down_proj.weight}
    if hasattr(module, "w1"):
        return {"gate": module.w1.weight, "up": module.w3.weight, "down": module.w2.weight}
    if hasattr(module, "gate_proj"):
        return {"gate": module.gate_proj.weight, "up": module.up_proj.weight, "down": module.down_proj.weight}
    raise TypeError(f"cannot read expert projections from {type(module)!r}")


class HybridMoE(nn.Module):
    def __init__(
        self,
        num_experts: int,
        top_k: int,
        hidden_size: int,
        moe_intermediate_size: int,
        gpu_experts: nn.ModuleDict,
        gpu_experts_mask: torch.Tensor,
        layer_idx: int,
        weight_path: str,
        num_threads: int = 16,
        numa_pools: int = 1,
        chunked_prefill_size: int = 512,
        method: str = "AMXINT4",
        offload_backend: str = "cpu",
        offload_backend_kwargs: Optional[Dict[str, object]] = None,
        residency_plan=None,
        dynamic_expert_scheduler=None,
        router_use_softmax: bool = False,
        normalize_topk_prob: bool = True,
        expert_key_template: Optional[str] = None,
        expert_proj_names: Optional[Dict[str, str]] = None,
        experts_are_packed: bool = False,
        hidden_act: str = "silu",
        expert_prefetch_cache_size: int = 8,
        expert_prefetch_workers: int = 1,
        expert_warm_cache_size: int = 4,
        expert_prepared_cache_size: Optional[int] = None,
        prepared_controller_aggressiveness: float = 0.0,
        expert_map_store=None,
        expert_map_prefetch_top_k: int = 2,
        *,
        quantization: Optional[str] = None,
        quantized_experts: Optional[Dict[int, Dict[str, GPTQLinearWeight]]] = None,
        shared_expert: Optional[nn.Module] = None,
        shared_expert_gate: Optional[nn.Module] = None,
        gate: Optional[nn.Module] = None,
        offload_backend_impl: Optional[object] = None,
        max_tokens: int = 65536,
    ):
        super().__init__()
        if hidden_act != "silu":
            raise NotImplementedError(f"hidden_act={hidden_act!r}: the expert kernels implement SwiGLU (silu)")
        if dynamic_expert_scheduler is not None and getattr(dynamic_expert_scheduler, "enabled", False):
            raise NotImplementedError("expert migration scheduling is not part of the HBM-resident expert path")
        if quantization is not None and quantization not in _QUANTIZERS:
            raise ValueError(f"quantization must be None or one of {sorted(_QUANTIZERS)}")
        if (shared_expert is None) != (shared_expert_gate is None):
            raise ValueError("shared_expert and shared_expert_gate go together")
        self.num_experts = num_experts
        self.top_k = top_k
        self.hidden_size = hidden_size
        self.moe_intermediate_size = moe_intermediate_size
        self.gpu_experts = gpu_experts
        self.gpu_experts_mask = gpu_experts_mask
        self.layer_idx = layer_idx
        self.weight_path = weight_path
        self.chunked_prefill_size = chunked_prefill_size
        self.router_use_softmax = router_use_softmax
        self.normalize_topk_prob = normalize_topk_prob
        self.experts_are_packed = experts_are_packed
        self.hidden_act = hidden_act
        self.expert_key_template = (
            expert_key_template or "model.layers.{layer}.block_sparse_moe.experts.{expert}.{proj}.weight")
        self.expert_proj_names = expert_proj_names
        self.quantization = quantization
        self.quantized_experts = quantized_experts or {}
        self.shared_expert = shared_expert
        self.shared_expert_gate = shared_expert_gate
        # optional router nn.Linear(H, E, bias=False) (the decoder layer's self.gate,
        # nano_ktrans/models/mixtral.py:127): with it, forward(x) without
        # router_logits runs the router GEMV inside the expert path (the library)
        self.gate = gate
        self.max_tokens = max_tokens
        mask = [bool(m) for m in gpu_experts_mask.reshape(-1).tolist()] if gpu_experts_mask is not None \
            else [True] * num_experts
        if offload_backend_impl is not None and not all(mask):
            # the mask decides residency; the backend serves the other experts
            self.offload_backend = offload_backend_impl
            self.resident = mask
        else:
            self.offload_backend = None  # every expert is HBM-resident
            self.resident = [True] * num_experts
        self._native: Optional[NativeMoE] = None
        self.forward_calls = 0
        self.last_phase = ""

    # ---------------------------------------------------------------- weights
    def _expert_sources(self, e: int, loader: Optional[ExpertWeightLoader]):
        if e in self.quantized_experts:
            return self.quantized_experts[e]
        in_mask = bool(self.gpu_experts_mask[e]) if self.gpu_experts_mask is not None else True
        if in_mask and str(e) in self.gpu_experts:
            return _module_projections(self.gpu_experts[str(e)])
        if loader is None:
            raise KeyError(f"expert {e}: not in gpu_experts and no weight_path to read it from")
        proj_map = self.expert_proj_names or {"gate": "w1", "up": "w3", "down": "w2"}
        if loader.is_gptq_expert(self.layer_idx, e, self.expert_key_template, proj_map):
            if "gate_up" in proj_map:
                raise NotImplementedError("GPTQ checkpoints store gate and up separately")
            return {p: loader.load_gptq_expert_linear(layer_idx=self.layer_idx, expert_idx=e, proj_name=p,
                                                      key_template=self.expert_key_template,
                                                      proj_name_map=proj_map)
                    for p in ("gate", "up", "down")}
        return loader.load_expert(self.layer_idx, e, key_template=self.expert_key_template,
                                  proj_name_map=proj_map)

    def _materialize(self, device: torch.device, act_dtype: torch.dtype) -> None:
        loader = ExpertWeightLoader(self.weight_path) if self.weight_path else None
        sources = {e: self._expert_sources(e, loader) for e in range(self.num_experts) if self.resident[e]}
        if self.quantization is not None:
            quant = _QUANTIZERS[self.quantization]
            for e, src in sources.items():
                sources[e] = {p: (w if isinstance(w, GPTQLinearWeight) else quant(w.detach()))
                              for p, w in src.items()}
        formats = {weight_format_of(w, act_dtype) for src in sources.values() for w in src.values()}
        if len(formats) != 1:
            raise ValueError(f"experts mix weight formats {sorted(formats)}; pass quantization= to unify")
        fmt = formats.pop()
        shared_I = 0
        shared_src = None
        if self.shared_expert is not None:
            shared_src = _module_projections(self.shared_expert)
            if self.quantization is not None:
                quant = _QUANTIZERS[self.quantization]
                shared_src = {p: quant(w.detach()) for p, w in shared_src.items()}
            shared_I = int(shared_src["gate"].shape[0] if not isinstance(shared_src["gate"], GPTQLinearWeight)
                           else shared_src["gate"].output_dim)
        native = NativeMoE(
            num_experts=self.num_experts, top_k=self.top_k, hidden_size=self.hidden_size,
            intermediate_size=self.moe_intermediate_size, shared_intermediate_size=shared_I,
            weight_format=fmt, act_dtype=act_dtype, use_softmax=self.router_use_softmax,
            renorm=self.normalize_topk_prob, max_tokens=self.max_tokens, device=device)
        with torch.no_grad():
            for e, src in sources.items():
                native.load_expert(e, src["gate"], src["up"], src["down"])
            if shared_src is not None:
                native.load_shared_expert(shared_src["gate"], shared_src["up"], shared_src["down"],
                                          self.shared_expert_gate.weight.detach())
            if self.gate is not None and act_dtype == torch.bfloat16:
                native.load_router(self.gate.weight.detach())
        if self.offload_backend is not None:
            native.set_residency(torch.tensor(self.resident, dtype=torch.bool))
        self._native = native

    def reload_weights(self) -> None:
        """Re-ingest expert weights (after the caller changed them)."""
        if self._native is not None:
            dev, dt = self._native.device, self._native.act_dtype
            self._native = None
            self._materialize(dev, dt)

    # ---------------------------------------------------------------- compute
    def _ensure(self, x: torch.Tensor) -> NativeMoE:
        if self._native is None or self._native.device != x.device or self._native.act_dtype != x.dtype:
            self._materialize(x.device, x.dtype)
        return self._native

    def route(self, router_logits: torch.Tensor):
        """(topk_weights in the logits dtype, topk_ids int64), as the reference's routing block returns."""
        native = self._ensure(router_logits)
        ids, w, *_ = native.route(router_logits.reshape(-1, self.num_experts))
        return w.to(router_logits.dtype), ids.to(torch.int64)

    def forward(self, hidden_states: torch.Tensor, router_logits: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The reference forward (hidden_states, router_logits).  router_logits=None
        (with gate= given at construction, bf16 activations) computes the logits
        inside the expert path: the library runs the router GEMV, then routing."""
        self.forward_calls += 1
        self.last_phase = "prefill" if get_context().is_prefill else "decode"
        native = self._ensure(hidden_states)
        shape = hidden_states.shape
        x = hidden_states.reshape(-1, self.hidden_size)
        if self.offload_backend is not None:
            return self._forward_mixed(native, x, router_logits).view(shape)
        if router_logits is None:
            if self.gate is None:
                raise ValueError("router_logits is required unless HybridMoE was built with gate=")
            if hidden_states.dtype != torch.bfloat16:
                raise ValueError("the fused router needs bf16 activations; pass router_logits")
            return native.forward_hidden(x).view(shape)
        out = native.forward(x, router_logits.reshape(-1, self.num_experts))
        return out.view(shape)

    def _forward_mixed(self, native: NativeMoE, x: torch.Tensor, router_logits: Optional[torch.Tensor]):
        """Routing -> backend submit -> resident experts on the GPU -> backend sync ->
        combine with the backend's sum (hybrid_moe.py:3373-3378, 3563-3570)."""
        T = x.shape[0]
        stream = torch.cuda.current_stream(x.device).cuda_stream
        if router_logits is None:
            if self.gate is None:
                raise ValueError("router_logits is required unless HybridMoE was built with gate=")
            logits, ids, w, *_ = native.route_hidden(x)
        else:
            logits = router_logits.reshape(-1, self.num_experts)
            ids, w, *_ = native.route(logits)
        self.offload_backend.submit_forward(x, ids.to(torch.int64), w.to(logits.dtype), stream)
        native.experts(x)
        if self.shared_expert is not None:
            native.shared(x)
        extra = self.offload_backend.sync_forward(x, stream)
        return native.combine(T, extra=extra.reshape(T, self.hidden_size).to(x.dtype))

    def diagnostics(self) -> dict:
        n = self._native
        return {
            "layer_idx": self.layer_idx,
            "forward_calls": self.forward_calls,
            "last_phase": self.last_phase,
            "weight_format": None if n is None else n.weight_format,
            "experts_resident": sum(self.resident),
            "offload_backend": None if self.offload_backend is None else type(self.offload_backend).__name__,
        }
