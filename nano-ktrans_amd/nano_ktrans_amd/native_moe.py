"""Device-resident MoE layer driven through the C ABI (include/nkt_moe.h).

``NativeMoE`` owns one layer's packed expert weights (torch tensors in HBM,
written once by ``nkt_moe_pack_weight``) and a workspace, and enqueues the
five kernels on torch's current HIP stream.  No call synchronises the host.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional, Sequence, Union

import torch

from . import _native as N
from .kernels.weight_loader import GPTQLinearWeight

WeightLike = Union[torch.Tensor, GPTQLinearWeight]

_FORMATS = {
    "f32": N.WEIGHT_F32,
    "bf16": N.WEIGHT_BF16,
    "int8_per_channel": N.WEIGHT_INT8_PC,
    "int4_g128": N.WEIGHT_INT4_G128,
}


def weight_format_of(w: WeightLike, act_dtype: torch.dtype) -> str:
    """The device weight format a source weight maps to."""
    if isinstance(w, GPTQLinearWeight):
        if w.bits == 4 and w.group_size == 128:
            return "int4_g128"
        if w.bits == 8 and w.group_size == w.input_dim:
            return "int8_per_channel"
        raise NotImplementedError(
            f"unsupported quantized weight: bits={w.bits} group_size={w.group_size} "
            "(supported: int4 group 128, int8 one group per row)")
    return "f32" if act_dtype == torch.float32 else "bf16"


def _require_cuda(device: torch.device) -> None:
    if device.type != "cuda" or not torch.cuda.is_available():
        raise N.NativeError(
            "the MoE expert path runs only on a ROCm GPU (gfx950); got device "
            f"{device} with torch.cuda.is_available()={torch.cuda.is_available()}")


class NativeMoE:
    """One MoE layer: routing flags, shapes, packed weights and a workspace."""

    def __init__(
        self,
        *,
        num_experts: int,
        top_k: int,
        hidden_size: int,
        intermediate_size: int,
        shared_intermediate_size: int = 0,
        weight_format: str = "bf16",
        act_dtype: torch.dtype = torch.bfloat16,
        use_softmax: bool = True,
        renorm: bool = True,
        max_tokens: int = 4096,
        device: Optional[torch.device] = None,
    ):
        self.device = torch.device(device if device is not None else "cuda")
        _require_cuda(self.device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        if weight_format not in _FORMATS:
            raise ValueError(f"unknown weight_format {weight_format!r}")
        if act_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"activations must be fp32 or bf16, got {act_dtype}")
        self.lib = N.lib()
        self.err = N.ErrBuf()
        self.num_experts = num_experts
        self.top_k = top_k
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.shared_intermediate_size = shared_intermediate_size
        self.weight_format = weight_format
        self.act_dtype = act_dtype
        self.max_tokens = max_tokens
        flags = (N.ROUTE_SOFTMAX if use_softmax else 0) | (N.ROUTE_RENORM if renorm else 0)
        with torch.cuda.device(self.device):
            h = self.lib.nkt_moe_create(
                num_experts, top_k, hidden_size, intermediate_size, shared_intermediate_size,
                _FORMATS[weight_format], N.DTYPE_F32 if act_dtype == torch.float32 else N.DTYPE_BF16,
                flags, max_tokens, self.err.buf, self.err.size)
        if not h:
            raise N.NativeError(f"nkt_moe_create failed: {self.err.buf.value.decode()}")
        self.handle = ctypes.c_void_p(h)
        self.slots: Dict[int, torch.Tensor] = {}
        for slot in range(N.NUM_SLOTS):
            if slot == N.SLOT_ROUTER:
                continue  # allocated and bound by load_router (the fused router is optional)
            nbytes = self._slot_bytes(slot)
            if nbytes:
                self.slots[slot] = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self._bind()
        self._ws: Optional[torch.Tensor] = None
        self._ws_streams: set = set()

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                self.lib.nkt_moe_destroy(h)
            except Exception:
                pass

    # ------------------------------------------------------------------ weights
    def _slot_bytes(self, slot: int) -> int:
        nbytes = ctypes.c_size_t(0)
        self.err.check(self.lib.nkt_moe_weight_bytes(self.handle, slot, ctypes.byref(nbytes),
                                                     self.err.buf, self.err.size), "nkt_moe_weight_bytes")
        return nbytes.value

    def _bind(self) -> None:
        arr = (ctypes.c_void_p * N.NUM_SLOTS)()
        for slot in range(N.NUM_SLOTS):
            t = self.slots.get(slot)
            arr[slot] = t.data_ptr() if t is not None else None
        self.err.check(self.lib.nkt_moe_bind_weights(self.handle, arr, self.err.buf, self.err.size),
                       "nkt_moe_bind_weights")

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _source(self, parts: Sequence[WeightLike]):
        """Stack row blocks (gate then up, or a single projection) in the source layout."""
        fmt = self.weight_format
        if fmt in ("int4_g128", "int8_per_channel"):
            for p in parts:
                if not isinstance(p, GPTQLinearWeight) or weight_format_of(p, self.act_dtype) != fmt:
                    raise ValueError(f"expected {fmt} GPTQLinearWeight parts")
            q = torch.cat([p.qweight.to(torch.int32) for p in parts], dim=0)
            s = torch.cat([p.scales.to(torch.float32) for p in parts], dim=0).to(torch.bfloat16)
            return (q.to(self.device).contiguous(), s.to(self.device).contiguous())
        dt = torch.float32 if fmt == "f32" else torch.bfloat16
        for p in parts:
            if isinstance(p, GPTQLinearWeight):
                raise ValueError("dense weight format given a quantized weight")
        w = torch.cat([p.to(dt) for p in parts], dim=0)
        return (w.to(self.device).contiguous(), None)

    def _pack(self, slot: int, expert: int, parts: Sequence[WeightLike], n: int, k: int) -> None:
        src, scales = self._source(parts)
        rows = src.shape[0]
        if rows != n:
            raise ValueError(f"slot {slot}: expected {n} rows, got {rows}")
        cols = src.shape[1] * (8 if self.weight_format == "int4_g128" else 4 if self.weight_format == "int8_per_channel" else 1)
        if cols != k:
            raise ValueError(f"slot {slot}: expected {k} input columns, got {cols}")
        dst = self.slots[slot]
        dst_s = self.slots.get(slot + 1)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_pack_weight(
                self.handle, slot, expert, src.data_ptr(), scales.data_ptr() if scales is not None else None,
                dst.data_ptr(), dst_s.data_ptr() if dst_s is not None else None, self._stream(),
                self.err.buf, self.err.size), "nkt_moe_pack_weight")
        # src/scales may be freed now: the caching allocator only hands their
        # memory to work enqueued later on this stream, after the pack kernel.

    def load_expert(self, expert: int, gate: WeightLike, up: WeightLike, down: WeightLike) -> None:
        """Ingest one routed expert: gate/up [I, H], down [H, I] (dense tensors or GPTQLinearWeight)."""
        I, H = self.intermediate_size, self.hidden_size
        self._pack(N.SLOT_GATE_UP, expert, [gate, up], 2 * I, H)
        self._pack(N.SLOT_DOWN, expert, [down], H, I)

    def load_shared_expert(self, gate: WeightLike, up: WeightLike, down: WeightLike,
                           gate_weight: torch.Tensor) -> None:
        """Ingest the shared expert and its ``shared_expert_gate.weight`` [1, H]."""
        if self.shared_intermediate_size <= 0:
            raise ValueError("this layer was created without a shared expert")
        Is, H = self.shared_intermediate_size, self.hidden_size
        self._pack(N.SLOT_SHARED_GATE_UP, 0, [gate, up], 2 * Is, H)
        self._pack(N.SLOT_SHARED_DOWN, 0, [down], H, Is)
        g = gate_weight.reshape(-1).to(self.act_dtype).to(self.device).contiguous()
        if g.numel() != H:
            raise ValueError(f"shared_expert_gate weight must have {H} elements")
        self.slots[N.SLOT_SHARED_GATE].view(self.act_dtype).copy_(g)

    def load_router(self, gate_weight: torch.Tensor) -> None:
        """Ingest the router gate weight [E, H] (nn.Linear(H, E, bias=False).weight) for
        the fused router GEMV of ``route_hidden`` / ``forward_hidden`` (bf16 layers)."""
        if self.act_dtype != torch.bfloat16:
            raise ValueError("the fused router needs bf16 activations")
        w = gate_weight.to(torch.bfloat16).to(self.device).contiguous()
        if tuple(w.shape) != (self.num_experts, self.hidden_size):
            raise ValueError(f"router weight must be [{self.num_experts}, {self.hidden_size}], got {tuple(w.shape)}")
        if N.SLOT_ROUTER not in self.slots:
            self.slots[N.SLOT_ROUTER] = torch.empty(self._slot_bytes(N.SLOT_ROUTER), dtype=torch.uint8,
                                                    device=self.device)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_pack_weight(
                self.handle, N.SLOT_ROUTER, 0, w.data_ptr(), None, self.slots[N.SLOT_ROUTER].data_ptr(), None,
                self._stream(), self.err.buf, self.err.size), "nkt_moe_pack_weight(router)")
        self._bind()

    # ---------------------------------------------------------------- workspace
    def workspace_bytes(self, num_tokens: int) -> int:
        nbytes = ctypes.c_size_t(0)
        self.err.check(self.lib.nkt_moe_workspace_bytes(self.handle, num_tokens, ctypes.byref(nbytes),
                                                        self.err.buf, self.err.size), "nkt_moe_workspace_bytes")
        return nbytes.value

    def workspace(self, num_tokens: int) -> torch.Tensor:
        """The workspace for num_tokens tokens, grown when too small.  Every
        stream a call enqueued on is remembered: before a smaller buffer is
        dropped it is marked in use on each of them (record_stream), so the
        caching allocator does not hand its memory out while kernels queued
        there may still read or write it.  (The library's own side stream
        joins back into the caller's stream before each call returns.)"""
        need = self.workspace_bytes(num_tokens)
        stream = torch.cuda.current_stream(self.device)
        if self._ws is None or self._ws.numel() < need:
            if self._ws is not None:
                for s in self._ws_streams:
                    self._ws.record_stream(s)
            # zeroed: the workspace's leading sync area must start at zero (every call leaves it so)
            self._ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=self.device)
            self._ws_streams = set()
        self._ws_streams.add(stream)
        return self._ws

    def region(self, num_tokens: int, region: int, dtype: torch.dtype, shape) -> torch.Tensor:
        """A view of one workspace region (valid after the call that fills it)."""
        off = ctypes.c_size_t(0)
        self.err.check(self.lib.nkt_moe_workspace_region(self.handle, num_tokens, region, ctypes.byref(off),
                                                         self.err.buf, self.err.size), "nkt_moe_workspace_region")
        ws = self.workspace(num_tokens)
        n = 1
        for s in shape:
            n *= int(s)
        esz = torch.tensor([], dtype=dtype).element_size()
        return ws[off.value: off.value + n * esz].view(dtype).view(*shape)

    # ------------------------------------------------------------------ compute
    def _check_input(self, t: torch.Tensor, cols: int, name: str) -> torch.Tensor:
        if t.device != self.device:
            raise ValueError(f"{name} on {t.device}, layer on {self.device}")
        if t.dtype != self.act_dtype:
            raise ValueError(f"{name} dtype {t.dtype}, layer expects {self.act_dtype}")
        t = t.reshape(-1, t.shape[-1])
        if t.shape[1] != cols:
            raise ValueError(f"{name} has {t.shape[1]} columns, expected {cols}")
        return t.contiguous()

    def route(self, router_logits: torch.Tensor):
        """K1 + K2.  Returns (ids int32 [T,k], weights fp32 [T,k], counts [E], offsets [E+1],
        perm [T*k], inv [T*k]) as views of the workspace."""
        logits = self._check_input(router_logits, self.num_experts, "router_logits")
        T = logits.shape[0]
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_route(self.handle, logits.data_ptr(), T, ws.data_ptr(), ws.numel(),
                                                  self._stream(), self.err.buf, self.err.size), "nkt_moe_route")
        k, E = self.top_k, self.num_experts
        return (self.region(T, N.WS_TOPK_IDS, torch.int32, (T, k)),
                self.region(T, N.WS_TOPK_WEIGHTS, torch.float32, (T, k)),
                self.region(T, N.WS_COUNTS, torch.int32, (E,)),
                self.region(T, N.WS_OFFSETS, torch.int32, (E + 1,)),
                self.region(T, N.WS_PERM, torch.int32, (T * k,)),
                self.region(T, N.WS_INV, torch.int32, (T * k,)))

    def _check_routing(self, topk_ids: torch.Tensor, topk_weights: torch.Tensor, T: int):
        """The caller's routing as the C ABI takes it: int64 ids and fp32 weights, [T, k], contiguous."""
        k = self.top_k
        for name, t in (("topk_ids", topk_ids), ("topk_weights", topk_weights)):
            if t.device != self.device:
                raise ValueError(f"{name} on {t.device}, layer on {self.device}")
            if t.numel() != T * k:
                raise ValueError(f"{name} has {t.numel()} entries, expected [{T}, {k}]")
        if topk_ids.dtype not in (torch.int64, torch.int32):
            raise ValueError(f"topk_ids must be an integer tensor, got {topk_ids.dtype}")
        if not topk_weights.dtype.is_floating_point:
            raise ValueError(f"topk_weights must be floating point, got {topk_weights.dtype}")
        ids = topk_ids.reshape(T, k).to(torch.int64).contiguous()
        w = topk_weights.reshape(T, k).to(torch.float32).contiguous()
        self._routing = (ids, w)  # kept alive while the kernels read them
        return ids, w

    def route_given(self, topk_ids: torch.Tensor, topk_weights: torch.Tensor):
        """K2 from the caller's routing (K1 not run): ``topk_ids`` [T, k] (int64 or int32) and
        ``topk_weights`` [T, k].  Returns the same workspace views as ``route``.  A slot whose id is
        outside [0, E) or repeats an earlier slot's id of its token is dropped and sets the
        STATUS_BAD_ROUTING word (``check_status``)."""
        T = topk_ids.reshape(-1, self.top_k).shape[0] if topk_ids.numel() else 0
        ids, w = self._check_routing(topk_ids, topk_weights, T)
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_route_given(self.handle, ids.data_ptr(), w.data_ptr(), T, ws.data_ptr(),
                                                        ws.numel(), self._stream(), self.err.buf, self.err.size),
                           "nkt_moe_route_given")
        k, E = self.top_k, self.num_experts
        return (self.region(T, N.WS_TOPK_IDS, torch.int32, (T, k)),
                self.region(T, N.WS_TOPK_WEIGHTS, torch.float32, (T, k)),
                self.region(T, N.WS_COUNTS, torch.int32, (E,)),
                self.region(T, N.WS_OFFSETS, torch.int32, (E + 1,)),
                self.region(T, N.WS_PERM, torch.int32, (T * k,)),
                self.region(T, N.WS_INV, torch.int32, (T * k,)))

    def forward_routed(self, hidden_states: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The layer on the caller's routing: out[t] = sum over the token's slots (ascending expert id)
        of topk_weights[t, j] * expert_{topk_ids[t, j]}(x_t), plus the gated shared expert when the
        layer has one; experts marked non-resident (``set_residency``) add nothing."""
        x = self._check_input(hidden_states, self.hidden_size, "hidden_states")
        T = x.shape[0]
        ids, w = self._check_routing(topk_ids, topk_weights, T)
        if out is None:
            out = torch.empty(T, self.hidden_size, dtype=self.act_dtype, device=self.device)
        if T == 0:
            return out
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_forward_routed(self.handle, x.data_ptr(), ids.data_ptr(), w.data_ptr(), T,
                                                           out.data_ptr(), ws.data_ptr(), ws.numel(), self._stream(),
                                                           self.err.buf, self.err.size), "nkt_moe_forward_routed")
        return out

    # ------------------------------------------------------------------ status
    def status(self) -> Dict[str, int]:
        """The workspace's status word (synchronises the device): bad_routing = 1 when a
        given-routing call dropped a slot since it was last cleared, else 0."""
        if self._ws is None:
            return {"bad_routing": 0}
        torch.cuda.synchronize(self.device)
        words = self._ws[:128].view(torch.int32).cpu()
        return {"bad_routing": int(words[N.STATUS_BAD_ROUTING])}

    def check_status(self, clear: bool = True) -> None:
        """Raise ``NativeError`` if a status word reports a fault (after clearing it when ``clear``)."""
        st = self.status()
        bad = {k: v for k, v in st.items() if v}
        if bad and clear:
            self._ws[:128].view(torch.int32)[N.STATUS_BAD_ROUTING].zero_()
            torch.cuda.synchronize(self.device)
        if bad:
            raise N.NativeError(f"MoE layer status: {bad}")

    def route_hidden(self, hidden_states: torch.Tensor):
        """Router GEMV + K1 + K2 from hidden states (after ``load_router``).  Returns
        (router_logits bf16 [T, E], ids, weights, counts, offsets, perm, inv) as views."""
        x = self._check_input(hidden_states, self.hidden_size, "hidden_states")
        T = x.shape[0]
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_route_hidden(self.handle, x.data_ptr(), T, ws.data_ptr(), ws.numel(),
                                                         self._stream(), self.err.buf, self.err.size),
                           "nkt_moe_route_hidden")
        k, E = self.top_k, self.num_experts
        return (self.region(T, N.WS_ROUTER_LOGITS, torch.bfloat16, (T, E)),
                self.region(T, N.WS_TOPK_IDS, torch.int32, (T, k)),
                self.region(T, N.WS_TOPK_WEIGHTS, torch.float32, (T, k)),
                self.region(T, N.WS_COUNTS, torch.int32, (E,)),
                self.region(T, N.WS_OFFSETS, torch.int32, (E + 1,)),
                self.region(T, N.WS_PERM, torch.int32, (T * k,)),
                self.region(T, N.WS_INV, torch.int32, (T * k,)))

    def experts(self, hidden_states: torch.Tensor):
        """K3 after ``route``: returns h [T*k, I] (act dtype) by position and y [T*k, H] (fp32), whose row is
        the pair t*k + slot in the decode form (T*k / E up to 4.5 for int8 weights (3.5 with a shared
        expert), 8 for int4 (6 for I >= 8192), 12 for the others) and the position otherwise."""
        x = self._check_input(hidden_states, self.hidden_size, "hidden_states")
        T = x.shape[0]
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_experts(self.handle, x.data_ptr(), T, ws.data_ptr(), ws.numel(),
                                                    self._stream(), self.err.buf, self.err.size), "nkt_moe_experts")
        P = T * self.top_k
        return (self.region(T, N.WS_H, self.act_dtype, (P, self.intermediate_size)),
                self.region(T, N.WS_Y, torch.float32, (P, self.hidden_size)))

    def expert_phase(self, phase: int, hidden_states: Optional[torch.Tensor], num_tokens: int) -> None:
        """One K3 launch after ``route``: phase 0 gate_up + SwiGLU, phase 1 down."""
        xp = None
        if phase == 0:
            xp = self._check_input(hidden_states, self.hidden_size, "hidden_states").data_ptr()
        ws = self.workspace(num_tokens)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_experts_phase(self.handle, phase, xp, num_tokens, ws.data_ptr(),
                                                          ws.numel(), self._stream(), self.err.buf,
                                                          self.err.size), "nkt_moe_experts_phase")

    def expert_phase_timed(self, phase: int, hidden_states: Optional[torch.Tensor], num_tokens: int,
                           start: "torch.cuda.Event", stop: "torch.cuda.Event") -> None:
        """``expert_phase`` with its expert-GEMM kernel stamped by ``start``/``stop``
        (events created with enable_timing=True) at the kernel's own start and end."""
        xp = None
        if phase == 0:
            xp = self._check_input(hidden_states, self.hidden_size, "hidden_states").data_ptr()
        ws = self.workspace(num_tokens)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_experts_phase_timed(
                self.handle, phase, xp, num_tokens, ws.data_ptr(), ws.numel(), self._stream(),
                ctypes.c_void_p(start.cuda_event), ctypes.c_void_p(stop.cuda_event),
                self.err.buf, self.err.size), "nkt_moe_experts_phase_timed")

    def shared(self, hidden_states: torch.Tensor):
        """K4 + K3 on the shared expert: returns (gate fp32 [T], y_shared fp32 [T, H])."""
        x = self._check_input(hidden_states, self.hidden_size, "hidden_states")
        T = x.shape[0]
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_shared(self.handle, x.data_ptr(), T, ws.data_ptr(), ws.numel(),
                                                   self._stream(), self.err.buf, self.err.size), "nkt_moe_shared")
        return (self.region(T, N.WS_SHARED_GATE, torch.float32, (T,)),
                self.region(T, N.WS_SHARED_Y, torch.float32, (T, self.hidden_size)))

    def combine(self, num_tokens: int, out: Optional[torch.Tensor] = None,
                extra: Optional[torch.Tensor] = None) -> torch.Tensor:
        """K5 after ``route``/``experts`` (and ``shared`` when the layer has one).
        extra [T, H] (act dtype): an offload backend's sum for the non-resident
        experts, added inside the same fixed-order fp32 sum."""
        T = num_tokens
        if out is None:
            out = torch.empty(T, self.hidden_size, dtype=self.act_dtype, device=self.device)
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            if extra is None:
                self.err.check(self.lib.nkt_moe_combine(self.handle, T, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                                        self._stream(), self.err.buf, self.err.size),
                               "nkt_moe_combine")
            else:
                e = self._check_input(extra, self.hidden_size, "extra")
                if e.shape[0] != T:
                    raise ValueError(f"extra has {e.shape[0]} rows, expected {T}")
                self._extra = e  # kept alive until the next call (the kernel reads it asynchronously)
                self.err.check(self.lib.nkt_moe_combine_extra(self.handle, T, e.data_ptr(), out.data_ptr(),
                                                              ws.data_ptr(), ws.numel(), self._stream(),
                                                              self.err.buf, self.err.size), "nkt_moe_combine_extra")
        return out

    def set_residency(self, resident: Optional[torch.Tensor]) -> None:
        """Which experts have their weights in HBM (bool [E]); None = all.  Non-resident
        experts get no GEMM work; their sum comes in through ``combine(extra=...)``."""
        if resident is None:
            self._resident = None
            ptr = None
        else:
            r = torch.as_tensor(resident).reshape(-1)
            if r.numel() != self.num_experts:
                raise ValueError(f"residency mask needs {self.num_experts} entries")
            self._resident = r.to(torch.uint8).to(self.device).contiguous()
            ptr = self._resident.data_ptr()
        self.err.check(self.lib.nkt_moe_bind_residency(self.handle, ptr, self.err.buf, self.err.size),
                       "nkt_moe_bind_residency")

    def forward_hidden(self, hidden_states: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The whole layer from hidden states (router GEMV fused; after ``load_router``)."""
        x = self._check_input(hidden_states, self.hidden_size, "hidden_states")
        T = x.shape[0]
        if out is None:
            out = torch.empty(T, self.hidden_size, dtype=self.act_dtype, device=self.device)
        if T == 0:
            return out
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_forward_hidden(self.handle, x.data_ptr(), T, out.data_ptr(),
                                                           ws.data_ptr(), ws.numel(), self._stream(),
                                                           self.err.buf, self.err.size), "nkt_moe_forward_hidden")
        return out

    def forward_block(self, hidden_states: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The decoder layer's MoE half: hidden + MoE(RMSNorm(hidden)) with the fused
        router (after ``load_router``); the RMSNorm output stays in NKT_WS_NORMED."""
        x = self._check_input(hidden_states, self.hidden_size, "hidden_states")
        T = x.shape[0]
        w = norm_weight.to(self.act_dtype).to(self.device).reshape(-1).contiguous()
        if w.numel() != self.hidden_size:
            raise ValueError(f"norm weight must have {self.hidden_size} entries")
        if out is None:
            out = torch.empty(T, self.hidden_size, dtype=self.act_dtype, device=self.device)
        if T == 0:
            return out
        self._norm_w = w  # kept alive while the kernels run
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_forward_block(self.handle, x.data_ptr(), w.data_ptr(), float(eps), T,
                                                          out.data_ptr(), ws.data_ptr(), ws.numel(), self._stream(),
                                                          self.err.buf, self.err.size), "nkt_moe_forward_block")
        return out

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The whole layer; returns [T, H] in the activation dtype."""
        x = self._check_input(hidden_states, self.hidden_size, "hidden_states")
        logits = self._check_input(router_logits, self.num_experts, "router_logits")
        T = x.shape[0]
        if logits.shape[0] != T:
            raise ValueError(f"router_logits has {logits.shape[0]} rows, hidden_states {T}")
        if out is None:
            out = torch.empty(T, self.hidden_size, dtype=self.act_dtype, device=self.device)
        if T == 0:
            return out
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_forward(self.handle, x.data_ptr(), logits.data_ptr(), T, out.data_ptr(),
                                                    ws.data_ptr(), ws.numel(), self._stream(),
                                                    self.err.buf, self.err.size), "nkt_moe_forward")
        return out

    def forward_noalloc(self, hidden_states: torch.Tensor, router_logits: torch.Tensor,
                        out: torch.Tensor) -> torch.Tensor:
        """``forward`` through nkt_moe_forward_noalloc: the library's static
        per-GPU scratch replaces the workspace, so the call allocates nothing
        (``out`` is the caller's).  Calls that overlap on one GPU race."""
        x = self._check_input(hidden_states, self.hidden_size, "hidden_states")
        logits = self._check_input(router_logits, self.num_experts, "router_logits")
        T = x.shape[0]
        if logits.shape[0] != T:
            raise ValueError(f"router_logits has {logits.shape[0]} rows, hidden_states {T}")
        if out.dtype != self.act_dtype or tuple(out.shape) != (T, self.hidden_size) or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous [{T}, {self.hidden_size}] {self.act_dtype} tensor")
        with torch.cuda.device(self.device):
            self.err.check(self.lib.nkt_moe_forward_noalloc(self.handle, x.data_ptr(), logits.data_ptr(), T,
                                                            out.data_ptr(), self._stream(), self.err.buf,
                                                            self.err.size), "nkt_moe_forward_noalloc")
        return out
