"""The reference's expert offload contract, served from HBM by the HIP path.

``ExpertOffloadBackend`` restates the contract of
nano_ktrans/kernels/offload_backend.py:29-60 (the part HybridMoE calls:
``submit_forward`` / ``sync_forward`` / ``update_gpu_expert_mask``).  The
reference's backends (CPU via kt-kernel, PIM) run the experts whose
``gpu_experts_mask`` entry is False and return the routing-weighted sum of
their outputs, which HybridMoE adds to its own
(nano_ktrans/layers/hybrid_moe.py:3373-3378, 3563-3570).

``HbmExpertBackend`` is that backend on the GPU: its experts sit in HBM in the
library's packed layout and one ``nkt_moe_forward_routed`` launch sequence
computes the sum from the caller's ``topk_ids`` / ``topk_weights`` on the
caller's stream -- the C-ABI counterpart of kt-kernel's
``forward_task(bsz, k, expert_ids, weights, input, output)`` submitted with
``submit_with_cuda_stream`` (nano_ktrans/kernels/cpu_moe.py:570-592).  So the
reference's unchanged HybridMoE can hand its offloaded experts to the GPU
path, and expert compute can run on routing computed elsewhere.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Optional

import torch

from ..native_moe import NativeMoE


class ExpertOffloadBackend(ABC):
    """submit_forward enqueues the offloaded experts' work for one layer call;
    sync_forward returns its [T, H] sum (offloaded experts only)."""

    backend_name = "unknown"

    def __init__(self) -> None:
        self.submit_calls = 0
        self.sync_calls = 0

    @abstractmethod
    def submit_forward(self, hidden_states: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                       cuda_stream: Optional[int]) -> None:
        raise NotImplementedError

    @abstractmethod
    def sync_forward(self, hidden_states: torch.Tensor, cuda_stream: Optional[int]) -> torch.Tensor:
        raise NotImplementedError

    def update_gpu_expert_mask(self, gpu_experts_mask: torch.Tensor) -> None:
        raise NotImplementedError

    def diagnostics(self) -> dict:
        return {"backend_name": self.backend_name, "submit_calls": self.submit_calls,
                "sync_calls": self.sync_calls}


def _stream_of(cuda_stream: Optional[int], device: torch.device) -> torch.cuda.Stream:
    if cuda_stream is None:
        return torch.cuda.current_stream(device)
    return torch.cuda.ExternalStream(int(cuda_stream), device=device)


class HbmExpertBackend(ExpertOffloadBackend):
    """The experts a HybridMoE offloads (``gpu_experts_mask`` False), computed
    by the HIP path from the caller's routing.

    ``native`` holds the layer's experts (at least those this backend serves);
    the backend marks the experts with mask True non-resident in it, so they
    add nothing and get no GEMM work.  ``submit_forward`` enqueues the whole
    computation on ``cuda_stream`` (the caller's stream when None) and returns
    at once; ``sync_forward`` makes the stream it is given wait for that work
    and returns the sum in the activation dtype.  One submit / sync pair is in
    flight at a time, as in the reference."""

    backend_name = "hbm"

    def __init__(self, native: NativeMoE, gpu_experts_mask: torch.Tensor):
        super().__init__()
        if native.shared_intermediate_size:
            raise ValueError("an offload backend serves routed experts only; build its layer without a shared expert")
        self.native = native
        self._out: Optional[torch.Tensor] = None
        self._done: Optional[torch.cuda.Event] = None
        self._stream: Optional[torch.cuda.Stream] = None
        self.update_gpu_expert_mask(gpu_experts_mask)

    def update_gpu_expert_mask(self, gpu_experts_mask: torch.Tensor) -> None:
        mask = torch.as_tensor(gpu_experts_mask).reshape(-1).to(torch.bool).cpu()
        if mask.numel() != self.native.num_experts:
            raise ValueError(f"gpu_experts_mask needs {self.native.num_experts} entries, got {mask.numel()}")
        self.gpu_experts_mask = mask
        self.native.set_residency(~mask)

    def submit_forward(self, hidden_states: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                       cuda_stream: Optional[int]) -> None:
        self.submit_calls += 1
        flat = hidden_states.reshape(-1, hidden_states.shape[-1])
        stream = _stream_of(cuda_stream, flat.device)
        with torch.cuda.stream(stream):
            self._out = self.native.forward_routed(flat, topk_ids.reshape(flat.shape[0], -1),
                                                   topk_weights.reshape(flat.shape[0], -1))
            self._done = torch.cuda.Event()
            self._done.record(stream)
        self._stream = stream

    def sync_forward(self, hidden_states: torch.Tensor, cuda_stream: Optional[int]) -> torch.Tensor:
        self.sync_calls += 1
        if self._out is None:
            return torch.zeros_like(hidden_states.reshape(-1, hidden_states.shape[-1]))
        consumer = _stream_of(cuda_stream, self._out.device)
        consumer.wait_event(self._done)
        out, self._out = self._out, None
        if consumer != self._stream:
            out.record_stream(consumer)  # made on the submit stream, read on this one
        return out
