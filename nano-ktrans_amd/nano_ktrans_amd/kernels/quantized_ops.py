"""Weight-only symmetric quantizers in the GPTQLinearWeight convention.

``quantize_symmetric_w4a32`` restates nano_ktrans/kernels/quantized_ops.py:17-59
with torch ops on any device: per output row and per group of ``group_size``
inputs, ``scale = max(|w|).clamp(1e-6) / 7``,
``q = round_half_even(w / scale).clamp(-8, 7)``, stored ``q + 8``, packed eight
nibbles per int32 word with input column 8w+j at bits [4j, 4j+4)
(pack_int4_matrix, quantized_ops.py:62-72).

``quantize_symmetric_int8_per_channel`` is the same algorithm at 8 bits with
one group per row (scale = max|w| / 127, clamp [-128, 127], stored q + 128,
four bytes per word, column 4w+j at bits [8j, 8j+8)).  The reference rejects
bits != 4 in its quantizer (quantized_ops.py:24-25) but its grouped matvec
(quantized_ops.py:86-124) consumes this layout unchanged.

These run once at weight ingest; the device format is produced from their
output by ``nkt_moe_pack_weight``.
"""
from __future__ import annotations

import torch

from .weight_loader import GPTQLinearWeight


def _pack_words(qvalues: torch.Tensor, bits: int) -> torch.Tensor:
    n, k = qvalues.shape
    per = 32 // bits
    if k % per != 0:
        raise ValueError(f"input_dim must be divisible by {per} for {bits}-bit packing.")
    v = qvalues.to(torch.int64).reshape(n, k // per, per)
    shifts = (torch.arange(per, dtype=torch.int64, device=qvalues.device) * bits).view(1, 1, per)
    words = (v << shifts).sum(dim=2)
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32).contiguous()


def pack_int4_matrix(qvalues: torch.Tensor) -> torch.Tensor:
    """uint8 codes [out, in] (0..15) -> int32 words [out, in/8]."""
    if qvalues.ndim != 2:
        raise ValueError(f"Expected 2D qvalues, got shape={tuple(qvalues.shape)}")
    return _pack_words(qvalues, 4)


def pack_int8_matrix(qvalues: torch.Tensor) -> torch.Tensor:
    """uint8 codes [out, in] (0..255) -> int32 words [out, in/4]."""
    if qvalues.ndim != 2:
        raise ValueError(f"Expected 2D qvalues, got shape={tuple(qvalues.shape)}")
    return _pack_words(qvalues, 8)


def quantize_symmetric_w4a32(
    weight: torch.Tensor,
    *,
    group_size: int = 128,
    bits: int = 4,
    linear_prefix: str = "synthetic",
) -> GPTQLinearWeight:
    if bits != 4:
        raise NotImplementedError("Only 4-bit symmetric group quantization is supported here.")
    w = weight.to(dtype=torch.float32).contiguous()
    out_dim, in_dim = w.shape
    if in_dim % group_size != 0:
        raise ValueError("input_dim must be divisible by group_size.")
    groups = in_dim // group_size
    chunks = w.reshape(out_dim, groups, group_size)
    max_abs = chunks.abs().amax(dim=2).clamp(min=1e-6)
    scale = max_abs / 7
    q = torch.round(chunks / scale.unsqueeze(2)).clamp(-8, 7)
    qvalues = (q + 8.0).to(torch.uint8).reshape(out_dim, in_dim)
    return GPTQLinearWeight(
        qweight=pack_int4_matrix(qvalues),
        scales=scale.contiguous(),
        zero_points=None,
        group_size=group_size,
        bits=4,
        sym=True,
        linear_prefix=linear_prefix,
    )


def quantize_symmetric_int8_per_channel(
    weight: torch.Tensor,
    *,
    linear_prefix: str = "synthetic",
) -> GPTQLinearWeight:
    w = weight.to(dtype=torch.float32).contiguous()
    out_dim, in_dim = w.shape
    max_abs = w.abs().amax(dim=1).clamp(min=1e-6)
    scale = max_abs / 127
    q = torch.round(w / scale.unsqueeze(1)).clamp(-128, 127)
    qvalues = (q + 128.0).to(torch.uint8)
    return GPTQLinearWeight(
        qweight=pack_int8_matrix(qvalues),
        scales=scale.unsqueeze(1).contiguous(),
        zero_points=None,
        group_size=in_dim,
        bits=8,
        sym=True,
        linear_prefix=linear_prefix,
    )


def to_bf16_scales(qw: GPTQLinearWeight) -> GPTQLinearWeight:
    """The same codes with scales rounded to bf16 (the device scale format)."""
    return GPTQLinearWeight(
        qweight=qw.qweight,
        scales=qw.scales.to(torch.bfloat16).to(torch.float32),
        zero_points=qw.zero_points,
        group_size=qw.group_size,
        bits=qw.bits,
        sym=qw.sym,
        linear_prefix=qw.linear_prefix,
    )
