"""MI355X (gfx950) MoE expert path for nano-ktrans.

The HybridMoE routing, token grouping, SwiGLU expert compute over quantized
experts, shared-expert gate and combine run as hand-written HIP kernels
behind the C ABI in include/nkt_moe.h (libnkt_moe.so, loaded with ctypes).
"""
from .kernels.quantized_ops import (
    pack_int4_matrix,
    pack_int8_matrix,
    quantize_symmetric_int8_per_channel,
    quantize_symmetric_w4a32,
)
from .kernels.weight_loader import ExpertWeightLoader, GPTQLinearWeight
from .layers.expert_mlp import PackedSparseExpertMLP, SparseExpertMLP, build_expert_module, load_expert_weights
from .layers.hybrid_moe import HybridMoE
from .native_moe import NativeMoE

__all__ = [
    "ExpertWeightLoader",
    "GPTQLinearWeight",
    "HybridMoE",
    "NativeMoE",
    "PackedSparseExpertMLP",
    "SparseExpertMLP",
    "build_expert_module",
    "load_expert_weights",
    "pack_int4_matrix",
    "pack_int8_matrix",
    "quantize_symmetric_int8_per_channel",
    "quantize_symmetric_w4a32",
]
