"""ctypes binding of the gfx950 MoE library (C ABI: include/nkt_moe.h).

The binding style (explicit argtypes/restype, handle + error buffer + int
return code) follows the reference's native bridge binding in
nano_ktrans/kernels/pim_quantized_runtime.py:72-209.

There is no fallback: if the shared library is missing or no GPU is visible,
every entry point raises ``NativeError``.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnkt_moe.so")

NKT_OK = 0

WEIGHT_F32 = 0
WEIGHT_BF16 = 1
WEIGHT_INT8_PC = 2
WEIGHT_INT4_G128 = 3

DTYPE_F32 = 0
DTYPE_BF16 = 1

ROUTE_SOFTMAX = 1
ROUTE_RENORM = 2

SLOT_GATE_UP = 0
SLOT_GATE_UP_SCALES = 1
SLOT_DOWN = 2
SLOT_DOWN_SCALES = 3
SLOT_SHARED_GATE_UP = 4
SLOT_SHARED_GATE_UP_SCALES = 5
SLOT_SHARED_DOWN = 6
SLOT_SHARED_DOWN_SCALES = 7
SLOT_SHARED_GATE = 8
SLOT_ROUTER = 9
NUM_SLOTS = 10

WS_TOPK_IDS = 0
WS_TOPK_WEIGHTS = 1
WS_COUNTS = 2
WS_OFFSETS = 3
WS_PERM = 4
WS_INV = 5
WS_H = 6
WS_Y = 7
WS_SHARED_GATE = 8
WS_SHARED_H = 9
WS_SHARED_Y = 10
WS_ROUTER_LOGITS = 11
WS_NORMED = 12
WS_SYNC = 13

# status word inside WS_SYNC (uint32 index): 1 after a given-routing call dropped a slot,
# cleared by the caller
STATUS_BAD_ROUTING = 30

# leading bytes of every workspace that must start at zero (every call leaves
# them zero, the status word aside when a call reports a fault)
SYNC_AREA_BYTES = 65792

EXPORTED_SYMBOLS = (
    "nkt_moe_create",
    "nkt_moe_destroy",
    "nkt_moe_weight_bytes",
    "nkt_moe_pack_weight",
    "nkt_moe_bind_weights",
    "nkt_moe_workspace_bytes",
    "nkt_moe_workspace_region",
    "nkt_moe_route",
    "nkt_moe_route_given",
    "nkt_moe_experts",
    "nkt_moe_experts_phase",
    "nkt_moe_experts_phase_timed",
    "nkt_moe_shared",
    "nkt_moe_combine",
    "nkt_moe_combine_extra",
    "nkt_moe_bind_residency",
    "nkt_moe_forward",
    "nkt_moe_forward_routed",
    "nkt_moe_route_hidden",
    "nkt_moe_forward_hidden",
    "nkt_moe_forward_block",
    "nkt_moe_forward_noalloc",
    "nkt_moe_version",
)

# bytes of the static scratch behind nkt_moe_forward_noalloc (NKT_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 64 << 20


class NativeError(RuntimeError):
    """Raised when the native library is unavailable or a call fails."""


_lib = None


def lib() -> ctypes.CDLL:
    """Load libnkt_moe.so and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NativeError(
            f"native MoE library not built: {LIB_PATH} is missing "
            "(build with `make -C nano-ktrans_amd/csrc` or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, cp, i, u = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_int, ctypes.c_uint
    szp = ctypes.POINTER(ctypes.c_size_t)
    L.nkt_moe_create.argtypes = [i, i, i, i, i, i, i, u, i, cp, sz]
    L.nkt_moe_create.restype = vp
    L.nkt_moe_destroy.argtypes = [vp]
    L.nkt_moe_destroy.restype = None
    L.nkt_moe_weight_bytes.argtypes = [vp, i, szp, cp, sz]
    L.nkt_moe_weight_bytes.restype = i
    L.nkt_moe_pack_weight.argtypes = [vp, i, i, vp, vp, vp, vp, vp, cp, sz]
    L.nkt_moe_pack_weight.restype = i
    L.nkt_moe_bind_weights.argtypes = [vp, ctypes.POINTER(vp), cp, sz]
    L.nkt_moe_bind_weights.restype = i
    L.nkt_moe_workspace_bytes.argtypes = [vp, i, szp, cp, sz]
    L.nkt_moe_workspace_bytes.restype = i
    L.nkt_moe_workspace_region.argtypes = [vp, i, i, szp, cp, sz]
    L.nkt_moe_workspace_region.restype = i
    L.nkt_moe_route.argtypes = [vp, vp, i, vp, sz, vp, cp, sz]
    L.nkt_moe_route.restype = i
    L.nkt_moe_route_given.argtypes = [vp, vp, vp, i, vp, sz, vp, cp, sz]
    L.nkt_moe_route_given.restype = i
    L.nkt_moe_experts.argtypes = [vp, vp, i, vp, sz, vp, cp, sz]
    L.nkt_moe_experts.restype = i
    L.nkt_moe_experts_phase.argtypes = [vp, i, vp, i, vp, sz, vp, cp, sz]
    L.nkt_moe_experts_phase.restype = i
    L.nkt_moe_experts_phase_timed.argtypes = [vp, i, vp, i, vp, sz, vp, vp, vp, cp, sz]
    L.nkt_moe_experts_phase_timed.restype = i
    L.nkt_moe_shared.argtypes = [vp, vp, i, vp, sz, vp, cp, sz]
    L.nkt_moe_shared.restype = i
    L.nkt_moe_combine.argtypes = [vp, i, vp, vp, sz, vp, cp, sz]
    L.nkt_moe_combine.restype = i
    L.nkt_moe_forward.argtypes = [vp, vp, vp, i, vp, vp, sz, vp, cp, sz]
    L.nkt_moe_forward.restype = i
    L.nkt_moe_forward_routed.argtypes = [vp, vp, vp, vp, i, vp, vp, sz, vp, cp, sz]
    L.nkt_moe_forward_routed.restype = i
    L.nkt_moe_combine_extra.argtypes = [vp, i, vp, vp, vp, sz, vp, cp, sz]
    L.nkt_moe_combine_extra.restype = i
    L.nkt_moe_bind_residency.argtypes = [vp, vp, cp, sz]
    L.nkt_moe_bind_residency.restype = i
    L.nkt_moe_route_hidden.argtypes = [vp, vp, i, vp, sz, vp, cp, sz]
    L.nkt_moe_route_hidden.restype = i
    L.nkt_moe_forward_hidden.argtypes = [vp, vp, i, vp, vp, sz, vp, cp, sz]
    L.nkt_moe_forward_hidden.restype = i
    L.nkt_moe_forward_block.argtypes = [vp, vp, vp, ctypes.c_float, i, vp, vp, sz, vp, cp, sz]
    L.nkt_moe_forward_block.restype = i
    L.nkt_moe_forward_noalloc.argtypes = [vp, vp, vp, i, vp, vp, cp, sz]
    L.nkt_moe_forward_noalloc.restype = i
    L.nkt_moe_version.argtypes = []
    L.nkt_moe_version.restype = ctypes.c_char_p
    _lib = L
    return L


class ErrBuf:
    """A reusable error-message buffer for the C ABI."""

    def __init__(self, size: int = 512):
        self.buf = ctypes.create_string_buffer(size)
        self.size = size

    def check(self, rc: int, what: str) -> None:
        if rc != NKT_OK:
            raise NativeError(f"{what} failed: {self.buf.value.decode(errors='replace')}")
