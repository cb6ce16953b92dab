"""CPU oracle for the MoE expert path.  TEST INFRASTRUCTURE ONLY.

This module is the checker that the HIP kernels are compared against.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product package never does.

Numpy float32 restatement of the reference's CPU expert loop, plus ctypes
bindings for the routing/grouping restatement in ``nkt_oracle.c``.  Each
function cites the reference code it follows (paths relative to the
nano-ktrans tree):

* ``quantize_int4``           nano_ktrans/kernels/quantized_ops.py:17-59 (+ pack 62-72)
* ``quantize_int8_pc``        same algorithm at 8 bits with one group per row (an
                              extension: the reference rejects bits != 4 at :24-25,
                              its matvec at :86-124 is bit-width generic)
* ``unpack_words``            nano_ktrans/kernels/quantized_ops.py:75-83,
                              nano_ktrans/kernels/weight_loader.py:51-55
* ``dequantize``              nano_ktrans/kernels/weight_loader.py:57-69
* ``matvec_grouped``          nano_ktrans/kernels/quantized_ops.py:86-124
* ``expert_dense``            nano_ktrans/layers/expert_mlp.py:20-23, 37-41
* ``expert_quant``            nano_ktrans/kernels/cpu_moe.py:419-450
* ``router_logits``           nano_ktrans/models/mixtral.py:127, 212 (the gate
                              nn.Linear(H, E, bias=False) in bf16: exact dot
                              products rounded once to bf16)
* ``rms_norm``                nano_ktrans/layers/norm.py:11-17 (the post-attention
                              RMSNorm of the decoder-block form)
* ``route``                   nano_ktrans/layers/hybrid_moe.py:3321-3329 (C restatement)
* ``group``                   nano_ktrans/layers/hybrid_moe.py:3512-3526,
                              nano_ktrans/kernels/cpu_moe.py:515-523 (C restatement)
* ``moe_forward``             nano_ktrans/kernels/cpu_moe.py:491-539 (quantized
                              experts, fp32 accumulation, one cast at the end) and
                              nano_ktrans/layers/hybrid_moe.py:3501-3533, 3570 (dense);
                              shared expert nano_ktrans/models/mixtral.py:215-218

Parity pins for every function are in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libnkt_oracle.so")
_lib = None


def lib() -> ctypes.CDLL:
    """Load the C half of the oracle (built by ``oracle/Makefile``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle C library missing: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        ip = ctypes.POINTER(ctypes.c_int32)
        L.orc_expf.argtypes = [ctypes.c_float]
        L.orc_expf.restype = ctypes.c_float
        L.orc_bf16_round.argtypes = [ctypes.c_float]
        L.orc_bf16_round.restype = ctypes.c_float
        L.orc_expf_array.argtypes = [fp, fp, ctypes.c_int64]
        L.orc_expf_array.restype = None
        L.orc_softmax_row.argtypes = [fp, ctypes.c_int, fp]
        L.orc_softmax_row.restype = None
        L.orc_route.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.c_int, ctypes.c_int, ip, fp]
        L.orc_route.restype = ctypes.c_int
        L.orc_group.argtypes = [ip, ctypes.c_int, ctypes.c_int, ctypes.c_int, ip, ip, ip, ip]
        L.orc_group.restype = ctypes.c_int
        _lib = L
    return _lib


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _iptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


# ---------------------------------------------------------------------------
# bf16
# ---------------------------------------------------------------------------
def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), kept as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    r = np.where(nan, (u | 0x00400000) & 0xFFFF0000, r)
    return r.astype(np.uint32).view(np.float32).reshape(x.shape)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """uint16 bit patterns of bf16-valued float32 input."""
    return (np.ascontiguousarray(bf16_round(x)).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# exp / softmax / routing / grouping (C restatement)
# ---------------------------------------------------------------------------
def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.empty_like(x)
    lib().orc_expf_array(_fptr(x), _fptr(y), x.size)
    return y


def softmax_row(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    p = np.empty_like(x)
    lib().orc_softmax_row(_fptr(x), x.size, _fptr(p))
    return p


def router_logits(x: np.ndarray, gate: np.ndarray) -> np.ndarray:
    """router_logits = gate(x) for bf16 x [T, H] and gate weight [E, H]
    (nano_ktrans/models/mixtral.py:127, 212, nn.Linear(H, E, bias=False) in
    bf16): dot products accumulated in float64 (rounding errors far below
    bf16 resolution), then rounded once to bf16 (ties to even); float32 out."""
    acc = np.asarray(x, dtype=np.float64) @ np.asarray(gate, dtype=np.float64).T
    return round64_to_bf16(acc)


def round64_to_bf16(a: np.ndarray) -> np.ndarray:
    """float64 -> nearest bf16 (ties to even) in a single rounding, as float32:
    round to float32 with round-to-odd (truncate, set the last bit when
    inexact), then to bf16 with ties-to-even -- float32 carries more than two
    extra bits, so the two steps equal one correct rounding."""
    a = np.asarray(a, dtype=np.float64)
    f = a.astype(np.float32)
    f64 = f.astype(np.float64)
    exact = f64 == a
    toward_zero = np.where(np.abs(f64) > np.abs(a), np.nextafter(f, np.float32(0)), f).astype(np.float32)
    odd = (toward_zero.view(np.uint32) | np.uint32(1)).view(np.float32)
    return bf16_round(np.where(exact, f, odd).astype(np.float32))


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """RMSNorm of bf16 rows x [T, H] with bf16 weight [H]
    (nano_ktrans/layers/norm.py:11-17): t = x * rsqrt(mean(x^2) + eps) cast to
    bf16, then t * weight cast to bf16.  The mean and the scaling in float64,
    each bf16 cast one rounding; float32 out."""
    x64 = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    t = round64_to_bf16(x64 * inv)
    return round64_to_bf16(t.astype(np.float64) * np.asarray(weight, dtype=np.float64))


def route(logits: np.ndarray, top_k: int, use_softmax: bool, renorm: bool, bf16: bool):
    """Top-k routing of ``logits`` [T, E].  Returns (ids int32 [T,k], weights fp32 [T,k])."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    ids = np.zeros((T, top_k), dtype=np.int32)
    w = np.zeros((T, top_k), dtype=np.float32)
    rc = lib().orc_route(_fptr(logits), T, E, top_k, int(use_softmax), int(renorm), int(bf16),
                         _iptr(ids), _fptr(w))
    if rc != 0:
        raise ValueError("orc_route rejected its arguments")
    return ids, w


def group(ids: np.ndarray, num_experts: int):
    """Counting sort of the (token, slot) pairs by expert, stable in token order.

    Returns counts [E], offsets [E+1], perm [T*k], inv [T*k] (int32)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, k = ids.shape
    counts = np.zeros(num_experts, dtype=np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    perm = np.zeros(T * k, dtype=np.int32)
    inv = np.zeros(T * k, dtype=np.int32)
    rc = lib().orc_group(_iptr(ids), T, k, num_experts, _iptr(counts), _iptr(offsets),
                         _iptr(perm), _iptr(inv))
    if rc != 0:
        raise ValueError("orc_group: expert id out of range")
    return counts, offsets, perm, inv


# ---------------------------------------------------------------------------
# weight-only quantization in the GPTQLinearWeight convention
# ---------------------------------------------------------------------------
@dataclass
class QWeight:
    """qweight int32 [out, in*bits/32] (value j of word w is input column
    (32/bits)*w + j, stored as q + 2^(bits-1)); scales fp32 [out, groups]."""
    qweight: np.ndarray
    scales: np.ndarray
    bits: int
    group_size: int

    @property
    def out_dim(self) -> int:
        return self.qweight.shape[0]

    @property
    def in_dim(self) -> int:
        return self.qweight.shape[1] * (32 // self.bits)


def _pack_words(qvalues: np.ndarray, bits: int) -> np.ndarray:
    n, k = qvalues.shape
    per = 32 // bits
    v = qvalues.astype(np.uint64).reshape(n, k // per, per)
    shifts = (np.arange(per, dtype=np.uint64) * bits).reshape(1, 1, per)
    words = np.bitwise_or.reduce(v << shifts, axis=2)
    return (words & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def quantize_int4(w: np.ndarray, group_size: int = 128) -> QWeight:
    """Symmetric int4, one fp32 scale per (row, group): scale = max|w|/7 (|w| >= 1e-6),
    q = round_half_even(w / scale) clamped to [-8, 7], stored q + 8."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    if k % group_size != 0:
        raise ValueError("in_dim must be a multiple of group_size")
    groups = k // group_size
    q = np.empty((n, k), dtype=np.uint8)
    scales = np.empty((n, groups), dtype=np.float32)
    for g in range(groups):
        chunk = w[:, g * group_size:(g + 1) * group_size]
        max_abs = np.maximum(np.abs(chunk).max(axis=1), np.float32(1e-6)).astype(np.float32)
        scale = (max_abs / np.float32(7.0)).astype(np.float32)
        qq = np.clip(np.rint(chunk / scale[:, None]), -8, 7)
        q[:, g * group_size:(g + 1) * group_size] = (qq + np.float32(8.0)).astype(np.uint8)
        scales[:, g] = scale
    return QWeight(_pack_words(q, 4), scales, 4, group_size)


def quantize_int8_pc(w: np.ndarray) -> QWeight:
    """Symmetric int8, one fp32 scale per output row: scale = max|w|/127,
    q = round_half_even(w / scale) clamped to [-128, 127], stored q + 128."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    max_abs = np.maximum(np.abs(w).max(axis=1), np.float32(1e-6)).astype(np.float32)
    scale = (max_abs / np.float32(127.0)).astype(np.float32)
    qq = np.clip(np.rint(w / scale[:, None]), -128, 127)
    q = (qq + np.float32(128.0)).astype(np.uint8)
    return QWeight(_pack_words(q, 8), scale[:, None].copy(), 8, k)


def with_bf16_scales(qw: QWeight) -> QWeight:
    """The same codes with scales rounded to bf16 (the device format)."""
    return QWeight(qw.qweight, bf16_round(qw.scales), qw.bits, qw.group_size)


def unpack_words(qweight: np.ndarray, bits: int) -> np.ndarray:
    per = 32 // bits
    u = np.ascontiguousarray(qweight).view(np.uint32)
    shifts = (np.arange(per, dtype=np.uint32) * bits).reshape(1, 1, per)
    vals = (u[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return vals.reshape(qweight.shape[0], qweight.shape[1] * per).astype(np.float32)


def dequantize(qw: QWeight) -> np.ndarray:
    q = unpack_words(qw.qweight, qw.bits)
    zero = np.float32(1 << (qw.bits - 1))
    out = np.empty_like(q)
    for g in range(qw.scales.shape[1]):
        s, e = g * qw.group_size, min((g + 1) * qw.group_size, qw.in_dim)
        out[:, s:e] = (q[:, s:e] - zero) * qw.scales[:, g:g + 1]
    return out


def matvec_grouped(x: np.ndarray, qw: QWeight) -> np.ndarray:
    """fp32 x [n, in] times the quantized weight, summed group by group in ascending order."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros((x.shape[0], qw.out_dim), dtype=np.float32)
    q = unpack_words(qw.qweight, qw.bits)
    zero = np.float32(1 << (qw.bits - 1))
    for g in range(qw.scales.shape[1]):
        s, e = g * qw.group_size, min((g + 1) * qw.group_size, qw.in_dim)
        wg = (q[:, s:e] - zero) * qw.scales[:, g:g + 1]
        out += x[:, s:e] @ wg.T
    return out


# ---------------------------------------------------------------------------
# experts and the MoE layer
# ---------------------------------------------------------------------------
def silu(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float32)
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


@dataclass
class Expert:
    """One SwiGLU expert: gate/up [I, H], down [H, I]; dense fp32 arrays or QWeight."""
    gate: object
    up: object
    down: object


def _lin(x: np.ndarray, w) -> np.ndarray:
    if isinstance(w, QWeight):
        return matvec_grouped(x, w)
    return x.astype(np.float32) @ np.asarray(w, dtype=np.float32).T


def expert_forward(x: np.ndarray, ex: Expert, h_bf16: bool = False) -> np.ndarray:
    """down(silu(gate(x)) * up(x)) in fp32.  h_bf16: the SwiGLU output h is
    rounded to bf16 before the down projection, as a bf16 module stores it
    (nano_ktrans/layers/expert_mlp.py:20-23 in bf16: act_fn(w1 x) * w3 x is a
    bf16 tensor)."""
    g = _lin(x, ex.gate)
    u = _lin(x, ex.up)
    h = silu(g) * u
    if h_bf16:
        h = bf16_round(h)
    return _lin(h, ex.down)


def moe_forward(x: np.ndarray, logits: np.ndarray, experts: List[Expert], top_k: int,
                use_softmax: bool, renorm: bool, bf16: bool,
                shared: Optional[Expert] = None, shared_gate: Optional[np.ndarray] = None,
                return_parts: bool = False, h_bf16: bool = False):
    """MoE layer output in fp32 before the final cast (cast with ``bf16_round`` for bf16).

    x [T, H] and logits [T, E] hold the activation-dtype values as float32.
    h_bf16: every expert's SwiGLU output rounded to bf16 (``expert_forward``)."""
    ids, w = route(logits, top_k, use_softmax, renorm, bf16)
    return moe_forward_given(x, ids, w, experts, shared, shared_gate, return_parts, h_bf16)


def moe_forward_given(x: np.ndarray, ids: np.ndarray, w: np.ndarray, experts: List[Expert],
                      shared: Optional[Expert] = None, shared_gate: Optional[np.ndarray] = None,
                      return_parts: bool = False, h_bf16: bool = False):
    """The expert loop on routing the caller computed: ids [T, k] (distinct
    ids in [0, E) per token, any slot order) and weights w [T, k] (fp32),
    as the offload backend's loop takes them (nano_ktrans/kernels/cpu_moe.py:
    491-539: for each expert in ascending id, the tokens that picked it in
    ascending order, y * w accumulated in fp32).  Same outputs as
    ``moe_forward``."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    T, H = x.shape
    top_k = ids.shape[1]
    E = len(experts)
    counts, offsets, perm, inv = group(ids, E)
    out = np.zeros((T, H), dtype=np.float32)
    y_pairs = np.zeros((T * top_k, H), dtype=np.float32)
    for e in range(E):
        if counts[e] == 0:
            continue
        pairs = perm[offsets[e]:offsets[e + 1]]
        toks = pairs // top_k
        y = expert_forward(x[toks], experts[e], h_bf16)
        y_pairs[pairs] = y
        out[toks] += y * w.reshape(-1)[pairs][:, None]
    gate_vals = None
    y_shared = None
    if shared is not None:
        gl = x @ np.asarray(shared_gate, dtype=np.float32).reshape(-1)
        gate_vals = (np.float32(1.0) / (np.float32(1.0) + np.exp(-gl.astype(np.float32)))).astype(np.float32)
        y_shared = expert_forward(x, shared, h_bf16)
        out += gate_vals[:, None] * y_shared
    if return_parts:
        return out, dict(ids=ids, weights=w, counts=counts, offsets=offsets, perm=perm, inv=inv,
                         y_pairs=y_pairs, shared_gate=gate_vals, y_shared=y_shared)
    return out


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
