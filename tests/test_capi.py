"""C ABI surface, checked without a GPU: the library loads, exports exactly what
include/nkt_moe.h declares, validates its arguments, and the Python layer refuses
to run anywhere but on the GPU (there is no CPU fallback)."""
import ctypes
import os
import re

import pytest
import torch

from nano_ktrans_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nkt_moe.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(nkt_moe_\w+)\s*\(", text)))


def test_header_declarations_match_binding():
    assert _declared() == sorted(N.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.nkt_moe_version().startswith(b"nkt_moe")


def _create(E=8, k=2, H=256, I=512, Is=0, wf=N.WEIGHT_F32, act=N.DTYPE_F32, flags=3, max_tokens=64):
    lib = N.lib()
    err = ctypes.create_string_buffer(256)
    h = lib.nkt_moe_create(E, k, H, I, Is, wf, act, flags, max_tokens, err, 256)
    return h, err.value.decode()


@pytest.mark.parametrize("kw,msg", [
    (dict(E=0), "num_experts"), (dict(E=300), "num_experts"), (dict(k=0), "top_k"), (dict(k=9, E=8), "top_k"),
    (dict(H=100), "hidden_size"), (dict(I=96), "moe_intermediate_size"), (dict(Is=100), "shared"),
    (dict(wf=7), "weight_format"), (dict(wf=N.WEIGHT_INT4_G128, act=N.DTYPE_F32), "fp32"),
    (dict(wf=N.WEIGHT_F32, act=N.DTYPE_BF16), "fp32"), (dict(max_tokens=0), "max_tokens"),
])
def test_create_rejects_bad_arguments(kw, msg):
    h, err = _create(**kw)
    assert not h
    assert msg in err


def test_weight_and_workspace_sizes():
    lib = N.lib()
    E, k, H, I, Is = 60, 4, 2048, 1408, 5632
    h, err = _create(E, k, H, I, Is, N.WEIGHT_INT8_PC, N.DTYPE_BF16, 1, 4096)
    assert h, err
    eb = ctypes.create_string_buffer(256)
    sz = ctypes.c_size_t()
    expect = {
        N.SLOT_GATE_UP: E * 2 * I * H, N.SLOT_GATE_UP_SCALES: E * 2 * I * 2,
        N.SLOT_DOWN: E * H * I, N.SLOT_DOWN_SCALES: E * H * 2,
        N.SLOT_SHARED_GATE_UP: 2 * Is * H, N.SLOT_SHARED_GATE_UP_SCALES: 2 * Is * 2,
        N.SLOT_SHARED_DOWN: H * Is, N.SLOT_SHARED_DOWN_SCALES: H * 2, N.SLOT_SHARED_GATE: H * 2,
    }
    for slot, nbytes in expect.items():
        assert lib.nkt_moe_weight_bytes(h, slot, ctypes.byref(sz), eb, 256) == 0
        assert sz.value == nbytes, slot
    prev = 0
    for T in (1, 16, 1024, 4096):
        assert lib.nkt_moe_workspace_bytes(h, T, ctypes.byref(sz), eb, 256) == 0
        assert sz.value > prev
        prev = sz.value
        offs = []
        for r in range(11):
            o = ctypes.c_size_t()
            assert lib.nkt_moe_workspace_region(h, T, r, ctypes.byref(o), eb, 256) == 0
            offs.append(o.value)
        assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)
        # the sync area (NKT_WS_SYNC, then the router's tagged words) leads the
        # workspace at a place and size independent of the token count
        o = ctypes.c_size_t()
        assert lib.nkt_moe_workspace_region(h, T, N.WS_SYNC, ctypes.byref(o), eb, 256) == 0
        assert o.value == 0
        assert offs[0] == N.SYNC_AREA_BYTES  # the same sync area for every handle
    assert lib.nkt_moe_workspace_bytes(h, 4097, ctypes.byref(sz), eb, 256) != 0
    lib.nkt_moe_destroy(h)


def test_int4_sizes():
    lib = N.lib()
    E, k, H, I = 128, 8, 2048, 768
    h, err = _create(E, k, H, I, 0, N.WEIGHT_INT4_G128, N.DTYPE_BF16, 3, 16)
    assert h, err
    sz = ctypes.c_size_t()
    eb = ctypes.create_string_buffer(256)
    # per expert: gate_up 1,572,864 B codes + 49,152 B scales; down 786,432 + 24,576
    for slot, nbytes in {N.SLOT_GATE_UP: E * 1572864, N.SLOT_GATE_UP_SCALES: E * 49152,
                         N.SLOT_DOWN: E * 786432, N.SLOT_DOWN_SCALES: E * 24576}.items():
        lib.nkt_moe_weight_bytes(h, slot, ctypes.byref(sz), eb, 256)
        assert sz.value == nbytes
    lib.nkt_moe_destroy(h)


def test_calls_validate_before_touching_the_gpu():
    lib = N.lib()
    h, _ = _create()
    eb = ctypes.create_string_buffer(256)
    # missing workspace and too many tokens are rejected with a message, no launch happens
    assert lib.nkt_moe_forward(h, None, None, 4, None, None, 0, None, eb, 256) == -1
    assert b"workspace" in eb.value
    assert lib.nkt_moe_route(h, None, 65, None, 0, None, eb, 256) == -1
    assert b"max_tokens" in eb.value
    nbytes, off = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.nkt_moe_workspace_bytes(h, 65, ctypes.byref(nbytes), eb, 256) == -1
    assert b"max_tokens=64" in eb.value
    assert lib.nkt_moe_workspace_bytes(h, 64, ctypes.byref(nbytes), eb, 256) == 0 and nbytes.value > 0
    assert lib.nkt_moe_workspace_region(h, 1, N.WS_SYNC + 1, ctypes.byref(off), eb, 256) == -1
    assert b"region" in eb.value
    assert lib.nkt_moe_pack_weight(h, 1, 0, None, None, None, None, None, eb, 256) == -1
    assert lib.nkt_moe_pack_weight(h, 0, 9, None, None, None, None, None, eb, 256) == -1
    assert lib.nkt_moe_shared(h, None, 1, None, 0, None, eb, 256) == -1
    lib.nkt_moe_destroy(h)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_no_cpu_fallback():
    from nano_ktrans_amd.layers.expert_mlp import SparseExpertMLP
    from nano_ktrans_amd.layers.hybrid_moe import HybridMoE
    from nano_ktrans_amd.native_moe import NativeMoE

    with pytest.raises(N.NativeError):
        NativeMoE(num_experts=8, top_k=2, hidden_size=128, intermediate_size=128, device="cpu")
    experts = torch.nn.ModuleDict({str(i): SparseExpertMLP(128, 128) for i in range(4)})
    moe = HybridMoE(4, 2, 128, 128, experts, torch.ones(4, dtype=torch.bool), 0, "")
    with pytest.raises(N.NativeError):
        moe(torch.randn(3, 128), torch.randn(3, 4))
