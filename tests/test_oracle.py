"""Pins for the CPU oracle (oracle/oracle.py + oracle/nkt_oracle.c).

Each oracle function is checked against something it does not itself
compute: float64 math, torch's independent implementations, closed forms on
hand-built inputs, brute force on small cases, and the reference's own test
expectations (nano-ktrans tests/test_quantized_ops.py:7-73, tests/test_core.py:
439-469).  The reference ships no golden vectors for this path.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O


# ---------------------------------------------------------------- exp / bf16
def test_expf_within_one_ulp_of_float64():
    x = np.linspace(-103.9, 88.7, 1_000_003).astype(np.float32)
    y = O.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    normal = ref > 1.18e-38
    assert np.max(np.abs(y - ref)[normal] / ulp[normal]) <= 1.0


def test_expf_special_values():
    assert O.expf(np.array([0.0], np.float32))[0] == 1.0
    assert O.expf(np.array([-np.inf], np.float32))[0] == 0.0
    assert O.expf(np.array([np.inf], np.float32))[0] == np.inf
    assert np.isnan(O.expf(np.array([np.nan], np.float32))[0])
    assert O.expf(np.array([-200.0], np.float32))[0] == 0.0
    # subnormal results: within one subnormal step of float64
    x = np.linspace(-103.0, -87.5, 2001).astype(np.float32)
    y = O.expf(x).astype(np.float64)
    assert np.max(np.abs(y - np.exp(x.astype(np.float64)))) <= 2.0 ** -149
    # monotone non-decreasing on a fine grid
    z = O.expf(np.linspace(-20, 20, 200001).astype(np.float32))
    assert np.all(np.diff(z) >= 0)


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, 1.0, 3.0e38, 1e-40, np.inf, -np.inf], np.float32)]).astype(np.float32)
    ours = O.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    # ties go to even: 1 + 2^-8 is exactly between two bf16 values
    assert O.bf16_round(np.array([1.0 + 2.0 ** -8], np.float32))[0] == 1.0
    assert O.bf16_round(np.array([1.0 + 3 * 2.0 ** -8], np.float32))[0] == 1.0 + 2.0 ** -6


# ---------------------------------------------------------------- router logits
def _nearest_bf16_brute(a: float) -> float:
    """Nearest bf16 to a float64 value by enumerating the bf16 neighbours."""
    f = np.float32(a)
    base = int(np.array([f], np.float32).view(np.uint32)[0]) & 0xFFFF0000
    cands = []
    for d in (-0x10000, 0, 0x10000):
        b = (base + d) & 0xFFFFFFFF
        cands.append((float(np.array([b], np.uint32).view(np.float32)[0]), b))
    best = min(abs(c - a) for c, _ in cands)
    ties = [(c, b) for c, b in cands if abs(c - a) == best]
    if len(ties) == 1:
        return ties[0][0]
    return [c for c, b in ties if ((b >> 16) & 1) == 0][0]  # ties to even


def test_round64_to_bf16_matches_brute_force():
    rng = np.random.default_rng(3)
    a = rng.standard_normal(3000) * 10.0 ** rng.integers(-6, 6, 3000)
    # exact halfway points and values a hair either side of them
    mids = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(2.0 + 2.0 ** -7), 96.0 + 0.25])
    a = np.concatenate([a, mids, mids + 1e-12, mids - 1e-12])
    ours = O.round64_to_bf16(a)
    ref = np.array([_nearest_bf16_brute(v) for v in a], np.float32)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_router_logits_one_hot_rows_pick_gate_columns():
    rng = np.random.default_rng(4)
    E, H = 12, 256
    gate = O.bf16_round(rng.standard_normal((E, H)).astype(np.float32))
    x = np.zeros((H, H), np.float32)
    x[np.arange(H), np.arange(H)] = 1.0
    assert np.array_equal(O.router_logits(x, gate), gate.T)
    # scaling an input row by a power of two scales its logits exactly
    x2 = O.bf16_round(rng.standard_normal((5, H)).astype(np.float32))
    assert np.array_equal(O.router_logits(4.0 * x2, gate), 4.0 * O.router_logits(x2, gate))


def test_router_logits_agree_with_torch_bf16_linear():
    """torch's CPU bf16 nn.Linear (fp32 accumulation, one rounding) lands on the
    same bf16 logit or one ulp away."""
    g = torch.Generator().manual_seed(5)
    E, H, T = 60, 2048, 64
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    ref = torch.nn.functional.linear(x, w).float().numpy()
    ours = O.router_logits(x.float().numpy(), w.float().numpy())
    # distance in bf16 steps (both are bf16 values; the sign never differs here)
    assert np.array_equal(np.sign(ref), np.sign(ours))
    ulp = np.abs((ref.view(np.int32) >> 16).astype(np.int64) - (ours.view(np.int32) >> 16).astype(np.int64))
    assert ulp.max() <= 1
    assert (ulp == 0).mean() > 0.98


def test_rms_norm_closed_forms():
    rng = np.random.default_rng(6)
    H = 512
    w = O.bf16_round(rng.standard_normal(H).astype(np.float32))
    # constant rows, eps 0: x / rms(x) = sign(x) exactly, so the output is +-w
    x = np.array([[3.0] * H, [-0.125] * H], np.float32)
    out = O.rms_norm(x, w, 0.0)
    assert np.array_equal(out[0], w) and np.array_equal(out[1], -w)
    # eps 0: scaling a row by a power of two leaves the output unchanged
    r = O.bf16_round(rng.standard_normal((4, H)).astype(np.float32))
    assert np.array_equal(O.rms_norm(r, w, 0.0), O.rms_norm(8.0 * r, w, 0.0))
    # unit weight: the rows have unit root-mean-square up to bf16 rounding
    n = O.rms_norm(r, np.ones(H, np.float32), 1e-6)
    assert np.allclose(np.sqrt(np.mean(n.astype(np.float64) ** 2, axis=1)), 1.0, atol=2e-3)
    # eps dominates a tiny row: x / sqrt(eps)
    tiny = np.full((1, H), 2.0 ** -20, np.float32)
    assert np.allclose(O.rms_norm(tiny, np.ones(H, np.float32), 1e-2), 2.0 ** -20 / np.sqrt(1e-2 + 2.0 ** -40),
                       rtol=2 ** -8)


# ---------------------------------------------------------------- softmax
@pytest.mark.parametrize("E", [8, 60, 64, 100, 128, 256])
def test_softmax_row_close_to_float64(E):
    rng = np.random.default_rng(E)
    for _ in range(20):
        x = (rng.standard_normal(E) * 3).astype(np.float32)
        p = O.softmax_row(x).astype(np.float64)
        x64 = x.astype(np.float64)
        ref = np.exp(x64 - x64.max())
        ref /= ref.sum()
        # fp32 rounding of (x - max) contributes |x - max| * 2^-24 relative error on top of
        # exp's ulp, the division's half ulp and the sum's rounding
        bound = np.abs(x64 - x64.max()) * 2.0 ** -23 + 8 * 2.0 ** -24
        assert np.all(np.abs(p - ref) / ref < bound)
        assert abs(p.sum() - 1.0) < 1e-6


def test_softmax_row_agrees_with_torch_to_a_few_ulp():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((64, 128)) * 0.9).astype(np.float32)
    ours = np.stack([O.softmax_row(r) for r in x])
    ref = torch.softmax(torch.from_numpy(x), dim=-1, dtype=torch.float32).numpy()
    ulp = np.spacing(ref)
    # two independent fp32 softmaxes, each a few ulp from the truth
    d = np.abs(ours - ref) / ulp
    assert np.max(d) <= 6 and np.mean(d) < 1.0


# ---------------------------------------------------------------- routing
def test_route_tie_rule_lower_id_first():
    # duplicate maxima at ids 5 and 2: the lower id must come first
    logits = np.full((1, 8), -1.0, np.float32)
    logits[0, 5] = 2.0
    logits[0, 2] = 2.0
    ids, w = O.route(logits, 2, use_softmax=True, renorm=True, bf16=False)
    assert ids.tolist() == [[2, 5]]
    assert w[0, 0] == w[0, 1] == np.float32(0.5)
    ids, _ = O.route(logits, 2, use_softmax=False, renorm=True, bf16=False)
    assert ids.tolist() == [[2, 5]]


def test_route_all_equal_logits_select_first_ids():
    for E, k in [(8, 2), (60, 4), (128, 8)]:
        logits = np.zeros((3, E), np.float32)
        ids, w = O.route(logits, k, use_softmax=True, renorm=True, bf16=True)
        assert (ids == np.arange(k)).all()
        assert np.allclose(w, 1.0 / k, rtol=2 ** -7)
        ids, w = O.route(logits, k, use_softmax=True, renorm=False, bf16=False)
        assert (ids == np.arange(k)).all()
        assert np.allclose(w, 1.0 / E, rtol=1e-6)


def test_route_one_hot_logits():
    E, k = 128, 8
    logits = np.zeros((E, E), np.float32)
    logits[np.arange(E), np.arange(E)] = 10.0
    ids, w = O.route(logits, k, use_softmax=True, renorm=True, bf16=True)
    assert (ids[:, 0] == np.arange(E)).all()
    # the remaining k-1 are the lowest ids other than the hot one
    for t in range(E):
        rest = [e for e in range(E) if e != t][: k - 1]
        assert ids[t, 1:].tolist() == rest


def test_route_negative_zero_equals_positive_zero():
    logits = np.array([[-0.0, 0.0, -1.0, -2.0]], np.float32)
    ids, _ = O.route(logits, 2, use_softmax=False, renorm=True, bf16=False)
    assert ids.tolist() == [[0, 1]]


@pytest.mark.parametrize("E,k", [(8, 2), (60, 4), (128, 8)])
def test_route_matches_torch_topk_without_ties(E, k):
    rng = np.random.default_rng(E * 31 + k)
    logits = (rng.standard_normal((256, E)) * 2).astype(np.float32)
    ids, w = O.route(logits, k, use_softmax=True, renorm=True, bf16=False)
    lt = torch.from_numpy(logits)
    p = torch.softmax(lt, dim=-1, dtype=torch.float32)
    tw, tid = torch.topk(p, k, dim=-1)
    tw = tw / tw.sum(-1, keepdim=True)
    assert np.array_equal(ids, tid.numpy().astype(np.int32))
    assert np.allclose(w, tw.numpy(), rtol=1e-6, atol=1e-7)
    # Mixtral order: topk on logits, then softmax of the k values
    ids2, w2 = O.route(logits, k, use_softmax=False, renorm=True, bf16=False)
    tv, tid2 = torch.topk(lt, k, dim=-1)
    assert np.array_equal(ids2, tid2.numpy().astype(np.int32))
    assert np.allclose(w2, torch.softmax(tv, dim=-1).numpy(), rtol=1e-6, atol=1e-7)
    # and in fp32 the two orders agree (softmax is monotone, renorm cancels the denominator)
    assert np.array_equal(ids, ids2)
    assert np.allclose(w, w2, rtol=1e-5)


def test_route_bf16_matches_torch_reference_semantics():
    """Softmax arch with bf16 logits: probs rounded to bf16 before selection, renorm in bf16."""
    E, k = 128, 8
    rng = np.random.default_rng(11)
    logits = O.bf16_round((rng.standard_normal((512, E)) * 0.9).astype(np.float32))
    ids, w = O.route(logits, k, use_softmax=True, renorm=True, bf16=True)
    lt = torch.from_numpy(logits).to(torch.bfloat16)
    p = torch.softmax(lt, dim=-1, dtype=torch.float32).to(torch.bfloat16)
    # selection: every chosen value must be >= every unchosen value (ties allowed) and
    # equal values must be taken in id order
    pf = p.float().numpy()
    for t in range(logits.shape[0]):
        chosen = pf[t, ids[t]]
        rest = np.delete(pf[t], ids[t])
        assert chosen.min() >= rest.max()
        assert np.all(np.diff(chosen) <= 0)
        for j in range(k - 1):
            if chosen[j] == chosen[j + 1]:
                assert ids[t, j] < ids[t, j + 1]
    # weights: bf16 renorm of the torch probs at our ids, up to 1 bf16 ulp where torch's exp
    # rounds the other way
    sel = torch.gather(p, 1, torch.from_numpy(ids).long())
    tw = (sel / sel.sum(-1, keepdim=True)).float().numpy()
    assert np.max(np.abs(w - tw) / np.abs(tw)) <= 2 ** -7
    assert np.mean(w == tw) > 0.99


def test_route_weights_sum_to_one_and_ids_in_range():
    # tests/test_core.py:439-469 of the reference: weights normalised, ids in range
    rng = np.random.default_rng(3)
    for (E, k, sm, rn, bf) in [(8, 2, False, True, False), (128, 8, True, True, True),
                               (60, 4, True, False, True), (8, 2, True, True, False)]:
        logits = (rng.standard_normal((33, E))).astype(np.float32)
        if bf:
            logits = O.bf16_round(logits)
        ids, w = O.route(logits, k, sm, rn, bf)
        assert ids.min() >= 0 and ids.max() < E
        assert all(len(set(r)) == k for r in ids.tolist())
        if rn or not sm:
            assert np.allclose(w.sum(-1), 1.0, atol=(k * 2 ** -8) if bf else 1e-6)
        else:
            assert np.all(w.sum(-1) <= 1.0 + 1e-2)


# ---------------------------------------------------------------- grouping
def _brute_group(ids, E):
    T, k = ids.shape
    pairs = sorted(((int(ids[t, j]), t, t * k + j) for t in range(T) for j in range(k)))
    perm = np.array([p for (_, _, p) in pairs], np.int32)
    counts = np.bincount(ids.ravel(), minlength=E).astype(np.int32)
    return counts, perm


@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (16, 8, 2), (37, 60, 4), (64, 128, 8), (5, 128, 8)])
def test_group_matches_brute_force_sort(T, E, k):
    rng = np.random.default_rng(T * 7 + E)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    counts, offsets, perm, inv = O.group(ids, E)
    bc, bperm = _brute_group(ids, E)
    assert np.array_equal(counts, bc)
    assert np.array_equal(perm, bperm)
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts) and offsets[-1] == T * k
    assert np.array_equal(inv[perm], np.arange(T * k))


def test_group_empty():
    counts, offsets, perm, inv = O.group(np.zeros((0, 2), np.int32), 8)
    assert counts.sum() == 0 and offsets.tolist() == [0] * 9 and perm.size == 0


# ---------------------------------------------------------------- quantizers
def test_quantize_int4_closed_form_small():
    # one row, group 8: max |w| = 7 -> scale 1, q = round_half_even(w)
    w = np.array([[7.0, -7.0, 2.5, 3.5, -2.5, 0.49, 0.5, 1.5] + [0.0] * 8], np.float32)
    qw = O.quantize_int4(w, group_size=8)
    assert qw.scales[0, 0] == np.float32(1.0)
    assert qw.scales[0, 1] == np.float32(1e-6 / 7)
    q = O.unpack_words(qw.qweight, 4)[0, :8] - 8
    assert q.tolist() == [7, -7, 2, 4, -2, 0, 0, 2]
    # nibble order: column 8w+j sits at bits [4j, 4j+4) of word w, stored q + 8
    stored = (np.array([7, -7, 2, 4, -2, 0, 0, 2]) + 8).astype(np.uint64)
    word = int(sum(int(v) << (4 * j) for j, v in enumerate(stored)))
    assert int(qw.qweight.view(np.uint32)[0, 0]) == word


def test_quantize_int4_roundtrip_bounds():
    rng = np.random.default_rng(5)
    w = rng.standard_normal((16, 128)).astype(np.float32)
    qw = O.quantize_int4(w, group_size=64)
    assert qw.qweight.shape == (16, 16) and qw.scales.shape == (16, 2)
    deq = O.dequantize(qw)
    # reference tolerance (tests/test_quantized_ops.py:7-17) and the half-step bound
    assert np.allclose(w, deq, atol=1.0, rtol=0.25)
    step = np.repeat(qw.scales, 64, axis=1)
    assert np.all(np.abs(w - deq) <= step / 2 * (1 + 1e-6))


def test_quantize_int8_closed_form_and_bounds():
    w = np.array([[127.0, -127.0, 0.5, 1.5, 2.5, -0.5, 64.0, 0.0]], np.float32)
    qw = O.quantize_int8_pc(w)
    assert qw.scales.shape == (1, 1) and qw.scales[0, 0] == np.float32(1.0)
    q = O.unpack_words(qw.qweight, 8)[0] - 128
    assert q.tolist() == [127, -127, 0, 2, 2, 0, 64, 0]
    rng = np.random.default_rng(6)
    w = rng.standard_normal((8, 256)).astype(np.float32)
    qw = O.quantize_int8_pc(w)
    deq = O.dequantize(qw)
    assert np.all(np.abs(w - deq) <= qw.scales / 2 * (1 + 1e-6))


def test_product_quantizers_match_oracle_bit_exact():
    from nano_ktrans_amd.kernels.quantized_ops import (quantize_symmetric_int8_per_channel,
                                                       quantize_symmetric_w4a32)
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((96, 512)) * 0.02).astype(np.float32)
    a = O.quantize_int4(w, 128)
    b = quantize_symmetric_w4a32(torch.from_numpy(w), group_size=128)
    assert np.array_equal(a.qweight, b.qweight.numpy())
    assert np.array_equal(a.scales, b.scales.numpy())
    a = O.quantize_int8_pc(w)
    b = quantize_symmetric_int8_per_channel(torch.from_numpy(w))
    assert np.array_equal(a.qweight, b.qweight.numpy())
    assert np.array_equal(a.scales, b.scales.numpy())


def test_matvec_grouped_equals_linear_of_dequantized():
    # reference tests/test_quantized_ops.py:55-73: grouped == dense == F.linear(dequant) at 1e-5
    rng = np.random.default_rng(10)
    for qw in (O.quantize_int4(rng.standard_normal((24, 128)).astype(np.float32), 64),
               O.quantize_int8_pc(rng.standard_normal((24, 128)).astype(np.float32))):
        x = rng.standard_normal((3, 128)).astype(np.float32)
        out = O.matvec_grouped(x, qw)
        ref = torch.nn.functional.linear(torch.from_numpy(x), torch.from_numpy(O.dequantize(qw))).numpy()
        assert np.allclose(out, ref, atol=1e-5, rtol=1e-5)
        ref64 = x.astype(np.float64) @ O.dequantize(qw).astype(np.float64).T
        assert np.allclose(out, ref64, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------- experts / layer
def _torch_swiglu64(x, g, u, d):
    x, g, u, d = (torch.from_numpy(np.asarray(a, np.float64)) for a in (x, g, u, d))
    return (torch.nn.functional.silu(x @ g.T) * (x @ u.T) @ d.T).numpy()


def test_expert_forward_is_dense_swiglu():
    rng = np.random.default_rng(12)
    H, I = 64, 96
    g, u, d = (rng.standard_normal(s).astype(np.float32) * 0.1 for s in ((I, H), (I, H), (H, I)))
    x = rng.standard_normal((5, H)).astype(np.float32)
    out = O.expert_forward(x, O.Expert(g, u, d))
    assert O.rel_l2(out, _torch_swiglu64(x, g, u, d)) < 1e-6


def test_expert_forward_bf16_h():
    """h_bf16 rounds the SwiGLU output to bf16 before the down projection:
    against torch's float64 SwiGLU with a torch bf16 cast of h, and the change
    from the fp32 result stays within the rounding bound 2^-9 |h| per element."""
    rng = np.random.default_rng(13)
    H, I = 64, 96
    g, u, d = (rng.standard_normal(s).astype(np.float32) * 0.3 for s in ((I, H), (I, H), (H, I)))
    x = rng.standard_normal((5, H)).astype(np.float32)
    ex = O.Expert(g, u, d)
    got = O.expert_forward(x, ex, h_bf16=True)
    x64, g64, u64, d64 = (torch.from_numpy(np.asarray(a, np.float64)) for a in (x, g, u, d))
    h64 = torch.nn.functional.silu(x64 @ g64.T) * (x64 @ u64.T)
    ref = (h64.to(torch.bfloat16).to(torch.float64) @ d64.T).numpy()
    assert O.rel_l2(got, ref) < 1e-5
    plain = O.expert_forward(x, ex)
    bound = (np.abs(h64.numpy()) * 2.0 ** -9) @ np.abs(d.astype(np.float64)).T
    assert np.all(np.abs(got.astype(np.float64) - plain) <= bound * 1.01 + 1e-5)
    assert O.rel_l2(got, plain) > 1e-4  # the rounding is really applied


def test_moe_forward_matches_independent_torch_loop():
    """C0 shape, fp32: the reference loop (softmax -> top-2 -> renorm, experts in ascending
    id, index_add_) written with torch float64 ops."""
    rng = np.random.default_rng(0)
    T, H, E, k, I = 16, 256, 8, 2, 512
    x = rng.standard_normal((T, H)).astype(np.float32)
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    experts = [O.Expert(*(rng.standard_normal(s).astype(np.float32) * 0.02 for s in ((I, H), (I, H), (H, I))))
               for _ in range(E)]
    logits = x @ router.T
    out = O.moe_forward(x, logits, experts, k, use_softmax=True, renorm=True, bf16=False)
    lt = torch.from_numpy(logits.astype(np.float64))
    p = torch.softmax(lt, -1)
    tw, tid = torch.topk(p, k, -1)
    tw = tw / tw.sum(-1, keepdim=True)
    ref = torch.zeros(T, H, dtype=torch.float64)
    for e in range(E):
        rows, slots = torch.where(tid == e)
        if rows.numel() == 0:
            continue
        ex = experts[e]
        y = torch.from_numpy(_torch_swiglu64(x[rows.numpy()], ex.gate, ex.up, ex.down))
        ref.index_add_(0, rows, y * tw[rows, slots].unsqueeze(1))
    assert O.rel_l2(out, ref.numpy()) < 1e-5


def test_moe_forward_given_matches_independent_torch_loop():
    """The loop on caller-given routing (the offload backend's side of the
    contract): ids in shuffled slot order, weights that neither sum to one
    nor descend by slot, the same expert picked by many tokens.  Against the
    reference loop's torch float64 restatement (cpu_moe.py:515-538: experts
    ascending, torch.where per expert, index_add_), and against moe_forward
    where the given routing is the oracle's own."""
    rng = np.random.default_rng(12)
    T, H, E, k, I = 11, 128, 6, 3, 128
    x = rng.standard_normal((T, H)).astype(np.float32)
    experts = [O.Expert(*(rng.standard_normal(s).astype(np.float32) * 0.05 for s in ((I, H), (I, H), (H, I))))
               for _ in range(E)]
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    ids[:5, 0] = 4  # a hot expert
    for t in range(5):
        rest = [e for e in range(E) if e != 4]
        ids[t, 1:] = rng.permutation(rest)[: k - 1]
    w = (rng.random((T, k)) * 2.0 - 0.5).astype(np.float32)
    out = O.moe_forward_given(x, ids, w, experts)
    tid = torch.from_numpy(ids.astype(np.int64))
    tw = torch.from_numpy(w.astype(np.float64))
    ref = torch.zeros(T, H, dtype=torch.float64)
    for e in range(E):
        rows, slots = torch.where(tid == e)
        if rows.numel() == 0:
            continue
        ex = experts[e]
        y = torch.from_numpy(_torch_swiglu64(x[rows.numpy()], ex.gate, ex.up, ex.down))
        ref.index_add_(0, rows, y * tw[rows, slots].unsqueeze(1))
    assert O.rel_l2(out, ref.numpy()) < 1e-5
    # the slot order of a token does not matter
    perm = np.stack([rng.permutation(k) for _ in range(T)])
    shuf = O.moe_forward_given(x, np.take_along_axis(ids, perm, 1), np.take_along_axis(w, perm, 1), experts)
    assert np.array_equal(shuf, out)
    # given the oracle's own routing, it is moe_forward
    logits = rng.standard_normal((T, E)).astype(np.float32)
    rid, rw = O.route(logits, k, True, True, False)
    assert np.array_equal(O.moe_forward_given(x, rid, rw, experts),
                          O.moe_forward(x, logits, experts, k, True, True, False))


def test_moe_forward_single_expert_reduces_to_dense_mlp():
    rng = np.random.default_rng(4)
    T, H, I = 7, 128, 128
    ex = O.Expert(*(rng.standard_normal(s).astype(np.float32) * 0.05 for s in ((I, H), (I, H), (H, I))))
    x = rng.standard_normal((T, H)).astype(np.float32)
    out = O.moe_forward(x, np.zeros((T, 1), np.float32), [ex], 1, use_softmax=True, renorm=True, bf16=False)
    assert O.rel_l2(out, _torch_swiglu64(x, ex.gate, ex.up, ex.down)) < 1e-6


def test_moe_forward_shared_expert_closed_form():
    rng = np.random.default_rng(8)
    T, H, E, k, I, Is = 6, 128, 4, 2, 128, 256
    x = rng.standard_normal((T, H)).astype(np.float32)
    experts = [O.Expert(*(rng.standard_normal(s).astype(np.float32) * 0.05 for s in ((I, H), (I, H), (H, I))))
               for _ in range(E)]
    sh = O.Expert(*(rng.standard_normal(s).astype(np.float32) * 0.05 for s in ((Is, H), (Is, H), (H, Is))))
    g = rng.standard_normal(H).astype(np.float32) * 0.05
    logits = rng.standard_normal((T, E)).astype(np.float32)
    base = O.moe_forward(x, logits, experts, k, True, False, False)
    full = O.moe_forward(x, logits, experts, k, True, False, False, shared=sh, shared_gate=g)
    gate = 1.0 / (1.0 + np.exp(-(x.astype(np.float64) @ g)))
    expect = base + gate[:, None] * _torch_swiglu64(x, sh.gate, sh.up, sh.down)
    assert O.rel_l2(full, expect) < 1e-6


def test_torch_cpu_loop_matches_oracle():
    """oracle/cpu_loop.py (the torch restatement timed as the CPU baseline)
    equals the numpy oracle's forward: int4 and int8 experts, and dense fp32."""
    import cpu_loop as C

    rng = np.random.default_rng(21)
    T, H, E, k, I = 9, 256, 6, 2, 256
    x = O.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = O.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    for kind in ("int4", "int8", "f32"):
        def mk(n, kk):
            w = rng.standard_normal((n, kk)).astype(np.float32) * 0.05
            if kind == "int4":
                return O.with_bf16_scales(O.quantize_int4(w))
            if kind == "int8":
                return O.with_bf16_scales(O.quantize_int8_pc(w))
            return w
        experts = [O.Expert(mk(I, H), mk(I, H), mk(H, I)) for _ in range(E)]
        ref = O.moe_forward(x, logits, experts, k, True, True, True)
        ids, w = O.route(logits, k, True, True, True)
        got = C.moe_loop(x, ids, w, [C.to_torch_expert(e) for e in experts])
        assert O.rel_l2(got, ref) < 1e-5, kind
