#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X.

Headline workload: one Qwen3-30B-A3B-shaped MoE layer (H=2048, 128 experts,
top-8, moe_intermediate=768, int4 group-128 weights with bf16 scales, bf16
activations) decoding 16 tokens.  A step is one layer forward (route, group,
gate_up GEMM + SwiGLU, down GEMM, combine) on a new weight copy: steps rotate
over --layers distinct copies of the layer (> 2 GB in total, beyond the 256 MB
last-level cache) and over 8 seeded inputs, step i taking input
(i + i // layers) mod 8, so 8 x layers (copy, input) pairs -- each its own set
of routed experts -- pass before one recurs, the way consecutive layers of a
model would stream their weights from HBM (at one token a step reads ~19 MB of
experts: 64 pairs still exceed the last-level cache).  After --warmup eager steps,
exactly --steps steps are timed as one replay of a HIP graph holding them,
with HIP events between device synchronisations.

Printed JSON fields beyond the standard ones:
  us_per_layer   layer latency
  breakdown_us   per-stage device time from HIP events (eager, the host kept ahead)
  roofline       dominant kernel: algorithmic bytes (active experts' codes + scales,
                 activations in/out) / its average event-timed duration vs 8 TB/s;
                 traffic (and, for the prefill form, MFMA busy %) from rocprofv3
                 counters on nano-ktrans_amd/nkt_probe (profiles/pmc_moe_layer_counters.md);
                 beside the rated peak, the practical ones measured in the same run:
                 vendor_gemv (torch.matmul of T tokens by a 512 MB fp16 weight, weight
                 bytes read/s: a read-only stream of the decode GEMV's kind) and
                 vendor_copy (a 256 MB torch device copy, read + write bytes/s) for
                 the HBM bound, vendor_gemm (torch.matmul in fp16 of the same
                 multiply-adds as one dense [T k, N, K] GEMM) for the MFMA bound
  cpu_baseline   the reference CPU expert loop (oracle/cpu_loop.py, a torch
                 restatement of nano_ktrans/kernels/cpu_moe.py:491-539) on this
                 host's cores for the headline; cpu_baselines: every config at
                 every token count the bench reports (Mixtral T=2048 on a
                 512-token sample)
  secondary      other token counts (T=1, 4), the layer from hidden states
                 (router GEMV inside; plus RMSNorm and residual), the tiny
                 fp32 Mixtral-style layer (T=16), the int8 per-channel prefill
                 at T=512/2048/4096 (Zipf-skewed routing), a Mixtral-8x7B-shaped
                 int4 layer (T=1, 16, 2048) and a Qwen1.5-MoE-shaped int8 layer
                 with its shared expert (T=1, 16, 1024); roofline_alt gives the
                 other bound's fraction where a shape sits near the ridge
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nano-ktrans_amd"))

HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
MFMA_BF16_PEAK = 2.5e15    # FLOP/s, dense bf16 (fp16 the same)
MFMA_F32_PEAK = 157.3e12   # FLOP/s, dense fp32 matrix cores

METRIC = "MoE-layer tokens/s + decode µs/layer (Qwen3-30B-A3B shape); % HBM/MFMA roofline"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --------------------------------------------------------------------- problem
class Workload:
    """One MoE layer shape.  probe: the name nano-ktrans_amd/nkt_probe and the
    counter table in profiles/ use for it."""

    def __init__(self, name, H, E, k, I, wfmt, softmax, renorm, tokens, zipf=0.0, seed=1, shared=0,
                 act="bf16", probe=""):
        self.name, self.H, self.E, self.k, self.I = name, H, E, k, I
        self.wfmt, self.softmax, self.renorm, self.tokens, self.zipf, self.seed = wfmt, softmax, renorm, tokens, zipf, seed
        self.shared = shared  # shared-expert intermediate size (0: none)
        self.act, self.probe = act, probe

    @property
    def act_dtype(self):
        import torch
        return torch.float32 if self.act == "f32" else torch.bfloat16

    @property
    def act_bytes(self):
        return 4 if self.act == "f32" else 2

    def _bytes(self, n, kk):
        if self.wfmt == "int4_g128":
            return n * kk // 2 + n * (kk // 128) * 2
        if self.wfmt == "int8_per_channel":
            return n * kk + n * 2
        if self.wfmt == "f32":
            return n * kk * 4
        return n * kk * 2

    def bytes_per_expert(self, proj):
        n, kk = (2 * self.I, self.H) if proj == "gate_up" else (self.H, self.I)
        return self._bytes(n, kk)

    def shared_bytes(self):
        """Shared expert (gate_up + down) plus its gate vector, read once per layer call."""
        if not self.shared:
            return 0
        return self._bytes(2 * self.shared, self.H) + self._bytes(self.H, self.shared) + self.H * self.act_bytes


QWEN3_INT4 = dict(H=2048, E=128, k=8, I=768, wfmt="int4_g128", softmax=True, renorm=True, seed=1, probe="qwen3_int4")
QWEN3_INT8 = dict(H=2048, E=128, k=8, I=768, wfmt="int8_per_channel", softmax=True, renorm=True, seed=1, zipf=1.1,
                  probe="qwen3_int8")
# Mixtral-8x7B-shaped layer (top-k on the logits, then softmax over the k) and
# Qwen1.5-MoE-A2.7B-shaped layer (60 experts, softmax without renormalisation,
# shared expert with a sigmoid gate)
MIXTRAL_INT4 = dict(H=4096, E=8, k=2, I=14336, wfmt="int4_g128", softmax=False, renorm=False, seed=2,
                    probe="mixtral_int4")
QWEN15_INT8 = dict(H=2048, E=60, k=4, I=1408, wfmt="int8_per_channel", softmax=True, renorm=False, seed=3,
                   shared=5632, probe="qwen15_int8")
# the reference's own CPU-runnable case: tiny Mixtral-style layer, fp32, dense experts
TINY_F32 = dict(H=256, E=8, k=2, I=512, wfmt="f32", softmax=True, renorm=True, seed=0, act="f32", probe="tiny_f32")


def make_layers(w, n_layers, device, max_tokens):
    """One seeded layer (quantized on the GPU) in n_layers distinct device copies,
    plus its expert weights on the host (the CPU baseline's weights):
    (router, layers, {"experts": [{gate, up, down}], "shared": {...} | None, "shared_gate": tensor | None})."""
    import torch
    from nano_ktrans_amd.kernels.quantized_ops import (quantize_symmetric_int8_per_channel,
                                                       quantize_symmetric_w4a32)
    from nano_ktrans_amd.kernels.weight_loader import GPTQLinearWeight
    from nano_ktrans_amd.native_moe import NativeMoE

    if w.wfmt == "int4_g128":
        quant = lambda t: quantize_symmetric_w4a32(t, group_size=128)
    elif w.wfmt == "int8_per_channel":
        quant = quantize_symmetric_int8_per_channel
    else:
        quant = lambda t: t.to(w.act_dtype)

    def host(q):
        if isinstance(q, GPTQLinearWeight):
            return GPTQLinearWeight(q.qweight.cpu(), q.scales.to(torch.bfloat16).float().cpu(), None, q.group_size,
                                    q.bits, q.sym, q.linear_prefix)
        return q.float().cpu()

    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    router = torch.randn(w.E, w.H, generator=g, device=device) * 0.02
    layers = []
    mk = lambda: NativeMoE(num_experts=w.E, top_k=w.k, hidden_size=w.H, intermediate_size=w.I,
                           shared_intermediate_size=w.shared, weight_format=w.wfmt, act_dtype=w.act_dtype,
                           use_softmax=w.softmax, renorm=w.renorm, max_tokens=max_tokens, device=device)
    first = mk()
    src = {"experts": [], "shared": None, "shared_gate": None}
    for e in range(w.E):
        gate_up = torch.randn(2 * w.I, w.H, generator=g, device=device) * 0.02
        down = torch.randn(w.H, w.I, generator=g, device=device) * 0.02
        qs = (quant(gate_up[: w.I]), quant(gate_up[w.I:]), quant(down))
        first.load_expert(e, *qs)
        src["experts"].append({"gate": host(qs[0]), "up": host(qs[1]), "down": host(qs[2])})
        del gate_up, down, qs
    if w.shared:
        gs = torch.randn(2 * w.shared, w.H, generator=g, device=device) * 0.02
        ds = torch.randn(w.H, w.shared, generator=g, device=device) * 0.02
        gw = torch.randn(1, w.H, generator=g, device=device) * 0.02
        qs = (quant(gs[: w.shared]), quant(gs[w.shared:]), quant(ds))
        first.load_shared_expert(*qs, gw)
        src["shared"] = {"gate": host(qs[0]), "up": host(qs[1]), "down": host(qs[2])}
        src["shared_gate"] = gw.to(w.act_dtype).float().reshape(-1).cpu()
        del gs, ds
    layers.append(first)
    for _ in range(1, n_layers):
        n = mk()
        for slot, t in first.slots.items():
            n.slots[slot].copy_(t)
        layers.append(n)
    torch.cuda.synchronize()
    return router, layers, src


def make_inputs(w, router, T, n_inputs, device):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(1000 + T)
    xs, ls = [], []
    for _ in range(n_inputs):
        x = torch.randn(T, w.H, generator=g, device=device).to(w.act_dtype)
        logits = x.float() @ router.T
        if w.zipf:
            e = torch.arange(w.E, device=device, dtype=torch.float32)
            logits = logits - w.zipf * torch.log(e + 1.0)
        xs.append(x)
        ls.append(logits.to(w.act_dtype))
    return xs, ls


def active_experts(layer, logits):
    import torch

    ids = layer.route(logits)[0]
    return int(torch.unique(ids).numel())


# --------------------------------------------------------------------- timing
def step_input(i, L):
    """Input of step i (taken modulo the input count) when steps rotate over L
    layer copies: i + i // L, so copy i % L meets a new input on every visit
    and L x (input count) (copy, input) pairs -- each reading its own routed
    experts -- pass before one recurs.  With the same input on every visit a
    one-token step over 8 copies would re-read ~150 MB of experts, which the
    256 MB last-level cache holds."""
    return i + i // L


def time_steps(layers, xs, outs, steps, warmup, call):
    """Exactly `steps` layer calls (call(layer, j, out): layer copy i % L,
    input j = step_input(i, L)), timed as one replay of a HIP graph that
    holds those calls, between device synchronisations, after `warmup` eager
    calls.  Returns ms per step."""
    import torch

    L = len(layers)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i, layer in enumerate(layers):  # make every workspace before capture
            call(layer, step_input(i, L), outs[i])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            call(layers[i % L], step_input(i, L), outs[i % L])
    for i in range(warmup):
        call(layers[i % L], step_input(i, L), outs[i % L])
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    del graph
    return ms


def time_graph(layers, xs, ls, outs, steps, warmup):
    """The layer from (hidden_states, router_logits): ms per step."""
    return time_steps(layers, xs, outs, steps, warmup,
                      lambda layer, j, out: layer.forward(xs[j % len(xs)], ls[j % len(ls)], out=out))


def time_graph_hidden(layers, xs, outs, steps, warmup, call=None):
    """The layer from hidden states alone (router GEMV inside the path; or
    call(layer, x, out)): ms per step."""
    if call is None:
        call = lambda layer, x, out: layer.forward_hidden(x, out=out)
    return time_steps(layers, xs, outs, steps, warmup, lambda layer, j, out: call(layer, xs[j % len(xs)], out))


def time_stages(layers, xs, ls, outs, rounds):
    """Per-stage device time with HIP events; a sleep kernel keeps the host ahead."""
    import torch

    names = ["route+group", "gate_up", "down", "combine"]
    acc = {n: 0.0 for n in names}
    count = 0
    stream = torch.cuda.current_stream()
    L = len(layers)
    for r in range(rounds):
        try:
            torch.cuda._sleep(50_000_000)  # keep the device busy while the host enqueues
        except Exception:
            pass
        evs = []
        for i, layer in enumerate(layers):
            j = step_input(r * L + i, L)
            x, lg = xs[j % len(xs)], ls[j % len(ls)]
            T = x.shape[0]
            e = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
            e[0].record(stream)
            layer.route(lg)
            e[1].record(stream)
            layer.expert_phase(0, x, T)
            e[2].record(stream)
            layer.expert_phase(1, None, T)
            e[3].record(stream)
            layer.combine(T, outs[i])
            e[4].record(stream)
            evs.append(e)
        torch.cuda.synchronize()
        for e in evs:
            for j, n in enumerate(names):
                acc[n] += e[j].elapsed_time(e[j + 1]) * 1e3
            count += 1
    return {n: acc[n] / count for n in names}


def time_kernel(layers, xs, ls, phase, passes=5):
    """Average duration (us) of one expert-GEMM kernel (phase 0: gate_up + SwiGLU,
    1: down).  Each pass routes every layer copy i on input step_input(p L + i, L)
    (and, for the down kernel, runs its gate_up), then runs the phase once per
    copy, back to back, each launch with its own pair of HIP events, stamped by
    the dispatch at the kernel's start and end (nkt_moe_experts_phase_timed), on
    the stream the kernel runs on.  A sleep kernel keeps the host ahead so the
    launches run back to back over the rotating weight copies; a copy's routing
    changes from pass to pass, so no pass finds the previous one's experts in
    the last-level cache."""
    import torch

    T = xs[0].shape[0]
    L = len(layers)
    stream = torch.cuda.current_stream()
    pairs = []
    for _ in range(passes * len(layers)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)  # creates the events; the launch re-stamps them
        b.record(stream)
        pairs.append((a, b))
    torch.cuda.synchronize()
    try:
        torch.cuda._sleep(20_000_000)
    except Exception:
        pass
    n = 0
    for p in range(passes):
        inputs = [step_input(p * L + i, L) for i in range(L)]
        for layer, j in zip(layers, inputs):
            layer.route(ls[j % len(ls)])
            if phase == 1:
                layer.expert_phase(0, xs[j % len(xs)], T)
        for layer, j in zip(layers, inputs):
            a, b = pairs[n]
            layer.expert_phase_timed(phase, xs[j % len(xs)] if phase == 0 else None, T, a, b)
            n += 1
    torch.cuda.synchronize()
    times = [a.elapsed_time(b) * 1e3 for a, b in pairs]
    return sum(times) / len(times)


def kernel_form(w, T):
    """Which K3 kernel the library runs for this shape (mirrors gemm_tile_m)."""
    avg = T * w.k / w.E
    if w.wfmt == "f32":
        return "gemm_kernel"
    int8 = 3.5 if w.shared else 4.5
    if avg <= {"int8_per_channel": int8, "int4_g128": 6 if w.I >= 8192 else 8}.get(w.wfmt, 12):
        return "gemv_kernel"
    # int8 and int4 (bf16 activations, buffers under 4 GiB: every bench shape) have pipelined kernels
    return {"int8_per_channel": "gemm2_i8_kernel", "int4_g128": "gemm2_i4_kernel"}.get(w.wfmt, "gemm2_kernel")


def bench_workload(w, T, layers, router, steps, warmup, device):
    import torch

    xs, ls = make_inputs(w, router, T, 8, device)
    outs = [torch.empty(T, w.H, dtype=w.act_dtype, device=device) for _ in layers]
    n_act = [active_experts(layers[0], l) for l in ls]
    mean_act = sum(n_act) / len(n_act)
    ms = time_graph(layers, xs, ls, outs, steps, warmup)
    stages = time_stages(layers, xs, ls, outs, rounds=3)
    gate_up_us = time_kernel(layers, xs, ls, 0)
    down_us = time_kernel(layers, xs, ls, 1)
    P = T * w.k
    ab = w.act_bytes
    gate_up_bytes = mean_act * w.bytes_per_expert("gate_up") + T * w.H * ab + P * w.I * ab
    down_bytes = mean_act * w.bytes_per_expert("down") + P * w.I * ab + P * w.H * 4
    layer_bytes = (mean_act * (w.bytes_per_expert("gate_up") + w.bytes_per_expert("down"))
                   + w.shared_bytes() + T * w.H * ab * 2 + T * w.E * ab)
    gate_up_flops = 2.0 * P * 2 * w.I * w.H
    down_flops = 2.0 * P * w.H * w.I
    form = kernel_form(w, T)
    return dict(workload=w.name, probe=w.probe, wfmt=w.wfmt, tokens=T, ms_per_step=ms, us_per_layer=ms * 1e3,
                steps=steps, warmup=warmup, tokens_per_s=T / (ms * 1e-3), mean_active_experts=mean_act,
                breakdown_us=stages, layer_bytes=layer_bytes, layer_hbm_frac=layer_bytes / (ms * 1e-3) / HBM_PEAK,
                gate_up=dict(kernel=form, bytes=gate_up_bytes, flops=gate_up_flops, us=gate_up_us),
                down=dict(kernel=form, bytes=down_bytes, flops=down_flops, us=down_us),
                shape=dict(k=w.k, H=w.H, I=w.I), inputs=(xs[0], ls[0]))


COUNTERS_MD = os.path.join(ROOT, "profiles", "pmc_moe_layer_counters.md")


def counter_table():
    """Per-launch HBM traffic and matrix-core counters of the expert GEMMs, measured
    with rocprofv3 --pmc on nkt_probe (profiles/pmc_moe_layer_counters.md), keyed
    (probe workload, tokens, phase) -> {"traffic": bytes, "mfma_util": %}."""
    try:
        text = open(COUNTERS_MD).read()
    except OSError:
        return {}
    out = {}
    for line in text.splitlines():
        # | `probe:T:phase` | kernel | grid | read B | write B | traffic B | MFMA busy % | MFMA GFLOP | ...
        if not line.startswith("| `") or line.count("|") < 9:
            continue
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        key = cells[0].strip("`")
        if key.count(":") != 2:
            continue
        try:
            out[key] = {"traffic": float(cells[5]),
                        "mfma_util": float(cells[6]) if cells[6] not in ("", "-") else None}
        except (ValueError, IndexError):
            pass
    return out


_CEILINGS = {}


def _event_ms(fn, reps):
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def vendor_gemm_tflops(M, N, K):
    """Rate (TFLOP/s) of one dense fp16 [M, K] x [K, N] product through
    torch.matmul (the vendor GEMM library) on this GPU: the practical
    matrix-core ceiling for the same multiply-add count, measured because
    MI355X's clock drops well below its rated one under sustained MFMA load."""
    key = ("gemm", M, N, K)
    if key not in _CEILINGS:
        import torch

        a = torch.randn(M, K, device="cuda", dtype=torch.float16)
        b = torch.randn(K, N, device="cuda", dtype=torch.float16)
        flop = 2.0 * M * N * K
        ms = _event_ms(lambda: a @ b, max(3, min(20, int(4e12 / flop))))
        _CEILINGS[key] = flop / (ms * 1e-3) / 1e12
        del a, b
    return _CEILINGS[key]


def vendor_copy_gbps(nbytes=256 << 20):
    """Rate (GB/s, bytes read + written) of a device-to-device copy of nbytes
    through torch on this GPU: the practical HBM streaming rate."""
    key = ("copy", nbytes)
    if key not in _CEILINGS:
        import torch

        src = torch.empty(nbytes // 2, device="cuda", dtype=torch.float16).normal_()
        dst = torch.empty_like(src)
        ms = _event_ms(lambda: dst.copy_(src), 20)
        _CEILINGS[key] = 2.0 * nbytes / (ms * 1e-3) / 1e9
        del src, dst
    return _CEILINGS[key]


def vendor_gemv_gbps(M):
    """Rate (GB/s, weight bytes read) of torch.matmul [M, 16384] x [16384, 16384]
    in fp16 on this GPU (the vendor BLAS, 512 MB of weights read once per
    product, M = the kernel's token count): a read-only weight stream of the
    decode GEMV's own kind, the fair comparator for kernels that only read
    weights (a device copy also writes, and torch's reductions read at well
    under either: 3.5 - 4.3 TB/s measured for sum / amax / dot over 512 MB)."""
    key = ("gemv", M)
    if key not in _CEILINGS:
        import torch

        K = N = 16384
        w = torch.empty(K, N, device="cuda", dtype=torch.float16).normal_()
        a = torch.empty(M, K, device="cuda", dtype=torch.float16).normal_()
        ms = _event_ms(lambda: a @ w, 20)
        _CEILINGS[key] = K * N * 2 / (ms * 1e-3) / 1e9
        del w, a
    return _CEILINGS[key]


def roofline_for(res, bound=None):
    """Roofline of the dominant kernel (the longer of the two expert-GEMM kernels),
    its duration from the dispatch-stamped events of time_kernel.  bound None:
    HBM for the decode form, MFMA for the prefill form."""
    k = "gate_up" if res["gate_up"]["us"] >= res["down"]["us"] else "down"
    if bound is None:
        bound = "hbm" if res[k]["kernel"] == "gemv_kernel" else "mfma"
    d = res[k]
    sec = d["us"] * 1e-6
    name = f"{d['kernel']} ({k}, {res['wfmt']}, T={res['tokens']})"
    row = counter_table().get(f"{res['probe']}:{res['tokens']}:{k}", {})
    traffic = row.get("traffic")
    if bound == "hbm":
        achieved = d["bytes"] / sec / 1e9
        copy = vendor_copy_gbps()
        read = vendor_gemv_gbps(max(1, min(res["tokens"], 64)))
        return dict(kernel=name, bound="hbm", achieved=round(achieved, 1),
                    peak=HBM_PEAK / 1e9, unit="GB/s", frac=round(achieved * 1e9 / HBM_PEAK, 4),
                    traffic=traffic, algorithmic_bytes_per_launch=round(d["bytes"]),
                    us_per_launch=round(d["us"], 2),
                    vendor_gemv=dict(GBps=round(read, 1), frac_of_peak=round(read * 1e9 / HBM_PEAK, 4),
                                     kernel_frac_of_vendor=round(achieved / read, 4),
                                     what=f"torch.matmul [{max(1, min(res['tokens'], 64))}, 16384] x [16384, 16384] "
                                          "fp16, weight bytes read / s"),
                    vendor_copy=dict(GBps=round(copy, 1), frac_of_peak=round(copy * 1e9 / HBM_PEAK, 4),
                                     kernel_frac_of_copy=round(achieved / copy, 4),
                                     what="256 MB device copy, bytes read + written / s"))
    peak = MFMA_F32_PEAK if res["wfmt"] == "f32" else MFMA_BF16_PEAK
    achieved = d["flops"] / sec / 1e12
    out = dict(kernel=name, bound="mfma", achieved=round(achieved, 1),
               peak=peak / 1e12, unit="TFLOP/s", frac=round(achieved * 1e12 / peak, 4),
               traffic=traffic, algorithmic_flops_per_launch=d["flops"], us_per_launch=round(d["us"], 2))
    if row.get("mfma_util") is not None:
        out["mfma_busy_pct_counters"] = row["mfma_util"]
    sh = res.get("shape")
    if sh and res["wfmt"] != "f32":
        # the same multiply-adds as one dense fp16 GEMM: M = T k (token, expert) pairs
        M = res["tokens"] * sh["k"]
        N, K = (2 * sh["I"], sh["H"]) if k == "gate_up" else (sh["H"], sh["I"])
        lib = vendor_gemm_tflops(M, N, K)
        out["vendor_gemm"] = dict(shape_mnk=[M, N, K], TFLOPs=round(lib, 1),
                                  frac_of_peak=round(lib * 1e12 / peak, 4),
                                  kernel_frac_of_vendor=round(achieved / lib, 4))
    return out


# --------------------------------------------------------------------- CPU baseline
def host_info():
    """Host identification for the CPU baseline: cores visible, cores this
    process may run on, the CPU model, whether kt-kernel is importable."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        affinity = os.cpu_count()
    try:
        import kt_kernel  # noqa: F401
        kt = "installed (not timed: its AMX/AVX-512 engine is not this path's restatement)"
    except ImportError:
        kt = "not installed"
    return dict(os_cpu_count=os.cpu_count(), affinity_cores=affinity, cpu_model=model, kt_kernel=kt)


def cpu_baseline(w, T, src, x, logits, sample=None, budget_s=8.0):
    """The reference CPU expert loop (oracle/cpu_loop.py: the torch restatement of
    nano_ktrans/kernels/cpu_moe.py:491-539 with quantized_ops.py:86-124, dense
    fp32 experts through linear) on this host's cores, torch threads = the cores
    this process may run on (os.cpu_count() on a shared host counts cores it does
    not own).  The same expert weights as the GPU run (its quantized codes and
    bf16 scales, copied back) and its first seeded input; sample: that many
    leading tokens of it (None: all).  Warm-up 3, then up to 10 timed calls
    (fewer once budget_s is spent), median and min."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cpu_loop as C
    import oracle as O

    info = host_info()
    threads = info["affinity_cores"]
    torch.set_num_threads(threads)
    n = T if sample is None else min(sample, T)
    xs = x[:n].float().cpu().numpy()
    lg = logits[:n].float().cpu().numpy()
    ids, wts = O.route(lg, w.k, w.softmax, w.renorm, w.act == "bf16")
    active = sorted(set(ids.ravel().tolist()))

    def conv(t):
        if hasattr(t, "qweight"):
            return O.QWeight(t.qweight.numpy(), t.scales.numpy().astype(np.float32), t.bits, t.group_size)
        return t.numpy().astype(np.float32)

    experts = [None] * w.E
    for e in active:
        d = src["experts"][e]
        experts[e] = C.to_torch_expert(O.Expert(conv(d["gate"]), conv(d["up"]), conv(d["down"])))
    shared = None
    if src["shared"] is not None:
        d = src["shared"]
        shared = C.to_torch_expert(O.Expert(conv(d["gate"]), conv(d["up"]), conv(d["down"])))
        sg = src["shared_gate"].float()

    def call():
        out = C.moe_loop(xs, ids, wts, experts)
        if shared is not None:
            xt = torch.from_numpy(xs)
            out = out + (torch.sigmoid(xt @ sg)[:, None] * C.expert_gptq(xt, shared)).numpy()
        return out

    with torch.no_grad():
        for _ in range(3):
            call()
        times = []
        start = time.perf_counter()
        while len(times) < 10 and (len(times) < 3 or time.perf_counter() - start < budget_s):
            t0 = time.perf_counter()
            call()
            times.append(time.perf_counter() - t0)
    med, mn = float(np.median(times)), float(min(times))
    what = f"{n} of the {T} tokens" if n < T else f"all {T} tokens"
    return dict(workload=w.name, tokens=T, value=round(n / med, 3), unit="tokens/s", cores=torch.get_num_threads(),
                kind="port", median_s=round(med, 5), min_s=round(mn, 5), best_tokens_per_s=round(n / mn, 3),
                warmup=3, repeats=len(times), torch_threads=torch.get_num_threads(), **info,
                sample=f"{what} of the bench's first seeded input ({len(active)} active experts), the GPU run's "
                       f"own expert weights; oracle/cpu_loop.py (torch restatement of the reference's CPU GPTQ "
                       f"loop, dense fp32 experts by linear), warm-up 3, {len(times)} timed calls")


# --------------------------------------------------------------------- counters (rocprofv3 --pmc on nkt_probe)
PMC_COPY_BYTES = 256 << 20   # nkt_probe's calibration kernel reads and writes this many bytes
SIMD_NUM = 1024              # 256 CUs x 4 SIMDs


def _pmc_rows(path):
    """{(kernel name, grid size): {counter: mean value per dispatch}} of a rocprofv3
    counter-collection CSV (a counter's rows of one dispatch summed)."""
    import collections
    import csv

    per_dispatch = collections.defaultdict(float)
    for r in csv.DictReader(open(path)):
        per_dispatch[(r["Kernel_Name"], r.get("Grid_Size", ""), r.get("Dispatch_Id", ""), r["Counter_Name"])] += \
            float(r["Counter_Value"])
    acc = collections.defaultdict(lambda: collections.defaultdict(list))
    for (name, grid, _, counter), v in per_dispatch.items():
        acc[(name, grid)][counter].append(v)
    return {k: {c: sum(v) / len(v) for c, v in d.items()} for k, d in acc.items()}


def _phase_of(name):
    """gate_up / down from an expert-GEMM kernel's template arguments (None otherwise)."""
    import re

    m = re.search(r"nkt::(gemv_kernel|gemm2_kernel|gemm_kernel|gemm2_i8_kernel|gemm2_i4_kernel)<([^>]*)>", name)
    if not m:
        return None
    args = [a.strip() for a in m.group(2).split(",")]
    # template arguments: gemv_kernel<WF, PHASE, ...>, gemm2_kernel<WF, PHASE, NW>,
    # gemm_kernel<WF, BM, NW, RT, PHASE, ...>, gemm2_i8_kernel<PHASE, F16>, gemm2_i4_kernel<PHASE, NARROW>
    idx = {"gemm2_i8_kernel": 0, "gemm2_i4_kernel": 0, "gemm_kernel": 4}.get(m.group(1), 1)
    val = args[idx].split(")")[-1]
    return "gate_up" if val == "0" else "down"


def summarize_pmc(probe, tokens, fetch_csv, write_csv, mfma_csv):
    """Markdown rows for one nkt_probe workload: HBM bytes per launch of each
    expert-GEMM kernel from FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each
    scaled by the factor that makes the calibration kernel read / write
    PMC_COPY_BYTES, plus MFMA busy % (MfmaUtil) and matrix-core flops per
    launch (MfmaFlopsBF16 + MfmaFlopsF16) from a third run.  Of two launches of
    one kernel with different grids (Qwen1.5: routed experts and the shared
    expert), the larger grid is the routed one."""
    fetch, write, mfma = _pmc_rows(fetch_csv), _pmc_rows(write_csv), _pmc_rows(mfma_csv)

    def calib(d, counter):
        cal = [v[counter] for (n, _), v in d.items() if "neg_kernel" in n and counter in v]
        if not cal:
            raise SystemExit(f"no calibration kernel in the {counter} counters")
        return PMC_COPY_BYTES / (cal[0] * 1024.0), cal[0]

    ff, fraw = calib(fetch, "FETCH_SIZE")
    wf, wraw = calib(write, "WRITE_SIZE")
    print(f"{probe} T={tokens}: calibration (fp32 negate, {PMC_COPY_BYTES} B in and out): FETCH_SIZE {fraw:.0f} KiB "
          f"-> factor {ff:.4f}; WRITE_SIZE {wraw:.0f} KiB -> factor {wf:.4f}\n")
    kernels = sorted({k for k in fetch if _phase_of(k[0])}, key=lambda k: (_phase_of(k[0]), -int(k[1] or 0)))
    seen = set()
    for name, grid in kernels:
        phase = _phase_of(name)
        role = phase if phase not in seen else "shared_" + phase
        seen.add(phase)
        f = fetch[(name, grid)].get("FETCH_SIZE", 0.0)
        w = write.get((name, grid), {}).get("WRITE_SIZE", 0.0)
        m = mfma.get((name, grid), {})
        rd, wr = f * 1024.0 * ff, w * 1024.0 * wf
        util = m.get("MfmaUtil")
        flops = (m.get("MfmaFlopsBF16", 0.0) + m.get("MfmaFlopsF16", 0.0)) / 1e9 if m else None
        valu_per_mfma = (m["SQ_INSTS_VALU"] - m["SQ_INSTS_MFMA"]) / m["SQ_INSTS_MFMA"] \
            if m.get("SQ_INSTS_MFMA") else None
        short = name.split("(")[0].replace("void ", "")
        print(f"| `{probe}:{tokens}:{role}` | `{short}` | {grid} | {rd:.0f} | {wr:.0f} | {rd + wr:.0f} | "
              f"{'-' if util is None else f'{util:.2f}'} | {'-' if flops is None else f'{flops:.2f}'} | "
              f"{'-' if valu_per_mfma is None else f'{valu_per_mfma:.2f}'} |")


def summarize_trace(trace_csv):
    """Markdown table of the nkt kernels in a rocprofv3 kernel-trace CSV, grouped by
    kernel and launch grid (workgroups in x, y): durations End - Start."""
    import collections
    import csv
    import statistics

    d = collections.defaultdict(list)
    meta = {}
    for r in csv.DictReader(open(trace_csv)):
        n = r["Kernel_Name"]
        if "nkt::" not in n:
            continue
        name = n.split("(")[0].replace("void ", "")
        key = (name, int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]), int(r["Grid_Size_Y"]))
        d[key].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        meta[key] = (r["VGPR_Count"], r["Accum_VGPR_Count"], r["LDS_Block_Size"], r["Scratch_Size"],
                     r["Workgroup_Size_X"])
    print("| kernel | grid (x, y) | wg | calls | avg us | median us | min us | vgpr/agpr | lds B | scratch |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for k, v in sorted(d.items()):
        m = meta[k]
        print(f"| `{k[0]}` | {k[1]}, {k[2]} | {m[4]} | {len(v)} | {statistics.mean(v) / 1e3:.2f} | "
              f"{statistics.median(v) / 1e3:.2f} | {min(v) / 1e3:.2f} | {m[0]}/{m[1]} | {m[2]} | {m[3]} |")


# --------------------------------------------------------------------- main
def _slim(r):
    keep = ("workload", "tokens", "us_per_layer", "tokens_per_s", "steps", "warmup", "mean_active_experts",
            "breakdown_us", "roofline", "roofline_alt", "layer_hbm_frac")
    return {k: v for k, v in r.items() if k in keep}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--tokens", type=int, default=16)
    ap.add_argument("--layers", type=int, default=8, help="distinct weight copies rotated per step")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--summarize-pmc", nargs=5, metavar=("PROBE", "TOKENS", "FETCH_CSV", "WRITE_CSV", "MFMA_CSV"),
                    help="print counter rows for one nkt_probe workload from three rocprofv3 --pmc CSVs")
    ap.add_argument("--summarize-trace", metavar="TRACE_CSV",
                    help="print the nkt kernels of a rocprofv3 kernel-trace CSV as a markdown table")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (the MoE path here has no multi-GPU build); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs the MI355X GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    do_cpu = not args.no_cpu_baseline
    cpu_all = []
    head = Workload("qwen3_30b_a3b_moe_layer_int4_g128_decode", tokens=args.tokens, **QWEN3_INT4)
    log(f"building {args.layers} copies of the int4 layer")
    router, layers, src = make_layers(head, args.layers, dev, max_tokens=max(args.tokens, 16))
    log(f"headline: {head.name} T={args.tokens}")
    res = bench_workload(head, args.tokens, layers, router, args.steps, args.warmup, dev)
    head_inputs = res.pop("inputs")
    log(json.dumps({k: v for k, v in res.items()}))
    secondary = []
    head_small = {}
    if not args.no_secondary:
        for T in (1, 4):
            log(f"secondary: {head.name} T={T}")
            r = bench_workload(head, T, layers, router, args.steps, args.warmup, dev)
            head_small[T] = tuple(t.cpu() for t in r.pop("inputs"))
            r["roofline"] = roofline_for(r, "hbm")
            log(json.dumps(r))
            secondary.append(r)
        # the layer from hidden states: the router GEMV [E, H] inside the path
        gate = router.to(torch.bfloat16)
        for layer in layers:
            layer.load_router(gate)
        T = args.tokens
        xs, _ = make_inputs(head, router, T, 8, dev)
        outs = [torch.empty(T, head.H, dtype=torch.bfloat16, device=dev) for _ in layers]
        ms = time_graph_hidden(layers, xs, outs, args.steps, args.warmup)
        r = dict(workload=head.name + "_fused_router", tokens=T, us_per_layer=ms * 1e3,
                 tokens_per_s=T / (ms * 1e-3), steps=args.steps, warmup=args.warmup)
        log(json.dumps(r))
        secondary.append(r)
        # the decoder layer's MoE half: residual + MoE(RMSNorm(hidden)), router inside
        norm_w = (1.0 + 0.1 * torch.randn(head.H, generator=torch.Generator().manual_seed(3))).to(dev)
        fwd = lambda layer, x, out: layer.forward_block(x, norm_w, 1e-6, out=out)
        ms = time_graph_hidden(layers, xs, outs, args.steps, args.warmup, call=fwd)
        r = dict(workload=head.name + "_decoder_block", tokens=T, us_per_layer=ms * 1e3,
                 tokens_per_s=T / (ms * 1e-3), steps=args.steps, warmup=args.warmup)
        log(json.dumps(r))
        secondary.append(r)
    del layers
    torch.cuda.empty_cache()
    cpu = None
    if do_cpu:
        log(f"cpu baseline: {head.name} T={args.tokens}")
        cpu = cpu_baseline(head, args.tokens, src, *head_inputs)
        log(json.dumps(cpu))
        cpu_all.append(cpu)
        for T, inp in head_small.items():
            log(f"cpu baseline: {head.name} T={T}")
            c = cpu_baseline(head, T, src, *inp)
            log(json.dumps(c))
            cpu_all.append(c)
    del src
    if not args.no_secondary:
        # the other configurations: (workload, weight copies, [(T, steps, warmup, bounds)],
        # [(T, CPU sample tokens or None)]); bounds: the roofline(s) reported, at the ridge both
        plan = [
            (Workload("tiny_mixtral_moe_layer_fp32", tokens=16, **TINY_F32), 8,
             [(16, 200, 20, ("hbm",))], [(16, None)]),
            (Workload("qwen3_30b_a3b_moe_layer_int8_pc_prefill_zipf", tokens=4096, **QWEN3_INT8), 2,
             [(4096, 20, 4, ("mfma",)), (512, 100, 10, ("mfma", "hbm")), (2048, 40, 6, ("mfma", "hbm"))],
             [(512, None), (2048, None), (4096, None)]),
            (Workload("mixtral_8x7b_moe_layer_int4_g128", tokens=16, **MIXTRAL_INT4), 4,
             [(1, 200, 20, ("hbm",)), (16, 200, 20, ("hbm",)), (2048, 20, 4, ("mfma",))],
             [(1, None), (16, None), (2048, 512)]),
            (Workload("qwen15_moe_a27b_layer_int8_pc_shared", tokens=16, **QWEN15_INT8), 4,
             [(1, 200, 20, ("hbm",)), (16, 200, 20, ("hbm",)), (1024, 40, 6, ("hbm", "mfma"))],
             [(1, None), (16, None), (1024, None)]),
        ]
        for w, copies, runs, cpu_runs in plan:
            max_t = max(T for T, *_ in runs)
            log(f"secondary: building {copies} copies of {w.name}")
            rtr, lays, wsrc = make_layers(w, copies, dev, max_tokens=max_t)
            inputs = {}
            for T, steps, warm, bounds in runs:
                log(f"secondary: {w.name} T={T}")
                r = bench_workload(w, T, lays, rtr, steps, warm, dev)
                inputs[T] = tuple(t.cpu() for t in r.pop("inputs"))
                r["roofline"] = roofline_for(r, bounds[0])
                if len(bounds) > 1:
                    r["roofline_alt"] = roofline_for(r, bounds[1])
                log(json.dumps(r))
                secondary.append(r)
            del lays
            torch.cuda.empty_cache()
            if do_cpu:
                for T, sample in cpu_runs:
                    log(f"cpu baseline: {w.name} T={T} sample={sample}")
                    c = cpu_baseline(w, T, wsrc, *inputs[T], sample=sample)
                    log(json.dumps(c))
                    cpu_all.append(c)
            del wsrc
    line = {
        "metric": METRIC,
        "value": round(res["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": head.name, "tokens": args.tokens, "hidden": head.H, "experts": head.E,
                   "top_k": head.k, "moe_intermediate": head.I, "weights": "int4 group-128, bf16 scales",
                   "weight_copies_rotated": args.layers, "parallelism": "single GPU"},
        "us_per_layer": round(res["us_per_layer"], 2),
        "mean_active_experts": res["mean_active_experts"],
        "layer_hbm_frac": round(res["layer_hbm_frac"], 4),
        "breakdown_us": {k: round(v, 2) for k, v in res["breakdown_us"].items()},
        "roofline": roofline_for(res, "hbm"),
        "cpu_baseline": cpu,
        "cpu_baselines": cpu_all,
        "secondary": [_slim(r) for r in secondary],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
