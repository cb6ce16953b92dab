#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X.

Headline workload: one Qwen3-30B-A3B-shaped MoE layer (H=2048, 128 experts,
top-8, moe_intermediate=768, int4 group-128 weights with bf16 scales, bf16
activations) decoding 16 tokens.  A step is one layer forward (route, group,
gate_up GEMM + SwiGLU, down GEMM, combine) on a new weight copy: steps rotate
over --layers distinct copies of the layer (> 2 GB in total, beyond the 256 MB
last-level cache) and over 8 seeded inputs, the way consecutive layers of a
model would stream their weights from HBM.  Steps are replayed from a HIP graph
(one graph = one pass over the layer copies), timed with HIP events between
device synchronisations.

Printed JSON fields beyond the standard ones:
  us_per_layer   layer latency
  breakdown_us   per-stage device time from HIP events (eager, the host kept ahead)
  roofline       dominant kernel: algorithmic bytes (active experts' codes + scales,
                 activations in/out) / its average event-timed duration vs 8 TB/s
  cpu_baseline   the oracle's restatement of the reference CPU expert loop
                 (nano_ktrans/kernels/cpu_moe.py:491-539), timed on this host
  secondary      other token counts (T=1, 4), the layer from hidden states
                 (router GEMV fused; plus RMSNorm and residual), the int8
                 per-channel prefill at T=512/2048/4096 (Zipf-skewed routing),
                 a Mixtral-8x7B-shaped int4 layer (T=1, 16, 2048) and a
                 Qwen1.5-MoE-shaped int8 layer with its shared expert (T=1, 16,
                 1024); roofline_alt gives the other bound's fraction where a
                 shape sits near the ridge
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nano-ktrans_amd"))

HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
MFMA_BF16_PEAK = 2.5e15    # FLOP/s, dense bf16

METRIC = "MoE-layer tokens/s + decode µs/layer (Qwen3-30B-A3B shape); % HBM/MFMA roofline"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --------------------------------------------------------------------- problem
class Workload:
    def __init__(self, name, H, E, k, I, wfmt, softmax, renorm, tokens, zipf=0.0, seed=1, shared=0):
        self.name, self.H, self.E, self.k, self.I = name, H, E, k, I
        self.wfmt, self.softmax, self.renorm, self.tokens, self.zipf, self.seed = wfmt, softmax, renorm, tokens, zipf, seed
        self.shared = shared  # shared-expert intermediate size (0: none)

    def _bytes(self, n, kk):
        if self.wfmt == "int4_g128":
            return n * kk // 2 + n * (kk // 128) * 2
        if self.wfmt == "int8_per_channel":
            return n * kk + n * 2
        return n * kk * 2

    def bytes_per_expert(self, proj):
        n, kk = (2 * self.I, self.H) if proj == "gate_up" else (self.H, self.I)
        return self._bytes(n, kk)

    def shared_bytes(self):
        """Shared expert (gate_up + down) plus its gate vector, read once per layer call."""
        if not self.shared:
            return 0
        return self._bytes(2 * self.shared, self.H) + self._bytes(self.H, self.shared) + self.H * 2


QWEN3_INT4 = dict(H=2048, E=128, k=8, I=768, wfmt="int4_g128", softmax=True, renorm=True, seed=1)
QWEN3_INT8 = dict(H=2048, E=128, k=8, I=768, wfmt="int8_per_channel", softmax=True, renorm=True, seed=1, zipf=1.1)
# Mixtral-8x7B-shaped layer (top-k on the logits, then softmax over the k) and
# Qwen1.5-MoE-A2.7B-shaped layer (60 experts, softmax without renormalisation,
# shared expert with a sigmoid gate)
MIXTRAL_INT4 = dict(H=4096, E=8, k=2, I=14336, wfmt="int4_g128", softmax=False, renorm=False, seed=2)
QWEN15_INT8 = dict(H=2048, E=60, k=4, I=1408, wfmt="int8_per_channel", softmax=True, renorm=False, seed=3,
                   shared=5632)


def make_layers(w, n_layers, device, max_tokens):
    """One seeded layer quantized on the GPU, then n_layers distinct device copies."""
    import torch
    from nano_ktrans_amd.kernels.quantized_ops import (quantize_symmetric_int8_per_channel,
                                                       quantize_symmetric_w4a32)
    from nano_ktrans_amd.native_moe import NativeMoE

    quant = (lambda t: quantize_symmetric_w4a32(t, group_size=128)) if w.wfmt == "int4_g128" \
        else quantize_symmetric_int8_per_channel
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    router = torch.randn(w.E, w.H, generator=g, device=device) * 0.02
    layers = []
    first = NativeMoE(num_experts=w.E, top_k=w.k, hidden_size=w.H, intermediate_size=w.I,
                      shared_intermediate_size=w.shared, weight_format=w.wfmt, act_dtype=torch.bfloat16,
                      use_softmax=w.softmax, renorm=w.renorm, max_tokens=max_tokens, device=device)
    for e in range(w.E):
        gate_up = torch.randn(2 * w.I, w.H, generator=g, device=device) * 0.02
        down = torch.randn(w.H, w.I, generator=g, device=device) * 0.02
        first.load_expert(e, quant(gate_up[: w.I]), quant(gate_up[w.I:]), quant(down))
        del gate_up, down
    if w.shared:
        gs = torch.randn(2 * w.shared, w.H, generator=g, device=device) * 0.02
        ds = torch.randn(w.H, w.shared, generator=g, device=device) * 0.02
        gw = torch.randn(1, w.H, generator=g, device=device) * 0.02
        first.load_shared_expert(quant(gs[: w.shared]), quant(gs[w.shared:]), quant(ds), gw)
        del gs, ds
    layers.append(first)
    for _ in range(1, n_layers):
        n = NativeMoE(num_experts=w.E, top_k=w.k, hidden_size=w.H, intermediate_size=w.I,
                      shared_intermediate_size=w.shared, weight_format=w.wfmt, act_dtype=torch.bfloat16,
                      use_softmax=w.softmax, renorm=w.renorm, max_tokens=max_tokens, device=device)
        for slot, t in first.slots.items():
            n.slots[slot].copy_(t)
        layers.append(n)
    torch.cuda.synchronize()
    return router, layers


def make_inputs(w, router, T, n_inputs, device):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(1000 + T)
    xs, ls = [], []
    for _ in range(n_inputs):
        x = torch.randn(T, w.H, generator=g, device=device).to(torch.bfloat16)
        logits = x.float() @ router.T
        if w.zipf:
            e = torch.arange(w.E, device=device, dtype=torch.float32)
            logits = logits - w.zipf * torch.log(e + 1.0)
        xs.append(x)
        ls.append(logits.to(torch.bfloat16))
    return xs, ls


def active_experts(layer, logits):
    import torch

    ids = layer.route(logits)[0]
    return int(torch.unique(ids).numel())


# --------------------------------------------------------------------- timing
def time_graph(layers, xs, ls, outs, steps, warmup):
    """Replay a graph of one forward per layer copy; returns ms per layer step."""
    import torch

    L = len(layers)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i, layer in enumerate(layers):  # warm the workspaces before capture
            layer.forward(xs[i % len(xs)], ls[i % len(ls)], out=outs[i])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i, layer in enumerate(layers):
            layer.forward(xs[i % len(xs)], ls[i % len(ls)], out=outs[i])
    reps_warm = max(1, (warmup + L - 1) // L)
    reps = max(1, (steps + L - 1) // L)
    for _ in range(reps_warm):
        graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1)
    return ms / (reps * L), reps * L


def time_graph_hidden(layers, xs, outs, steps, warmup, call=None):
    """time_graph for the layer from hidden states alone (router GEMV fused; or
    call(layer, x, out)): ms per layer step."""
    import torch

    if call is None:
        call = lambda layer, x, out: layer.forward_hidden(x, out=out)
    L = len(layers)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i, layer in enumerate(layers):
            call(layer, xs[i % len(xs)], outs[i])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i, layer in enumerate(layers):
            call(layer, xs[i % len(xs)], outs[i])
    for _ in range(max(1, (warmup + L - 1) // L)):
        graph.replay()
    torch.cuda.synchronize()
    reps = max(1, (steps + L - 1) // L)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / (reps * L)


def time_stages(layers, xs, ls, outs, rounds):
    """Per-stage device time with HIP events; a sleep kernel keeps the host ahead."""
    import torch

    names = ["route+group", "gate_up", "down", "combine"]
    acc = {n: 0.0 for n in names}
    count = 0
    stream = torch.cuda.current_stream()
    for r in range(rounds):
        try:
            torch.cuda._sleep(50_000_000)  # keep the device busy while the host enqueues
        except Exception:
            pass
        evs = []
        for i, layer in enumerate(layers):
            x, lg = xs[i % len(xs)], ls[i % len(ls)]
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
    1: down).  Every layer copy is routed (and its gate_up run) first; then each
    launch of the phase carries its own pair of HIP events, stamped by the
    dispatch at the kernel's start and end (nkt_moe_experts_phase_timed), on the
    stream the kernel runs on.  A sleep kernel keeps the host ahead so the
    launches run back to back over the rotating weight copies."""
    import torch

    T = xs[0].shape[0]
    for i, layer in enumerate(layers):
        layer.route(ls[i % len(ls)])
        layer.expert_phase(0, xs[i % len(xs)], T)
    torch.cuda.synchronize()
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
    for _ in range(passes):
        for i, layer in enumerate(layers):
            a, b = pairs[n]
            layer.expert_phase_timed(phase, xs[i % len(xs)] if phase == 0 else None, T, a, b)
            n += 1
    torch.cuda.synchronize()
    times = [a.elapsed_time(b) * 1e3 for a, b in pairs]
    return sum(times) / len(times)


def kernel_form(w, T):
    """Which K3 kernel the library runs for this shape (mirrors gemm_tile_m)."""
    avg = T * w.k / w.E
    if avg <= 12:
        return "gemv_kernel"
    if w.wfmt == "f32":
        return "gemm_kernel"
    # int8 and int4 (bf16 activations, buffers under 4 GiB: every bench shape) have pipelined kernels
    return {"int8_per_channel": "gemm2_i8_kernel", "int4_g128": "gemm2_i4_kernel"}.get(w.wfmt, "gemm2_kernel")


def bench_workload(w, T, layers, router, steps, warmup, device):
    import torch

    xs, ls = make_inputs(w, router, T, 8, device)
    outs = [torch.empty(T, w.H, dtype=torch.bfloat16, device=device) for _ in layers]
    n_act = [active_experts(layers[0], l) for l in ls]
    mean_act = sum(n_act) / len(n_act)
    ms, timed = time_graph(layers, xs, ls, outs, steps, warmup)
    stages = time_stages(layers, xs, ls, outs, rounds=3)
    gate_up_us = time_kernel(layers, xs, ls, 0)
    down_us = time_kernel(layers, xs, ls, 1)
    P = T * w.k
    gate_up_bytes = mean_act * w.bytes_per_expert("gate_up") + T * w.H * 2 + P * w.I * 2
    down_bytes = mean_act * w.bytes_per_expert("down") + P * w.I * 2 + P * w.H * 4
    layer_bytes = (mean_act * (w.bytes_per_expert("gate_up") + w.bytes_per_expert("down"))
                   + w.shared_bytes() + T * w.H * 2 * 2 + T * w.E * 2)
    gate_up_flops = 2.0 * P * 2 * w.I * w.H
    down_flops = 2.0 * P * w.H * w.I
    form = kernel_form(w, T)
    return dict(workload=w.name, wfmt=w.wfmt, tokens=T, ms_per_step=ms, us_per_layer=ms * 1e3, steps=timed,
                tokens_per_s=T / (ms * 1e-3), mean_active_experts=mean_act, breakdown_us=stages,
                layer_bytes=layer_bytes, layer_hbm_frac=layer_bytes / (ms * 1e-3) / HBM_PEAK,
                gate_up=dict(kernel=form, bytes=gate_up_bytes, flops=gate_up_flops, us=gate_up_us),
                down=dict(kernel=form, bytes=down_bytes, flops=down_flops, us=down_us))


def traffic_table():
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE),
    calibrated on a copy kernel, from profiles/pmc_traffic_moe_layer.md (None if absent)."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic_moe_layer.md")
    try:
        text = open(path).read()
    except OSError:
        return {}
    out = {}
    for line in text.splitlines():
        # | key | fetch bytes | write bytes | traffic bytes | ...
        if line.startswith("| `traffic:"):
            cells = [c.strip() for c in line.strip("|").split("|")]
            try:
                out[cells[0].strip("`")[len("traffic:"):]] = float(cells[3])
            except (ValueError, IndexError):
                pass
    return out


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
    traffic = traffic_table().get(f"{d['kernel']}:{k}:{res['wfmt']}:{res['tokens']}")
    if bound == "hbm":
        achieved = d["bytes"] / sec / 1e9
        return dict(kernel=name, bound="hbm", achieved=round(achieved, 1),
                    peak=HBM_PEAK / 1e9, unit="GB/s", frac=round(achieved * 1e9 / HBM_PEAK, 4),
                    traffic=traffic, algorithmic_bytes_per_launch=round(d["bytes"]),
                    us_per_launch=round(d["us"], 2))
    achieved = d["flops"] / sec / 1e12
    return dict(kernel=name, bound="mfma", achieved=round(achieved, 1),
                peak=MFMA_BF16_PEAK / 1e12, unit="TFLOP/s", frac=round(achieved * 1e12 / MFMA_BF16_PEAK, 4),
                traffic=traffic, algorithmic_flops_per_launch=d["flops"], us_per_launch=round(d["us"], 2))


# --------------------------------------------------------------------- CPU baseline
def cpu_baseline(w, T, budget_s=15.0):
    """The oracle's fp32 restatement of the reference CPU expert loop on one input."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    from nano_ktrans_amd.kernels.quantized_ops import quantize_symmetric_w4a32, to_bf16_scales

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    g = torch.Generator().manual_seed(w.seed)
    router = torch.randn(w.E, w.H, generator=g) * 0.02
    x = torch.randn(T, w.H, generator=g).to(torch.bfloat16)
    logits = (x.float() @ router.T).to(torch.bfloat16)
    ids, _ = O.route(logits.float().numpy(), w.k, w.softmax, w.renorm, True)
    active = sorted(set(ids.ravel().tolist()))
    experts = [None] * w.E
    for e in active:
        gu = torch.randn(2 * w.I, w.H, generator=g) * 0.02
        dn = torch.randn(w.H, w.I, generator=g) * 0.02
        q = lambda t: to_bf16_scales(quantize_symmetric_w4a32(t, group_size=128))
        conv = lambda qw: O.QWeight(qw.qweight.numpy(), qw.scales.numpy(), 4, 128)
        experts[e] = O.Expert(conv(q(gu[: w.I])), conv(q(gu[w.I:])), conv(q(dn)))
    xs = x.float().numpy()
    lg = logits.float().numpy()
    times = []
    ctx = threadpool_limits(limits=1) if threadpool_limits else None
    try:
        if ctx:
            ctx.__enter__()
        start = time.perf_counter()
        while True:
            t0 = time.perf_counter()
            O.moe_forward(xs, lg, experts, w.k, w.softmax, w.renorm, True)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - start > budget_s or len(times) >= 10:
                break
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    sec = float(np.median(times))
    return dict(value=round(T / sec, 3), unit="tokens/s", cores=1, kind="port",
                sample=f"{len(times)} layer calls of {T} tokens ({len(active)} active experts), median "
                       f"{sec * 1e3:.0f} ms; numpy fp32 grouped-matvec loop, BLAS limited to 1 thread")


# --------------------------------------------------------------------- HBM traffic (rocprofv3 --pmc)
PMC_COPY_BYTES = 256 << 20   # the calibration kernel reads and writes this many bytes
PMC_KERNELS = {  # kernel-name prefix -> traffic key (kernel:phase:weights:tokens) of the probe's launches
    "nkt::gemv_kernel<3, 0,": "gemv_kernel:gate_up:int4_g128:16",
    "nkt::gemv_kernel<3, 1,": "gemv_kernel:down:int4_g128:16",
}


def pmc_probe():
    """Launches for a counter run (counters restricted to these kernels with
    --kernel-include-regex): a calibration kernel of known traffic (fp32 negate,
    PMC_COPY_BYTES in and out), then route + both expert GEMMs of the headline
    decode (int4, T=16, 8 weight copies)."""
    import torch

    dev = torch.device("cuda", 0)
    a = torch.ones(PMC_COPY_BYTES // 4, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    del a, b
    for w, copies in ((Workload("decode", tokens=16, **QWEN3_INT4), 8),):
        log(f"pmc probe: {w.wfmt} T={w.tokens}")
        router, layers = make_layers(w, copies, dev, max_tokens=w.tokens)
        xs, ls = make_inputs(w, router, w.tokens, 8, dev)
        for _ in range(2):
            for i, layer in enumerate(layers):
                layer.route(ls[i % len(ls)])
                layer.expert_phase(0, xs[i % len(xs)], w.tokens)
                layer.expert_phase(1, None, w.tokens)
        torch.cuda.synchronize()
        del layers
        torch.cuda.empty_cache()
    log("pmc probe done")


def _pmc_per_kernel(path, counter):
    """Mean per-dispatch value of one counter for every kernel name in a rocprofv3 counter CSV."""
    import collections
    import csv

    per_dispatch = collections.defaultdict(float)
    for r in csv.DictReader(open(path)):
        if r.get("Counter_Name") != counter:
            continue
        per_dispatch[(r["Kernel_Name"], r.get("Dispatch_Id", ""))] += float(r["Counter_Value"])
    by_name = collections.defaultdict(list)
    for (name, _), v in per_dispatch.items():
        by_name[name].append(v)
    return {name: sum(v) / len(v) for name, v in by_name.items()}


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


def summarize_pmc(fetch_csv, write_csv):
    """Markdown rows of HBM bytes per launch: FETCH_SIZE and WRITE_SIZE (KiB per dispatch),
    each scaled by the factor that makes the calibration kernel read / write PMC_COPY_BYTES."""
    fetch = _pmc_per_kernel(fetch_csv, "FETCH_SIZE")
    write = _pmc_per_kernel(write_csv, "WRITE_SIZE")

    def calib(d, what):
        cal = [v for n, v in d.items() if "neg_kernel" in n]
        if not cal:
            raise SystemExit(f"no calibration kernel in the {what} counters")
        return PMC_COPY_BYTES / (cal[0] * 1024.0), cal[0]

    ff, fraw = calib(fetch, "FETCH_SIZE")
    wf, wraw = calib(write, "WRITE_SIZE")
    print(f"calibration (fp32 negate, {PMC_COPY_BYTES} B in and out): FETCH_SIZE {fraw:.0f} KiB -> factor "
          f"{ff:.4f}; WRITE_SIZE {wraw:.0f} KiB -> factor {wf:.4f}\n")
    print("| key | HBM read B/launch | HBM write B/launch | traffic B/launch | FETCH_SIZE KiB | WRITE_SIZE KiB |")
    print("|---|---|---|---|---|---|")
    for prefix, key in PMC_KERNELS.items():
        fk = [v for n, v in fetch.items() if prefix in n]
        wk = [v for n, v in write.items() if prefix in n]
        if not fk or not wk:
            continue
        rd, wr = fk[0] * 1024.0 * ff, wk[0] * 1024.0 * wf
        print(f"| `traffic:{key}` | {rd:.0f} | {wr:.0f} | {rd + wr:.0f} | {fk[0]:.0f} | {wk[0]:.0f} |")


# --------------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--tokens", type=int, default=16)
    ap.add_argument("--layers", type=int, default=8, help="distinct weight copies rotated per step")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-probe", action="store_true", help="only the launches of a rocprofv3 --pmc run")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print HBM traffic per launch from two rocprofv3 --pmc counter CSVs")
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
    if args.pmc_probe:
        pmc_probe()
        return
    dev = torch.device("cuda", 0)
    head = Workload("qwen3_30b_a3b_moe_layer_int4_g128_decode", tokens=args.tokens, **QWEN3_INT4)
    log(f"building {args.layers} copies of the int4 layer")
    router, layers = make_layers(head, args.layers, dev, max_tokens=max(args.tokens, 16))
    log(f"headline: {head.name} T={args.tokens}")
    res = bench_workload(head, args.tokens, layers, router, args.steps, args.warmup, dev)
    log(json.dumps(res))
    secondary = []
    if not args.no_secondary:
        for T in (1, 4):
            log(f"secondary: {head.name} T={T}")
            r = bench_workload(head, T, layers, router, args.steps, args.warmup, dev)
            r["roofline"] = roofline_for(r, "hbm")
            log(json.dumps(r))
            secondary.append(r)
    if not args.no_secondary:
        # the layer from hidden states: router GEMV [E, H] fused into the routing launch
        gate = router.to(torch.bfloat16)
        for layer in layers:
            layer.load_router(gate)
        T = args.tokens
        xs, _ = make_inputs(head, router, T, 8, dev)
        outs = [torch.empty(T, head.H, dtype=torch.bfloat16, device=dev) for _ in layers]
        ms = time_graph_hidden(layers, xs, outs, args.steps, args.warmup)
        r = dict(workload=head.name + "_fused_router", tokens=T, us_per_layer=ms * 1e3,
                 tokens_per_s=T / (ms * 1e-3))
        log(json.dumps(r))
        secondary.append(r)
        # the decoder layer's MoE half: residual + MoE(RMSNorm(hidden)), router fused
        norm_w = (1.0 + 0.1 * torch.randn(head.H, generator=torch.Generator().manual_seed(3))).to(dev)
        fwd = lambda layer, x, out: layer.forward_block(x, norm_w, 1e-6, out=out)
        ms = time_graph_hidden(layers, xs, outs, args.steps, args.warmup, call=fwd)
        r = dict(workload=head.name + "_decoder_block", tokens=T, us_per_layer=ms * 1e3,
                 tokens_per_s=T / (ms * 1e-3))
        log(json.dumps(r))
        secondary.append(r)
    del layers
    torch.cuda.empty_cache()
    if not args.no_secondary:
        # prefill and the other model shapes: (workload, weight copies, [(T, steps, warmup, bounds)])
        # bounds: the roofline(s) reported; at the ridge both
        plan = [
            (Workload("qwen3_30b_a3b_moe_layer_int8_pc_prefill_zipf", tokens=4096, **QWEN3_INT8), 2,
             [(4096, 20, 4, ("mfma",)), (512, 100, 10, ("mfma", "hbm")), (2048, 40, 6, ("mfma", "hbm"))]),
            (Workload("mixtral_8x7b_moe_layer_int4_g128", tokens=16, **MIXTRAL_INT4), 4,
             [(1, 200, 20, ("hbm",)), (16, 200, 20, ("hbm",)), (2048, 20, 4, ("mfma",))]),
            (Workload("qwen15_moe_a27b_layer_int8_pc_shared", tokens=16, **QWEN15_INT8), 4,
             [(1, 200, 20, ("hbm",)), (16, 200, 20, ("hbm",)), (1024, 40, 6, ("hbm", "mfma"))]),
        ]
        for w, copies, runs in plan:
            max_t = max(T for T, *_ in runs)
            log(f"secondary: building {copies} copies of {w.name}")
            rtr, lays = make_layers(w, copies, dev, max_tokens=max_t)
            for T, steps, warm, bounds in runs:
                log(f"secondary: {w.name} T={T}")
                r = bench_workload(w, T, lays, rtr, steps, warm, dev)
                r["roofline"] = roofline_for(r, bounds[0])
                if len(bounds) > 1:
                    r["roofline_alt"] = roofline_for(r, bounds[1])
                log(json.dumps(r))
                secondary.append(r)
            del lays
            torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle port of the reference CPU loop)")
        cpu = cpu_baseline(head, args.tokens)
    line = {
        "metric": METRIC,
        "value": round(res["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": res["steps"],
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
        "secondary": [{k: v for k, v in r.items() if k in ("workload", "tokens", "us_per_layer", "tokens_per_s",
                                                           "mean_active_experts", "breakdown_us", "roofline",
                                                           "roofline_alt", "layer_hbm_frac")}
                      for r in secondary],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
