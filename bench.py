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
  secondary      other token counts and the int8 prefill configuration
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
    def __init__(self, name, H, E, k, I, wfmt, softmax, renorm, tokens, zipf=0.0, seed=1):
        self.name, self.H, self.E, self.k, self.I = name, H, E, k, I
        self.wfmt, self.softmax, self.renorm, self.tokens, self.zipf, self.seed = wfmt, softmax, renorm, tokens, zipf, seed

    def bytes_per_expert(self, proj):
        import math
        n, kk = (2 * self.I, self.H) if proj == "gate_up" else (self.H, self.I)
        if self.wfmt == "int4_g128":
            return n * kk // 2 + n * (kk // 128) * 2
        if self.wfmt == "int8_per_channel":
            return n * kk + n * 2
        return n * kk * 2


QWEN3_INT4 = dict(H=2048, E=128, k=8, I=768, wfmt="int4_g128", softmax=True, renorm=True, seed=1)
QWEN3_INT8 = dict(H=2048, E=128, k=8, I=768, wfmt="int8_per_channel", softmax=True, renorm=True, seed=1, zipf=1.1)


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
                      weight_format=w.wfmt, act_dtype=torch.bfloat16, use_softmax=w.softmax,
                      renorm=w.renorm, max_tokens=max_tokens, device=device)
    for e in range(w.E):
        gate_up = torch.randn(2 * w.I, w.H, generator=g, device=device) * 0.02
        down = torch.randn(w.H, w.I, generator=g, device=device) * 0.02
        first.load_expert(e, quant(gate_up[: w.I]), quant(gate_up[w.I:]), quant(down))
    layers.append(first)
    for _ in range(1, n_layers):
        n = NativeMoE(num_experts=w.E, top_k=w.k, hidden_size=w.H, intermediate_size=w.I,
                      weight_format=w.wfmt, act_dtype=torch.bfloat16, use_softmax=w.softmax,
                      renorm=w.renorm, max_tokens=max_tokens, device=device)
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


def bench_workload(w, T, layers, router, steps, warmup, device):
    import torch

    xs, ls = make_inputs(w, router, T, 8, device)
    outs = [torch.empty(T, w.H, dtype=torch.bfloat16, device=device) for _ in layers]
    n_act = [active_experts(layers[0], l) for l in ls]
    mean_act = sum(n_act) / len(n_act)
    ms, timed = time_graph(layers, xs, ls, outs, steps, warmup)
    stages = time_stages(layers, xs, ls, outs, rounds=3)
    P = T * w.k
    gate_up_bytes = mean_act * w.bytes_per_expert("gate_up") + T * w.H * 2 + P * w.I * 2
    down_bytes = mean_act * w.bytes_per_expert("down") + P * w.I * 2 + P * w.H * 4
    layer_bytes = (mean_act * (w.bytes_per_expert("gate_up") + w.bytes_per_expert("down"))
                   + T * w.H * 2 * 2 + T * w.E * 2)
    gate_up_flops = 2.0 * P * 2 * w.I * w.H
    down_flops = 2.0 * P * w.H * w.I
    return dict(workload=w.name, tokens=T, ms_per_step=ms, us_per_layer=ms * 1e3, steps=timed,
                tokens_per_s=T / (ms * 1e-3), mean_active_experts=mean_act, breakdown_us=stages,
                layer_bytes=layer_bytes, layer_hbm_frac=layer_bytes / (ms * 1e-3) / HBM_PEAK,
                gate_up=dict(bytes=gate_up_bytes, flops=gate_up_flops, us=stages["gate_up"]),
                down=dict(bytes=down_bytes, flops=down_flops, us=stages["down"]))


def roofline_for(res, bound):
    """Roofline of the dominant kernel (the larger of the two expert GEMM launches)."""
    k = "gate_up" if res["gate_up"]["us"] >= res["down"]["us"] else "down"
    d = res[k]
    sec = d["us"] * 1e-6
    if bound == "hbm":
        achieved = d["bytes"] / sec / 1e9
        return dict(kernel=f"gemm_kernel ({k})", bound="hbm", achieved=round(achieved, 1),
                    peak=HBM_PEAK / 1e9, unit="GB/s", frac=round(achieved * 1e9 / HBM_PEAK, 4),
                    traffic=None, algorithmic_bytes_per_launch=round(d["bytes"]))
    achieved = d["flops"] / sec / 1e12
    return dict(kernel=f"gemm_kernel ({k})", bound="mfma", achieved=round(achieved, 1),
                peak=MFMA_BF16_PEAK / 1e12, unit="TFLOP/s", frac=round(achieved * 1e12 / MFMA_BF16_PEAK, 4),
                traffic=None, algorithmic_flops_per_launch=d["flops"])


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
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (the MoE path here has no multi-GPU build); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs the MI355X GPU", file=sys.stderr)
        sys.exit(1)
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
    del layers
    torch.cuda.empty_cache()
    if not args.no_secondary:
        w = Workload("qwen3_30b_a3b_moe_layer_int8_pc_prefill_zipf", tokens=4096, **QWEN3_INT8)
        log(f"secondary: {w.name} T=4096")
        router8, layers8 = make_layers(w, 2, dev, max_tokens=4096)
        r = bench_workload(w, 4096, layers8, router8, 20, 4, dev)
        r["roofline"] = roofline_for(r, "mfma")
        log(json.dumps(r))
        secondary.append(r)
        del layers8
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
                                                           "layer_hbm_frac")} for r in secondary],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
