#!/usr/bin/env python3
"""Benchmark of the MI355X attention-sublayer forward (one JSON line on stdout).

Metric: layer forward ms + TFLOP/s (% of MFMA peak).  The
workload of ``value`` is BASELINE config 1 -- B=64, d_model=128, H=4, S=128,
fp16, non-causal -- run as one hipGraph replay per step on inputs resident in
HBM.  A "step" is one full sublayer forward (LN1, QKV projection, attention,
out-projection + residual, LN2).

Also reported on the same line:
  * ``roofline``: the dominant kernel of the workload, timed alone with HIP
    events on the stream it is launched on; achieved = its algorithmic bytes
    (or FLOPs) per launch / average launch time;
  * ``cpu_baseline``: the fp32 oracle (this repo's restatement of the
    reference PyTorch layer) on the host cores, on a bounded sample;
  * ``long``: BASELINE config 5, B=32 d=1024 H=16 S=100000 (skip with --no-long);
  * ``graph_floor_us``: replay time of a one-kernel graph (launch floor).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-long] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "cobra-gpu-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

METRIC = "layer fwd ms + TFLOP/s (% MFMA peak), B64 d128 H4 S128 and B32 d1024 H16 S100k"
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA (published)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E (published)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def layer_flops(B, S, D, causal=False):
    attn = 4 * B * S * S * D
    return 8 * B * S * D * D + (attn // 2 if causal else attn)


def layer_bytes(B, S, D, io=2):
    return B * S * D * 2 * io + 4 * D * D * 2 + 8 * D * 4


def make_layer(D, H, dev):
    from cobra_amd import CobraAttentionSublayer

    torch.manual_seed(0)
    return CobraAttentionSublayer(D, H).to(device=dev, dtype=torch.float16).eval()


def time_loop(fn, iters, stream):
    """Average ms of fn() over iters launches, HIP events on `stream`."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def kernel_breakdown(layer, x, iters=200):
    """Time each kernel of the eager pipeline alone (same kernels the graph replays)."""
    from cobra_amd import ops

    B, S, D = x.shape
    H = layer.attention.num_heads
    hd = D // H
    p = layer._packed()
    stream = torch.cuda.current_stream()
    x2 = x.view(B * S, D)
    _, h = ops.add_ln(x2, None, None, p.ln1_w, p.ln1_b, cast_fp16=True, store_resid=False)
    qkv = ops.linear(h, p.w_qkv, p.b_qkv)
    ctx = ops.attn(qkv, B, S, H, hd, hd ** -0.5, causal=False)
    T = B * S
    kernels = {
        "ln_rows": (lambda: ops.add_ln(x2, None, None, p.ln1_w, p.ln1_b, True, 1e-5, False),
                    0, T * D * 4 + 8 * D),
        "gemm_qkv": (lambda: ops.linear(h, p.w_qkv, p.b_qkv),
                     2 * T * D * 3 * D, T * D * 2 + 3 * D * D * 2 + T * 3 * D * 2 + 12 * D),
        "attn_fwd": (lambda: ops.attn(qkv, B, S, H, hd, hd ** -0.5, causal=False),
                     4 * B * S * S * D, T * 3 * D * 2 + T * D * 2),
    }
    if D <= 128:
        kernels["gemm_out_ln"] = (lambda: ops.linear_ln(ctx, p.w_o, p.b_o, x2, p.ln2_w, p.ln2_b),
                                  2 * T * D * D, T * D * 2 * 3 + T * D * 4 + D * D * 2 + 12 * D)
    out = {}
    for name, (fn, flops, nbytes) in kernels.items():
        for _ in range(5):
            fn()
        ms = time_loop(fn, iters, stream)
        out[name] = {"ms": ms, "flops": flops, "bytes": nbytes}
    return out


def roofline_of(name, k):
    secs = k["ms"] / 1e3
    ai = k["flops"] / k["bytes"] if k["bytes"] else float("inf")
    ridge = PEAK_FP16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    if ai >= ridge:
        ach = k["flops"] / secs / 1e12
        return {"kernel": name, "bound": "mfma", "achieved": ach, "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                "frac": ach / PEAK_FP16_TFLOPS, "traffic": None, "avg_us": k["ms"] * 1e3}
    ach = k["bytes"] / secs / 1e9
    return {"kernel": name, "bound": "hbm", "achieved": ach, "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": ach / PEAK_HBM_GBS, "traffic": None, "avg_us": k["ms"] * 1e3}


def graph_floor_us(iters=500):
    t = torch.zeros(1, device="cuda")
    t.add_(1)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        t.add_(1)
    torch.cuda.synchronize()
    for _ in range(10):
        g.replay()
    return time_loop(g.replay, iters, torch.cuda.current_stream()) * 1e3


def cpu_baseline(B, S, D, H, budget_s=10.0):
    """fp32 oracle forward on the host cores; median over a ~budget_s sample."""
    from oracle import make_input, make_sublayer

    threads = torch.get_num_threads()
    layer = make_sublayer(D, H, seed=0)
    x = make_input(B, S, D, seed=0)
    samples = []
    with torch.inference_mode():
        layer(x)
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(samples) < 3:
            t0 = time.perf_counter_ns()
            layer(x)
            samples.append((time.perf_counter_ns() - t0) / 1e6)
    ms = statistics.median(samples)
    return {"value": layer_flops(B, S, D) / (ms / 1e3) / 1e12, "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "ms_per_forward": ms,
            "sample": f"full B{B} S{S} D{D} H{H} batch, fp32 oracle layer (torch CPU), median of {len(samples)} "
                      f"forwards in ~{budget_s:.0f}s"}


def bench_long(dev, steps=2, warmup=1):
    B, S, D, H = 32, 100000, 1024, 16
    layer = make_layer(D, H, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn(B, S, D, device=dev, dtype=torch.float16, generator=g)
    with torch.inference_mode():
        for _ in range(warmup):
            layer(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            y = layer(x)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        # attention kernel alone, on one sequence chunk of the same shape
        from cobra_amd import ops
        p = layer._packed()
        x1 = x[:2].reshape(2 * S, D)
        _, h = ops.add_ln(x1, None, None, p.ln1_w, p.ln1_b, True, 1e-5, False)
        qkv = ops.linear(h, p.w_qkv, p.b_qkv)
        hd = D // H
        fn = lambda: ops.attn(qkv, 2, S, H, hd, hd ** -0.5, causal=False)  # noqa: E731
        fn()
        a_ms = time_loop(fn, 2, torch.cuda.current_stream())
    del x, y
    fl = layer_flops(B, S, D)
    a_fl = 4 * 2 * S * S * D
    return {"config": {"workload": "B32 d1024 H16 S100000 fp16 non-causal", "batch": B, "seq_len": S,
                       "d_model": D, "heads": H},
            "ms_per_step": ms, "tflops": fl / (ms / 1e3) / 1e12,
            "mfma_frac": fl / (ms / 1e3) / 1e12 / PEAK_FP16_TFLOPS, "steps": steps, "warmup": warmup,
            "attn_fwd": {"ms_per_2_sequences": a_ms, "tflops": a_fl / (a_ms / 1e3) / 1e12,
                         "mfma_frac": a_fl / (a_ms / 1e3) / 1e12 / PEAK_FP16_TFLOPS}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-long", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the sublayer shards by batch with no exchange; see DESIGN.md)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    dev = torch.device("cuda:0")
    B, S, D, H = 64, 128, 128, 4
    layer = make_layer(D, H, dev)
    from oracle import make_input

    x = make_input(B, S, D, seed=0).half().to(dev)
    with torch.inference_mode():
        layer(x)                       # pack + capture the hipGraph
        xin = layer.input_buffer()     # graph's own input: no copy per step
        xin.copy_(x)
        for _ in range(args.warmup):
            layer(xin)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(args.steps):
            layer(xin)
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        # same loop with the per-call input copy the reference's graph path pays
        copy_ms = time_loop(lambda: layer(x), args.steps, stream)
        kernels = kernel_breakdown(layer, x)
        floor = graph_floor_us()
    dom = max(kernels, key=lambda k: kernels[k]["ms"])
    flops = layer_flops(B, S, D)
    tflops = flops / (ms / 1e3) / 1e12
    line = {
        "metric": METRIC,
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: x ~ N(0,1) seed 0 (CPU generator), nn.Linear default init under manual_seed(0)",
        "config": {"workload": "attention sublayer fwd B64 d128 H4 S128 fp16 non-causal, one hipGraph replay",
                   "batch": B, "seq_len": S, "d_model": D, "heads": H, "causal": False},
        "mfma_frac": tflops / PEAK_FP16_TFLOPS,
        "hbm_gbs": layer_bytes(B, S, D) / (ms / 1e3) / 1e9,
        "ms_per_step_with_input_copy": copy_ms,
        "graph_floor_us": floor,
        "kernels_us": {k: v["ms"] * 1e3 for k, v in kernels.items()},
        "roofline": roofline_of(dom, kernels[dom]),
    }
    log(f"[bench] base: {ms * 1e3:.2f} us/forward, {tflops:.2f} TFLOP/s; kernels {line['kernels_us']}")
    if not args.no_long:
        try:
            line["long"] = bench_long(dev)
            log(f"[bench] long: {line['long']['ms_per_step']:.1f} ms/forward")
        except torch.cuda.OutOfMemoryError as e:
            line["long"] = {"error": f"OOM: {e}"}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(B, S, D, H)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
