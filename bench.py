#!/usr/bin/env python3
"""Benchmark of the MI355X attention-sublayer forward (one JSON line on stdout).

Metric: layer forward ms + TFLOP/s (% of MFMA peak).  The
workload of ``value`` is BASELINE config 1 -- B=64, d_model=128, H=4, S=128,
fp16, non-causal -- on inputs resident in HBM.  A "step" is one full sublayer
forward through the drop-in module (LN1, QKV projection, attention,
out-projection + residual, LN2), which the library runs as ONE fused kernel
for this shape.

Also on the same line:
  * ``roofline``: the dominant kernel of the workload, timed alone with HIP
    events on the stream it is launched on (N launches captured in a graph and
    replayed, so launch gaps are excluded); achieved = algorithmic FLOPs (or
    bytes) per launch / average launch time;
  * ``cpu_baseline``: the fp32 oracle (this repo's restatement of the
    reference PyTorch layer) on the host cores, on a bounded sample;
  * ``long``: BASELINE config 5, B=32 d=1024 H=16 S=100000 (``--no-long`` skips), its
    input built per sequence from seeds (``synthetic_sequence``), with its own CPU
    baseline (the query-blocked oracle on one sequence, x32 extrapolated);
  * ``sweep``: every other BASELINE configuration, ms and TFLOP/s per forward, and three
    shapes with bf16 activations (the staged kernels with bf16 operands);
  * ``model``: the whole ``CobraTransformer`` stack on three of the reference's
    model cases (tools/sweep.py:31-47), causal, fp16;
  * ``measured_peaks``: fp16 GEMM TFLOP/s and device-copy GB/s on this box;
  * ``graph``: the same forward replayed as a hipGraph, and an empty-graph floor.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-long] [--no-cpu] [--no-sweep]
       python bench.py --only gemm,s1024   (just those sweep entries, one JSON line; for profiling)
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
    """x in, y out, fp16 weights, fp32 biases and LayerNorm parameters."""
    return B * S * D * 2 * io + 4 * D * D * 2 + 8 * D * 4


def synthetic_input(B, S, D, seed=0):
    """x ~ N(0, 1) from a seeded CPU generator, fp32."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(B, S, D, generator=g, dtype=torch.float32)


def synthetic_sequence(b, S, D, seed=0):
    """Sequence b of a per-sequence-seeded batch: [S, D] fp32 from a
    CPU generator seeded (seed << 32) | b, so any one sequence regenerates alone and a
    checker can rebuild exactly the sequences it samples."""
    g = torch.Generator(device="cpu").manual_seed((seed << 32) | b)
    return torch.randn(1, S, D, generator=g, dtype=torch.float32)[0]


def make_layer(D, H, dev, graph=None, dtype=torch.float16):
    from cobra_amd import CobraAttentionSublayer

    torch.manual_seed(0)
    return CobraAttentionSublayer(D, H, graph=graph).to(device=dev, dtype=dtype).eval()


def event_ms(fn, iters, stream=None):
    """Average ms per fn() over iters calls, HIP events on the current stream."""
    stream = stream or torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(iters):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / iters


def in_graph_ms(fn, n=50, reps=5):
    """Kernel time without launch gaps: n launches captured once, replayed reps times."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n):
            fn()
    g.replay()
    torch.cuda.synchronize()
    return event_ms(g.replay, reps) / n


def host_us_per_call(fn, bursts=50, n=200):
    """Host time of one fn() call, in us: perf_counter_ns over bursts of n calls, each
    burst started after a synchronisation (so the launch queue never fills and blocks
    the host), median of the bursts; 10k calls by default.  When it exceeds the kernel
    time, back-to-back forwards are bound by the host."""
    out = []
    for _ in range(bursts):
        torch.cuda.synchronize()
        t0 = time.perf_counter_ns()
        for _ in range(n):
            fn()
        out.append((time.perf_counter_ns() - t0) / n / 1e3)
    torch.cuda.synchronize()
    return statistics.median(out)


def layer_launcher(layer, x, y):
    """The module's own kernel launch for (x -> y), allocation-free (graph-capturable)."""
    from cobra_amd import ops

    p = layer._packed(x.dtype)
    B, S, D = x.shape
    ws = torch.empty(ops.layer_workspace_bytes(B, S, D, layer.attention.num_heads, False, x.dtype), dtype=torch.uint8,
                     device=x.device)

    def launch():
        ops.layer_fwd(x, p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln1_w, p.ln1_b, p.ln2_w, p.ln2_b, y, ws,
                      layer.attention.num_heads, False)
    return launch


def roofline(name, flops, nbytes, ms, peak_tflops=PEAK_FP16_TFLOPS, peak_gbs=PEAK_HBM_GBS):
    secs = ms / 1e3
    ridge = peak_tflops * 1e12 / (peak_gbs * 1e9)
    if flops / nbytes >= ridge:
        ach = flops / secs / 1e12
        return {"kernel": name, "bound": "mfma", "achieved": ach, "peak": peak_tflops, "unit": "TFLOP/s",
                "frac": ach / peak_tflops, "traffic": None, "avg_us": ms * 1e3,
                "flops_per_launch": flops, "bytes_per_launch": nbytes}
    ach = nbytes / secs / 1e9
    return {"kernel": name, "bound": "hbm", "achieved": ach, "peak": peak_gbs, "unit": "GB/s",
            "frac": ach / peak_gbs, "traffic": None, "avg_us": ms * 1e3,
            "flops_per_launch": flops, "bytes_per_launch": nbytes}


def measured_peaks(dev):
    """Sustained fp16 GEMM and copy rates of this box, for the "% of measured peak" figures.

    The GEMM is 8192^3 through torch (hipBLASLt) in the layout every projection
    on the path uses (A [M, K] row-major times W^T, W [N, K] row-major), on
    N(0,1) data, after ~0.2 s of warm-up; median of five 20-launch runs.  A cold
    10-launch NN measurement reads ~30 % lower on MI355X (clocks ramp, NN is a
    slower layout), which would flatter every fraction derived from it.
    """
    a = torch.randn(8192, 8192, device=dev, dtype=torch.float16)
    w = torch.randn(8192, 8192, device=dev, dtype=torch.float16)
    fn = lambda: torch.matmul(a, w.t())  # noqa: E731
    event_ms(fn, 150)
    ms = statistics.median([event_ms(fn, 20) for _ in range(5)])
    gemm = 2 * 8192 ** 3 / (ms / 1e3) / 1e12
    del a, w
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    event_ms(lambda: dst.copy_(src), 10)
    ms = statistics.median([event_ms(lambda: dst.copy_(src), 10) for _ in range(3)])
    bw = 2 * (1 << 30) / (ms / 1e3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return {"fp16_gemm_8192_tflops": gemm, "device_copy_gbs": bw,
            "method": "torch.matmul(A, W.t()) 8192^3 fp16 N(0,1), warm, median of 5x20; 1 GiB device copy, median of 3x10"}


def graph_floor_us(iters=500):
    t = torch.zeros(1, device="cuda")
    t.add_(1)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        t.add_(1)
    torch.cuda.synchronize()
    for _ in range(10):
        g.replay()
    return event_ms(g.replay, iters) * 1e3


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_info() -> dict:
    """The host CPU the baselines ran on.  `cores` on the baselines is the thread count
    torch used (the box's CPU share: OMP_NUM_THREADS), not the machine's core count."""
    return {"cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}


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
            "kind": "port", "ms_per_forward": ms, **host_info(),
            "sample": f"full B{B} S{S} D{D} H{H} batch, fp32 oracle layer (torch CPU, {threads} threads), "
                      f"median of {len(samples)} forwards in ~{budget_s:.0f}s"}


def cpu_baseline_long(budget_s=20.0, block_q=2048):
    """BASELINE config 5 on the host cores: the query-blocked fp32 oracle
    (tools/reference_chunked.py:73-128 restated) on one full S = 100000 sequence.

    Bounded sample: LN1, the three projections, the out-projection and LN2 run whole
    on the sequence; of its 16 heads x ceil(S / block_q) attention blocks, as many as
    fit in ~budget_s are timed (spread over heads and query positions) and their mean
    is scaled to all blocks.  s/sequence is that sum; the B = 32 forward is x32, which
    is exact for a batch of independent sequences (TTB:1446-1450).
    """
    from oracle import make_sublayer

    B, S, D, H = 32, 100000, 1024, 16
    threads = torch.get_num_threads()
    layer = make_sublayer(D, H, seed=0)
    att = layer.attention
    x = synthetic_sequence(0, S, D)[None]
    with torch.inference_mode():
        t0 = time.perf_counter()
        h = layer.norm1(x)
        q, k, v = att._heads(att.q_proj(h)), att._heads(att.k_proj(h)), att._heads(att.v_proj(h))
        t_proj = time.perf_counter() - t0
        nblk = -(-S // block_q)
        order = [(hh, (hh * 7 + i * 13) % nblk) for i in range(nblk) for hh in range(H)]
        times = []
        t_end = time.perf_counter() + budget_s
        for hh, blk in order:
            if times and time.perf_counter() > t_end:
                break
            q0 = blk * block_q
            q1 = min(q0 + block_q, S)
            t0 = time.perf_counter()
            att._probs_times_v(q[:, hh:hh + 1, q0:q1], k[:, hh:hh + 1], v[:, hh:hh + 1], q0, None, False, x.dtype)
            times.append((time.perf_counter() - t0) * (block_q / (q1 - q0)))
        ctx = torch.randn(1, S, D)
        t0 = time.perf_counter()
        layer.norm2(x + att.out_proj(ctx))
        t_out = time.perf_counter() - t0
    t_attn = statistics.mean(times) * H * nblk
    s_seq = t_proj + t_attn + t_out
    fl = layer_flops(B, S, D)
    return {"value": fl / (s_seq * B) / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "s_per_sequence": s_seq, "s_per_forward_x32_extrapolated": s_seq * B,
            "parts_s": {"ln1_qkv": t_proj, "attention_all_blocks": t_attn, "out_proj_ln2": t_out},
            **host_info(),
            "sample": f"one S={S} D={D} H={H} sequence (seed (0<<32)|0), fp32 query-blocked oracle "
                      f"(block_q {block_q}); projections and LayerNorms timed whole, {len(times)} of "
                      f"{H * nblk} attention blocks timed and scaled; forward = 32 x s/sequence "
                      f"(labelled extrapolation)"}


SWEEP = [  # name, B, S, D, H[, activation dtype]  (BASELINE configs other than the headline one)
    ("b1", 1, 128, 128, 4), ("b4", 4, 128, 128, 4), ("b16", 16, 128, 128, 4), ("b128", 128, 128, 128, 4),
    ("b10000", 10000, 128, 128, 4), ("s32", 64, 32, 128, 4), ("s1024", 64, 1024, 128, 4),
    ("h1", 64, 128, 128, 1), ("h2", 64, 128, 128, 2), ("h16", 64, 128, 128, 16), ("gemm", 64, 128, 1024, 4),
    # bf16 activations and weights (the staged kernels with bf16 operands), not a BASELINE config
    ("base_bf16", 64, 128, 128, 4, torch.bfloat16), ("gemm_bf16", 64, 128, 1024, 4, torch.bfloat16),
    ("s1024_bf16", 64, 1024, 128, 4, torch.bfloat16),
]


def sweep(dev, only=None):
    out = {}
    for name, B, S, D, H, *dt in SWEEP:
        if only and name not in only:
            continue
        dtype = dt[0] if dt else torch.float16
        layer = make_layer(D, H, dev, dtype=dtype)
        x = torch.randn(B, S, D, device=dev, dtype=dtype)
        with torch.inference_mode():
            layer(x)
            iters = 20 if B * S * D < 50_000_000 else 5
            for _ in range(3):
                layer(x)
            ms = event_ms(lambda: layer(x), iters)
            kms = in_graph_ms(layer_launcher(layer, x, torch.empty_like(x)), n=10 if B * S < 1_000_000 else 3,
                              reps=3)
        fl = layer_flops(B, S, D)
        out[name] = {"B": B, "S": S, "D": D, "H": H, "dtype": str(dtype).replace("torch.", ""),
                     "plan": "fused" if layer.plan == 0 else "staged",
                     "ms_per_forward": ms, "tflops": fl / (ms / 1e3) / 1e12,
                     "kernels_ms_in_graph": kms, "tflops_in_graph": fl / (kms / 1e3) / 1e12,
                     "hbm_gbs_in_graph": layer_bytes(B, S, D) / (kms / 1e3) / 1e9}
        log(f"[sweep] {name}: {ms * 1e3:.1f} us/forward ({out[name]['tflops']:.1f} TFLOP/s), "
            f"in-graph {kms * 1e3:.1f} us, plan {out[name]['plan']}")
        del layer, x
    torch.cuda.empty_cache()
    return out


def bench_long(dev, steps=2, warmup=1):
    from cobra_amd import ops

    B, S, D, H = 32, 100000, 1024, 16
    layer = make_layer(D, H, dev)
    x = torch.empty(B, S, D, device=dev, dtype=torch.float16)
    for b in range(B):  # per-sequence seeds: any sequence of the timed input can be rebuilt alone
        x[b].copy_(synthetic_sequence(b, S, D).half())
    with torch.inference_mode():
        for _ in range(warmup):
            layer(x)
        torch.cuda.synchronize()
        ms = event_ms(lambda: layer(x), steps)
        # host-resident input (8 sequences, pageable): streamed in chunks with the copies
        # overlapping compute; the PCIe-inclusive rate, never `value`
        xh = x[:8].cpu()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        yh = layer(xh)
        torch.cuda.synchronize()
        host_ms = (time.perf_counter() - t0) * 1e3
        del xh, yh
        # the attention kernel alone, on two sequences of the same shape
        p = layer._packed()
        x2 = x[:2].reshape(2 * S, D)
        _, h = ops.add_ln(x2, None, None, p.ln1_w, p.ln1_b, True, 1e-5, False)
        qkv = ops.linear(h, p.w_qkv, p.b_qkv)
        hd = D // H
        a_ms = event_ms(lambda: ops.attn(qkv, 2, S, H, hd, hd ** -0.5, causal=False), 2) / 2
    del x
    torch.cuda.empty_cache()
    fl = layer_flops(B, S, D)
    a_fl = 4 * S * S * D
    return {"config": {"workload": "B32 d1024 H16 S100000 fp16 non-causal", "batch": B, "seq_len": S,
                       "d_model": D, "heads": H},
            "ms_per_step": ms, "tflops": fl / (ms / 1e3) / 1e12,
            "mfma_frac": fl / (ms / 1e3) / 1e12 / PEAK_FP16_TFLOPS, "steps": steps, "warmup": warmup,
            "host_resident_8seq": {"ms": host_ms, "tflops": fl / 4 / (host_ms / 1e3) / 1e12,
                                   "device_resident_ms_same_work": ms / 4,
                                   "note": "pageable host input and output, 4 chunks of 2 sequences, H2D/D2H and "
                                           "host staging copies overlapped with compute (PCIe-inclusive)"},
            "roofline": dict(roofline("attn_fwd_kernel (per sequence)", a_fl, 4 * S * D * 2, a_ms),
                             traffic=committed_traffic(LONG_TRAFFIC_FILE))}


MODEL_CASES = [  # the reference's whole-model cases (tools/sweep.py:31-47): #, B, S, D, H, F, layers (causal)
    ("case1", 64, 128, 128, 4, 128, 4), ("case8", 64, 128, 1024, 4, 1024, 4), ("case13", 64, 1024, 128, 4, 128, 4),
]
# The full matrix of tools/sweep.py:31-47 (``--matrix``); case 14 runs with 8 of its 32
# sequences (one forward is ~2.8 s at full batch).
MATRIX_CASES = [
    ("case1", 64, 128, 128, 4, 128, 4), ("case2", 1, 128, 128, 4, 128, 4), ("case3", 4, 128, 128, 4, 128, 4),
    ("case4", 16, 128, 128, 4, 128, 4), ("case5", 128, 128, 128, 4, 128, 4), ("case6", 10000, 128, 128, 4, 128, 4),
    ("case7", 64, 128, 32, 4, 32, 4), ("case8", 64, 128, 1024, 4, 1024, 4), ("case9", 64, 128, 128, 1, 128, 4),
    ("case10", 64, 128, 128, 2, 128, 4), ("case11", 64, 128, 128, 16, 128, 4), ("case12", 64, 32, 128, 4, 128, 4),
    ("case13", 64, 1024, 128, 4, 128, 4), ("case14_8seq", 8, 100000, 1024, 16, 1024, 2),
]


def bench_model(dev, iters=20, cases=MODEL_CASES):
    """The whole ``CobraTransformer`` stack (hipGraph replay for inputs <= 64 MiB), causal, fp16."""
    from cobra_amd import CobraTransformer, TransformerConfig

    out = {}
    for name, B, S, D, H, F, L in cases:
        n = 1 if B * S * D >= 100_000_000 else iters
        torch.manual_seed(0)
        model = CobraTransformer(TransformerConfig(B, S, D, H, F, L, True)).to(device=dev,
                                                                                dtype=torch.float16).eval()
        x = torch.randn(B, S, D, device=dev, dtype=torch.float16)
        with torch.inference_mode():
            for _ in range(3 if n > 1 else 1):
                model(x)
            ms = statistics.median([event_ms(lambda: model(x), n) for _ in range(3)])
        T = B * S
        fl = L * (8 * T * D * D + 2 * B * S * S * D + 4 * T * D * F)  # causal attention: half the S^2 work
        out[name] = {"B": B, "S": S, "D": D, "H": H, "ffn_dim": F, "layers": L, "causal": True,
                     "ms_per_forward": ms, "tflops": fl / (ms / 1e3) / 1e12}
        log(f"[model] {name}: {ms:.3f} ms/forward ({out[name]['tflops']:.1f} TFLOP/s)")
        del model, x
    torch.cuda.empty_cache()
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_layer_split_kernel_B64_d128_H4_S128.txt")
LONG_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_attn_fwd_kernel_B32_d1024_H16_S100000.txt")


def committed_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch of a kernel, from its committed PMC summary (or None)."""
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch="):
                return float(line.split("=", 1)[1])
    except OSError:
        pass
    return None


PMC_CONFIGS = {  # --pmc-driver workloads: name -> (B, S, D, H)
    "base": (64, 128, 128, 4), "gemm": (64, 128, 1024, 4), "b10000": (10000, 128, 128, 4),
    "s1024": (64, 1024, 128, 4), "long2": (2, 100000, 1024, 16),
    "h1": (64, 128, 128, 1), "h2": (64, 128, 128, 2), "h16": (64, 128, 128, 16), "b128": (128, 128, 128, 4),
    "s32": (64, 32, 128, 4), "b1": (1, 128, 128, 4),
}


def pmc_driver(dev, name="base") -> None:
    """Workload for `rocprofv3 --pmc ...`: the counter calibration, then one configuration.

    Calibration, known HBM bytes: a 64 MiB device copy (ordinary loads and stores,
    __amd_rocclr_copyBuffer) five times, and a GEMM whose operand tiles arrive by
    LDS-DMA like every kernel on the path (gemm_dma_kernel, 65536 x 128 x 64: A, 8 MiB,
    read once; W, 16 KiB; C, 16 MiB fp16, written once) five times.  Then three forwards
    of the named configuration (PMC_CONFIGS; "long2" = two sequences of the long shape),
    inputs already on the device.
    """
    from cobra_amd import ops

    src = torch.randn(16 << 20, device=dev)  # 64 MiB
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    a = torch.randn(65536, 64, device=dev).half()
    w = torch.randn(128, 64, device=dev).half()
    for _ in range(5):
        ops.linear(a, w, None)
    torch.cuda.synchronize()
    del src, dst, a, w
    B, S, D, H = PMC_CONFIGS[name]
    layer = make_layer(D, H, dev)
    if name == "long2":
        x = torch.empty(B, S, D, device=dev, dtype=torch.float16)
        for b in range(B):
            x[b].copy_(synthetic_sequence(b, S, D).half())
    else:
        x = synthetic_input(B, S, D, seed=0).half().to(dev)
    launch = layer_launcher(layer, x, torch.empty_like(x))
    with torch.inference_mode():
        for _ in range(3):
            launch()
    torch.cuda.synchronize()
    print(f"pmc driver done: {name} B{B} S{S} D{D} H{H}", flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--pmc-driver", nargs="?", const="base", default=None, choices=sorted(PMC_CONFIGS),
                    help="run the PMC calibration workload and one configuration, then exit")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-long", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--only", default="", help="comma-separated sweep entries to time alone (" +
                    ", ".join(n for n, *_ in SWEEP) + ")")
    ap.add_argument("--matrix", action="store_true",
                    help="time CobraTransformer on the reference's whole-model case matrix and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(sequences are independent, so the sublayer would shard by batch with no exchange "
              "between GPUs; one GPU's figure is one shard's)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    dev = torch.device("cuda:0")
    if args.matrix:
        print(json.dumps({"matrix": bench_model(torch.device("cuda:0"), cases=MATRIX_CASES)}), flush=True)
        return 0
    if args.pmc_driver:
        pmc_driver(dev, args.pmc_driver)
        return 0
    if args.only:
        names = [n for n in args.only.split(",") if n]
        unknown = [n for n in names if n not in {s[0] for s in SWEEP}]
        if unknown:
            print(f"unknown sweep entries {unknown}", file=sys.stderr)
            return 2
        print(json.dumps({"sweep": sweep(dev, set(names))}), flush=True)
        return 0
    B, S, D, H = 64, 128, 128, 4
    x = synthetic_input(B, S, D, seed=0).half().to(dev)
    layer = make_layer(D, H, dev)
    with torch.inference_mode():
        layer(x)
        for _ in range(args.warmup):
            layer(x)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(args.steps):
            layer(x)
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        host_us = host_us_per_call(lambda: layer(x))
        # the dominant (here: the only) kernel -- the query-split fused kernel at
        # this batch -- launch gaps excluded
        k_ms = in_graph_ms(layer_launcher(layer, x, torch.empty_like(x)), n=50, reps=5)
        # the same forward replayed as a hipGraph (graph=True), and the empty-graph floor
        glayer = make_layer(D, H, dev, graph=True)
        glayer(x)
        gxin = glayer.input_buffer()
        g_ms = event_ms(lambda: glayer(gxin), args.steps)
        floor = graph_floor_us()
        del glayer
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
        "config": {"workload": "attention sublayer fwd B64 d128 H4 S128 fp16 non-causal (one fused kernel)",
                   "batch": B, "seq_len": S, "d_model": D, "heads": H, "causal": False},
        "host_us_per_forward": host_us,
        "mfma_frac": tflops / PEAK_FP16_TFLOPS,
        "hbm_gbs": layer_bytes(B, S, D) / (ms / 1e3) / 1e9,
        "roofline": dict(roofline("layer_split_kernel", flops, layer_bytes(B, S, D), k_ms),
                         traffic=committed_traffic()),
        "graph": {"ms_per_step_graph_replay": g_ms, "empty_graph_replay_us": floor,
                  "note": "the fused plan launches one kernel directly; replaying it as a hipGraph is slower"},
    }
    log(f"[bench] base: {ms * 1e3:.2f} us/forward, {tflops:.2f} TFLOP/s; kernel {k_ms * 1e3:.2f} us; "
        f"host {host_us:.2f} us/call; graph replay {g_ms * 1e3:.2f} us")
    peaks = line["measured_peaks"] = measured_peaks(dev)
    line["measured_mfma_frac"] = tflops / peaks["fp16_gemm_8192_tflops"]
    line["measured_hbm_frac"] = line["hbm_gbs"] / peaks["device_copy_gbs"]
    if not args.no_sweep:
        line["sweep"] = sweep(dev)
        for v in line["sweep"].values():
            v["measured_mfma_frac"] = v["tflops_in_graph"] / peaks["fp16_gemm_8192_tflops"]
            v["measured_hbm_frac"] = v["hbm_gbs_in_graph"] / peaks["device_copy_gbs"]
        line["model"] = bench_model(dev)
        for v in line["model"].values():
            v["measured_mfma_frac"] = v["tflops"] / peaks["fp16_gemm_8192_tflops"]
    if not args.no_long:
        try:
            line["long"] = bench_long(dev)
            line["long"]["measured_mfma_frac"] = line["long"]["tflops"] / peaks["fp16_gemm_8192_tflops"]
            log(f"[bench] long: {line['long']['ms_per_step']:.1f} ms/forward")
        except torch.cuda.OutOfMemoryError as e:
            line["long"] = {"error": f"OOM: {e}"}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(B, S, D, H)
        if not args.no_long:
            line["long"]["cpu_baseline"] = cpu_baseline_long()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
