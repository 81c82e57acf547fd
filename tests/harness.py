#!/usr/bin/env python3
"""Command-line counterpart of the reference's benchmark harness (TEST INFRASTRUCTURE).

Mirrors ``main()`` of torch_transformer_benchmark.py (TTB:1935-2084): the same
flags, validation and seeding; a baseline transformer and the drop-in optimised
one built from the same ``TransformerConfig``; a strict weight copy
(TTB:1544-1554); seeded accuracy trials gated per element with
``abs <= atol OR abs <= rtol * |ref|`` (TTB:1575-1697, 1700-1760); then latency
rounds that alternate the measurement order, HIP events per call, median /
mean / p90 / min and the speedup on the median (TTB:1804-1924).

What differs, on purpose:

* the baseline is this repository's fp32 restatement of the reference model
  (``oracle.OracleTransformer``, the checker of every parity test), and the
  optimised model is ``cobra_amd.CobraTransformer``;
* ``--reference-precision float32`` (the default) runs the baseline of the
  ACCURACY trials in fp32 on the same dtype-rounded inputs and weights -- the
  repository's parity policy, since the fp16 PyTorch layer rounds the
  probabilities to fp16 before P.V and a "more accurate" kernel can fail a
  difference gate against it.  ``harness`` compares against the baseline run at
  the harness dtype, as the reference does.  The timed baseline always runs at
  the harness dtype;
* ``bfloat16`` runs this library's bf16 kernels (bf16 MFMA operands, fp32
  accumulation and residual); the reference runs bf16 through its unmodified
  baseline ops instead (TTB:952-968), noting that at its default gate a bf16
  forward fails many elements (bf16 keeps 8 mantissa bits): pass a tolerance
  scaled to bf16, e.g. ``--atol 0.016`` (8 x the default, bf16's unit roundoff over
  fp16's).  ``--compile-*`` is refused (no eager fallback to compile);
* the optimised model needs a GPU (``--device cuda``); there is no CPU path.

Usage (from the repository root)::

    python tests/harness.py --batch-size 64 --seq-len 128 --d-model 128 --heads 4 \\
        --ffn-dim 128 --layers 4 --causal --dtype float16

Exit status: 0 when every trial passes, 2 otherwise (TTB:2072-2084).
"""

from __future__ import annotations

import argparse
import math
import os
import statistics
import sys
import time
from dataclasses import dataclass
from typing import List, Tuple

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for _p in (ROOT, os.path.join(ROOT, "cobra-gpu-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402


def parse_args(argv=None) -> argparse.Namespace:
    """The reference's flags (TTB:1935-1986), plus ``--reference-precision``."""
    p = argparse.ArgumentParser(description="Compare the baseline transformer and the MI355X drop-in")
    p.add_argument("--batch-size", type=int, default=8)
    p.add_argument("--seq-len", type=int, default=128)
    p.add_argument("--d-model", type=int, default=512)
    p.add_argument("--heads", type=int, default=8)
    p.add_argument("--ffn-dim", type=int, default=2048)
    p.add_argument("--layers", type=int, default=6)
    p.add_argument("--causal", action="store_true")
    p.add_argument("--device", default="auto", help="auto, cuda, cuda:0, ...")
    p.add_argument("--dtype", choices=("float32", "float16", "bfloat16"), default="float32")
    p.add_argument("--padding-ratio", type=float, default=0.0)
    p.add_argument("--input-scale", type=float, default=1.0)
    p.add_argument("--accuracy-trials", type=int, default=5)
    p.add_argument("--rtol", type=float, default=0.02)
    p.add_argument("--atol", type=float, default=0.002)
    p.add_argument("--seed", type=int, default=1234)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--repeats", type=int, default=100)
    p.add_argument("--benchmark-rounds", type=int, default=3)
    p.add_argument("--benchmark-on-failure", action="store_true")
    p.add_argument("--compile-baseline", action="store_true")
    p.add_argument("--compile-user", action="store_true")
    p.add_argument("--compile-mode", choices=("default", "reduce-overhead", "max-autotune"), default="default")
    p.add_argument("--non-strict-weight-copy", action="store_true")
    p.add_argument("--matmul-precision", choices=("highest", "high", "medium"), default="high")
    p.add_argument("--allow-tf32", action=argparse.BooleanOptionalAction, default=True)
    p.add_argument("--reference-precision", choices=("float32", "harness"), default="float32",
                   help="precision of the accuracy trials' baseline (see the module docstring)")
    return p.parse_args(argv)


_DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def resolve_device(arg: str) -> torch.device:
    if arg == "auto":
        return torch.device("cuda" if torch.cuda.is_available() else "cpu")
    dev = torch.device(arg)
    if dev.type == "cuda" and not torch.cuda.is_available():
        raise RuntimeError("a GPU was requested, but torch.cuda.is_available() is False")
    return dev


def validate_args(args: argparse.Namespace, device: torch.device) -> None:
    """The reference's checks (TTB:1989-2004) and this build's own limits."""
    if not 0.0 <= args.padding_ratio < 1.0:
        raise ValueError("padding_ratio must be in [0, 1)")
    if args.input_scale <= 0:
        raise ValueError("input_scale must be positive")
    if args.accuracy_trials <= 0:
        raise ValueError("accuracy_trials must be positive")
    if args.rtol < 0 or args.atol < 0:
        raise ValueError("rtol and atol must be non-negative")
    if args.warmup < 0:
        raise ValueError("warmup must be non-negative")
    if args.repeats <= 0 or args.benchmark_rounds <= 0:
        raise ValueError("repeats and benchmark_rounds must be positive")
    if args.compile_baseline or args.compile_user:
        raise ValueError("--compile-*: not supported (the optimised model has no eager path to compile)")
    if device.type != "cuda":
        raise ValueError("the optimised model runs on the GPU only: pass --device cuda")


def generate_random_case(config, device: torch.device, dtype: torch.dtype, seed: int, padding_ratio: float,
                         input_scale: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """TTB:1575-1612: x ~ N(0, 1) * scale from a device generator; with padding,
    per-sequence lengths in [round(S (1 - ratio)), S], left-aligned, padded
    tokens zero-filled."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=gen, device=device, dtype=dtype)
    x = x * input_scale
    if padding_ratio <= 0:
        return x, torch.ones(config.batch_size, config.seq_len, device=device, dtype=torch.bool)
    min_valid = max(1, int(round(config.seq_len * (1.0 - padding_ratio))))
    lengths = torch.randint(low=min_valid, high=config.seq_len + 1, size=(config.batch_size,), generator=gen,
                            device=device)
    valid = torch.arange(config.seq_len, device=device)[None, :] < lengths[:, None]
    return x.masked_fill(~valid[..., None], 0), valid


def percentile(values: List[float], q: float) -> float:
    """Linear interpolation between closest ranks (TTB:1763-1776)."""
    if not values:
        raise ValueError("values must not be empty")
    v = sorted(values)
    pos = (len(v) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    return v[lo] if lo == hi else v[lo] * (1.0 - (pos - lo)) + v[hi] * (pos - lo)


@dataclass
class TimingResult:
    samples_ms: List[float]

    @property
    def mean_ms(self) -> float:
        return statistics.fmean(self.samples_ms)

    @property
    def median_ms(self) -> float:
        return statistics.median(self.samples_ms)

    @property
    def p90_ms(self) -> float:
        return percentile(self.samples_ms, 0.90)

    @property
    def min_ms(self) -> float:
        return min(self.samples_ms)


def run_accuracy_tests(baseline, optimized, config, device, dtype, args) -> bool:
    """TTB:1700-1760, with the baseline precision of ``--reference-precision``."""
    from oracle import compare_outputs

    print("\n=== Accuracy check ===")
    print(f"criterion: abs_error <= {args.atol:g} OR relative_error <= {args.rtol:.2%}")
    if args.reference_precision == "float32":
        print("baseline: fp32 restatement on the same dtype-rounded inputs and weights")
    ok_all, max_abs, max_rel, n_failed, n_total = True, 0.0, 0.0, 0, 0
    with torch.inference_mode():
        for trial in range(args.accuracy_trials):
            x, valid = generate_random_case(config, device, dtype, args.seed + trial, args.padding_ratio,
                                            args.input_scale)
            ref = baseline(x.float() if args.reference_precision == "float32" else x, valid)
            out = optimized(x, valid)
            res = compare_outputs(ref, out, rtol=args.rtol, atol=args.atol)
            ok_all &= res.passed
            max_abs, max_rel = max(max_abs, res.max_abs_error), max(max_rel, res.max_relative_error)
            n_failed += res.failed_elements
            n_total += res.total_elements
            print(f"trial {trial + 1:02d}/{args.accuracy_trials}: {'PASS' if res.passed else 'FAIL'} | "
                  f"max_abs={res.max_abs_error:.6g} | max_rel={res.max_relative_error:.6g} | "
                  f"failed={res.failed_elements}/{res.total_elements}")
            if not res.passed:
                dims = res.failed_feature_dims[:16]
                more = "..." if len(res.failed_feature_dims) > len(dims) else ""
                print(f"  worst_index={res.worst_index}, baseline={res.reference_at_worst:.8g}, "
                      f"optimized={res.optimized_at_worst:.8g}")
                print(f"  failed output feature dims={dims}{more}")
    print(f"summary: {'PASS' if ok_all else 'FAIL'} | max_abs={max_abs:.6g} | max_rel={max_rel:.6g} | "
          f"failed={n_failed}/{n_total}")
    return ok_all


def _time_calls(model, x, valid, iterations: int, device: torch.device) -> List[float]:
    """One HIP event pair around each call on the current stream (TTB:1830-1849)."""
    with torch.inference_mode():
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
        torch.cuda.synchronize(device)
        for i in range(iterations):
            starts[i].record()
            model(x, valid)
            ends[i].record()
        torch.cuda.synchronize(device)
    return [a.elapsed_time(b) for a, b in zip(starts, ends)]


def benchmark_models(baseline, optimized, config, device, dtype, args) -> Tuple[TimingResult, TimingResult]:
    """TTB:1852-1924: fixed input, both models warmed up, rounds alternating order."""
    print("\n=== Performance benchmark ===")
    print("timing excludes random-data generation and uses a fixed input")
    print("latency is measured with torch.cuda.Event (HIP events) on the current stream")
    x, valid = generate_random_case(config, device, dtype, args.seed + 100000, args.padding_ratio,
                                    args.input_scale)
    with torch.inference_mode():
        for model in (baseline, optimized):
            for _ in range(args.warmup):
                model(x, valid)
    torch.cuda.synchronize(device)
    base, opt = [], []
    for r in range(args.benchmark_rounds):
        order = [(baseline, base), (optimized, opt)] if r % 2 == 0 else [(optimized, opt), (baseline, base)]
        for model, acc in order:
            acc.extend(_time_calls(model, x, valid, args.repeats, device))
    b, o = TimingResult(base), TimingResult(opt)
    tokens = config.batch_size * config.seq_len
    for name, t in (("baseline ", b), ("optimized", o)):
        print(f"{name}: median={t.median_ms:.4f} ms | mean={t.mean_ms:.4f} ms | p90={t.p90_ms:.4f} ms | "
              f"min={t.min_ms:.4f} ms | throughput={tokens * 1000.0 / t.median_ms:.2f} token/s")
    print(f"speedup  : {b.median_ms / o.median_ms:.3f}x based on median latency")
    return b, o


def main(argv=None) -> int:
    from cobra_amd import CobraTransformer, TransformerConfig
    from oracle import OracleTransformer, OracleTransformerConfig

    args = parse_args(argv)
    device = resolve_device(args.device)
    dtype = _DTYPES[args.dtype]
    fields = (args.batch_size, args.seq_len, args.d_model, args.heads, args.ffn_dim, args.layers, args.causal)
    config = TransformerConfig(*fields)
    config.validate()
    validate_args(args, device)

    torch.manual_seed(args.seed)  # TTB:2024-2031: seed, then construct the baseline first
    torch.set_float32_matmul_precision(args.matmul_precision)
    torch.cuda.manual_seed_all(args.seed)
    torch.backends.cuda.matmul.allow_tf32 = args.allow_tf32
    torch.backends.cudnn.allow_tf32 = args.allow_tf32

    baseline = OracleTransformer(OracleTransformerConfig(*fields))
    optimized = CobraTransformer(config)
    incompatible = optimized.load_state_dict(baseline.state_dict(), strict=not args.non_strict_weight_copy)
    if args.non_strict_weight_copy:
        if incompatible.missing_keys:
            print(f"[warning] missing optimized keys: {incompatible.missing_keys}")
        if incompatible.unexpected_keys:
            print(f"[warning] unexpected optimized keys: {incompatible.unexpected_keys}")
    baseline = baseline.to(device=device, dtype=dtype).eval()
    optimized = optimized.to(device=device, dtype=dtype).eval()
    # The accuracy baseline in fp32: the same dtype-rounded weights, upcast.
    acc_baseline = baseline
    if args.reference_precision == "float32" and dtype != torch.float32:
        acc_baseline = OracleTransformer(OracleTransformerConfig(*fields))
        acc_baseline.load_state_dict({k: v.float() for k, v in baseline.state_dict().items()})
        acc_baseline = acc_baseline.to(device).eval()

    print("=== Configuration ===")
    print(config)
    print(f"device={device}, dtype={dtype}, torch={torch.__version__}")
    print(f"gpu={torch.cuda.get_device_name(device)}")

    prev_tf32 = torch.backends.cuda.matmul.allow_tf32
    if args.reference_precision == "float32":
        torch.backends.cuda.matmul.allow_tf32 = False  # an exact fp32 baseline for the gate
    try:
        passed = run_accuracy_tests(acc_baseline, optimized, config, device, dtype, args)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev_tf32
    if not passed and not args.benchmark_on_failure:
        print("\nPerformance benchmark skipped because accuracy validation failed.")
        print("Use --benchmark-on-failure to benchmark an incorrect implementation anyway.")
        return 2
    benchmark_models(baseline, optimized, config, device, dtype, args)
    return 0 if passed else 2


if __name__ == "__main__":
    t0 = time.perf_counter()
    code = main()
    print(f"[harness] {time.perf_counter() - t0:.1f} s", file=sys.stderr)
    raise SystemExit(code)
