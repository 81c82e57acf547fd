"""The reference's per-element accuracy gate (test infrastructure).

Restates ``compare_outputs`` (``torch_transformer_benchmark.py:1630-1697``) and
its result record ``AccuracyResult`` (TTB:1616-1627).  An element passes when
both values are finite and ``|opt - ref| <= atol`` OR ``|opt - ref| <= rtol *
|ref|`` -- deliberately not ``torch.isclose``, whose ``atol + rtol*|ref|`` is
looser (TTB:1653-1654).  The benchmark's thresholds are ``atol = 2e-3``,
``rtol = 2e-2`` (argparse defaults, TTB:1959-1960).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import torch

ATOL = 2e-3
RTOL = 2e-2

# Opt-in log of every comparison, for the per-test worst-error report the test
# session writes (tests/conftest.py, COBRA_PARITY_REPORT).  None: not recording.
RECORD: "List[Tuple[float, float, int, int, float]] | None" = None


@dataclass
class AccuracyResult:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float


def compare_outputs(
    reference: torch.Tensor,
    optimized: torch.Tensor,
    rtol: float = RTOL,
    atol: float = ATOL,
) -> AccuracyResult:
    if tuple(reference.shape) != tuple(optimized.shape):  # TTB:1636-1640
        raise AssertionError(
            f"shape mismatch: baseline={tuple(reference.shape)}, "
            f"optimized={tuple(optimized.shape)}"
        )
    ref = reference.detach().float()
    opt = optimized.detach().float()

    err = (opt - ref).abs()
    ok = torch.isfinite(ref) & torch.isfinite(opt) & ((err <= atol) | (err <= rtol * ref.abs()))
    failed = ~ok
    n_failed = int(failed.sum().item())

    # Worst element by absolute error, unravelled to a multi-index (TTB:1662-1668).
    flat = int(err.reshape(-1).argmax().item()) if err.numel() else 0
    worst = []
    for size in reversed(reference.shape):
        worst.append(flat % size)
        flat //= size
    worst_index = tuple(reversed(worst))

    rel = err / ref.abs().clamp_min(1e-12)  # TTB:1670-1671

    if reference.ndim == 0:  # failures summarised by output feature, TTB:1674-1684
        dims = [0] if n_failed else []
    elif reference.ndim == 1:
        dims = torch.nonzero(failed).flatten().tolist()
    else:
        dims = torch.nonzero(failed.any(dim=tuple(range(reference.ndim - 1)))).flatten().tolist()

    max_abs = float(err.max().item()) if err.numel() else 0.0
    max_rel = float(rel.max().item()) if rel.numel() else 0.0
    if RECORD is not None:
        # The gate's margin: per element min(err / atol, err / (rtol |ref|)), <= 1 passes.
        ratio = torch.minimum(err / atol, err / (rtol * ref.abs()).clamp_min(1e-30))
        ratio = torch.where(torch.isfinite(ref) & torch.isfinite(opt), ratio, torch.full_like(ratio, float("inf")))
        worst_ratio = float(ratio.max().item()) if ratio.numel() else 0.0
        RECORD.append((max_abs, max_rel, n_failed, reference.numel(), worst_ratio))
    return AccuracyResult(
        passed=n_failed == 0,
        total_elements=reference.numel(),
        failed_elements=n_failed,
        max_abs_error=max_abs,
        max_relative_error=max_rel,
        mean_abs_error=float(err.mean().item()) if err.numel() else 0.0,
        failed_feature_dims=dims,
        worst_index=worst_index,
        reference_at_worst=float(ref[worst_index].item()) if ref.numel() else 0.0,
        optimized_at_worst=float(opt[worst_index].item()) if opt.numel() else 0.0,
    )
