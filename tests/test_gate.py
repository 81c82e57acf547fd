"""Pins the restated accuracy gate (oracle/gate.py, TTB:1630-1697) on crafted pairs."""

import math

import pytest
import torch

from oracle import compare_outputs


def test_abs_branch_inclusive_at_atol():
    ref = torch.tensor([0.0, 0.0])
    opt = torch.tensor([0.001, -0.001])
    r = compare_outputs(ref, opt, rtol=0.0, atol=0.001)
    assert r.passed and r.failed_elements == 0


def test_rel_branch_uses_reference_magnitude():
    ref = torch.tensor([10.0])
    opt = torch.tensor([10.15])  # err 0.15 > atol, <= 0.02 * |ref| = 0.2
    assert compare_outputs(ref, opt).passed
    # same error with |ref| small and |opt| large must fail: rel is against ref
    assert not compare_outputs(torch.tensor([0.1]), torch.tensor([0.25])).passed


def test_or_not_isclose_sum():
    """isclose would accept err <= atol + rtol*|ref|; the gate does not."""
    ref = torch.tensor([0.05])
    opt = ref + 0.0025  # > atol (0.002) and > rtol*|ref| (0.001), < their sum 0.003
    r = compare_outputs(ref, opt)
    assert not r.passed and r.failed_elements == 1
    assert torch.isclose(opt, ref, rtol=0.02, atol=0.002).all()


def test_non_finite_fails():
    ref = torch.tensor([1.0, 2.0, float("inf")])
    opt = torch.tensor([float("nan"), 2.0, float("inf")])
    r = compare_outputs(ref, opt)
    assert r.failed_elements == 2


def test_worst_index_and_feature_dims():
    ref = torch.zeros(2, 3, 4)
    opt = ref.clone()
    opt[1, 2, 3] = 0.5
    opt[0, 1, 1] = 0.01
    r = compare_outputs(ref, opt)
    assert r.worst_index == (1, 2, 3)
    assert r.failed_feature_dims == [1, 3]
    assert r.optimized_at_worst == 0.5 and r.reference_at_worst == 0.0
    assert math.isclose(r.max_abs_error, 0.5)
    assert r.total_elements == 24 and r.failed_elements == 2


def test_shape_mismatch_raises():
    with pytest.raises(AssertionError):
        compare_outputs(torch.zeros(2, 3), torch.zeros(3, 2))


def test_dtype_upcast_fp16_input():
    ref = torch.tensor([1.0, 2.0])
    opt = torch.tensor([1.0, 2.0], dtype=torch.float16)
    assert compare_outputs(ref, opt).passed
