"""The harness counterpart (tests/harness.py) of the reference's main()
(torch_transformer_benchmark.py:1935-2084): its flags, validation, input
generation and statistics on the CPU; an end-to-end run on the GPU."""

import os
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import harness  # noqa: E402


def test_defaults_are_the_reference_flags():
    """TTB:1935-1986 defaults."""
    a = harness.parse_args([])
    assert (a.batch_size, a.seq_len, a.d_model, a.heads, a.ffn_dim, a.layers) == (8, 128, 512, 8, 2048, 6)
    assert (a.causal, a.device, a.dtype, a.padding_ratio, a.input_scale) == (False, "auto", "float32", 0.0, 1.0)
    assert (a.accuracy_trials, a.rtol, a.atol, a.seed) == (5, 0.02, 0.002, 1234)
    assert (a.warmup, a.repeats, a.benchmark_rounds, a.benchmark_on_failure) == (20, 100, 3, False)
    assert (a.matmul_precision, a.allow_tf32, a.non_strict_weight_copy) == ("high", True, False)
    assert a.reference_precision == "float32"
    assert harness.parse_args(["--no-allow-tf32"]).allow_tf32 is False


@pytest.mark.parametrize("argv,msg", [
    (["--padding-ratio", "1.0"], "padding_ratio"),
    (["--input-scale", "0"], "input_scale"),
    (["--accuracy-trials", "0"], "accuracy_trials"),
    (["--rtol", "-1"], "rtol"),
    (["--warmup", "-1"], "warmup"),
    (["--repeats", "0"], "repeats"),
    (["--compile-user"], "compile"),
])
def test_validation_rejects(argv, msg):
    args = harness.parse_args(argv)
    with pytest.raises(ValueError, match=msg):
        harness.validate_args(args, torch.device("cuda"))


def test_validation_requires_the_gpu():
    with pytest.raises(ValueError, match="GPU"):
        harness.validate_args(harness.parse_args([]), torch.device("cpu"))


def test_percentile_is_linear_interpolation():
    rng = np.random.default_rng(0)
    for n in (1, 2, 7, 100):
        v = rng.normal(size=n).tolist()
        for q in (0.0, 0.5, 0.9, 1.0):
            assert harness.percentile(v, q) == pytest.approx(float(np.percentile(v, 100 * q)), rel=1e-12)
    with pytest.raises(ValueError):
        harness.percentile([], 0.5)


def test_random_case_padding_semantics():
    """TTB:1575-1612: lengths in [round(S (1 - r)), S], left-aligned mask, padded
    tokens zero-filled, same seed -> same case."""
    from cobra_amd import TransformerConfig

    cfg = TransformerConfig(16, 40, 8, 2, 8, 1, False)
    dev = torch.device("cpu")
    x, m = harness.generate_random_case(cfg, dev, torch.float32, 7, 0.3, 2.0)
    assert x.shape == (16, 40, 8) and m.shape == (16, 40) and m.dtype == torch.bool
    lengths = m.sum(1)
    assert int(lengths.min()) >= round(40 * 0.7) and int(lengths.max()) <= 40
    for b in range(16):  # left-aligned: valid tokens first
        assert bool(m[b, : int(lengths[b])].all()) and not bool(m[b, int(lengths[b]):].any())
    assert bool((x[~m] == 0).all())
    x2, m2 = harness.generate_random_case(cfg, dev, torch.float32, 7, 0.3, 2.0)
    assert torch.equal(x, x2) and torch.equal(m, m2)
    x3, m3 = harness.generate_random_case(cfg, dev, torch.float32, 7, 0.0, 1.0)
    assert bool(m3.all())
    # input_scale multiplies the N(0, 1) draw of the same generator stream
    assert torch.allclose(x[m], 2.0 * x3[m])


@pytest.mark.gpu
@pytest.mark.parametrize("extra", [
    ["--dtype", "float16", "--causal", "--padding-ratio", "0.3"],
    ["--dtype", "float16", "--d-model", "128", "--heads", "4", "--ffn-dim", "128"],
    ["--dtype", "float32", "--reference-precision", "harness"],
    ["--dtype", "bfloat16", "--causal", "--padding-ratio", "0.3", "--atol", "0.016"],
])
def test_harness_end_to_end(extra, capsys):
    argv = ["--device", "cuda", "--batch-size", "4", "--seq-len", "48", "--d-model", "64", "--heads", "2",
            "--ffn-dim", "96", "--layers", "2", "--accuracy-trials", "2", "--warmup", "1", "--repeats", "3",
            "--benchmark-rounds", "2"] + extra
    print(f"[harness] {' '.join(argv)}", flush=True)
    code = harness.main(argv)
    out = capsys.readouterr().out
    assert code == 0, out
    assert "summary: PASS" in out and "speedup  :" in out
