"""CPU tests of bench.py's accounting and its command-line contract."""

import os
import subprocess
import sys

import pytest
import torch
from torch.utils.flop_counter import FlopCounterMode

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from oracle import make_input, make_sublayer  # noqa: E402
from oracle.cases import oracle_forward  # noqa: E402


@pytest.mark.parametrize("B,S,D,H,causal", [(2, 16, 32, 4, False), (1, 24, 64, 2, False), (3, 8, 16, 1, False)])
def test_layer_flops_equal_an_independent_count(B, S, D, H, causal):
    """bench's FLOP formula (8 T D^2 + 4 B S^2 D) against torch's own count of the
    matrix products the oracle layer runs (four projections, q k^T, p v)."""
    layer = make_sublayer(D, H, seed=0)
    x = make_input(B, S, D, seed=0)
    with FlopCounterMode(display=False) as fc, torch.no_grad():
        oracle_forward(layer, x, causal=causal)
    assert fc.get_total_flops() == bench.layer_flops(B, S, D, causal)


def test_layer_bytes_match_the_committed_traffic_file():
    """The algorithmic bytes in the committed counter summary are bench's formula for
    the headline workload, and the measured traffic is at least that."""
    fields = {}
    with open(bench.TRAFFIC_FILE) as f:
        for line in f:
            if "=" in line and not line.startswith("#"):
                k, v = line.strip().split("=", 1)
                fields[k] = float(v)
    assert fields["algorithmic_bytes_per_launch"] == bench.layer_bytes(64, 128, 128)
    assert bench.committed_traffic() == fields["traffic_bytes_per_launch"]
    assert fields["traffic_bytes_per_launch"] >= fields["algorithmic_bytes_per_launch"]
    kib = 1024
    want = (fields["kernel_fetch_kib_per_dispatch"] * fields["fetch_scale"]
            + fields["kernel_write_kib_per_dispatch"] * fields["write_scale"]) * kib
    assert abs(want - fields["traffic_bytes_per_launch"]) <= 16 * kib  # scale rounded to 4 places


def test_roofline_picks_the_bound_by_arithmetic_intensity():
    ridge = bench.PEAK_FP16_TFLOPS * 1e12 / (bench.PEAK_HBM_GBS * 1e9)
    r = bench.roofline("k", flops=ridge * 2e6, nbytes=1e6, ms=1.0)
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s"
    assert r["achieved"] == pytest.approx(ridge * 2e6 / 1e-3 / 1e12)
    r = bench.roofline("k", flops=ridge * 0.5e6, nbytes=1e6, ms=1.0)
    assert r["bound"] == "hbm" and r["unit"] == "GB/s"
    assert r["frac"] == pytest.approx(1e6 / 1e-3 / 1e9 / bench.PEAK_HBM_GBS)


def _run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    res = _run_bench("--gpus", "2")
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout == ""


def test_without_a_gpu_bench_exits_with_a_message():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    res = _run_bench("--steps", "1", "--warmup", "0")
    assert res.returncode == 2
    assert "GPU" in res.stderr


def test_long_input_sequences_are_the_oracles():
    """The long leg builds its timed input per sequence; each must be exactly the
    sequence ``oracle.make_sequence`` regenerates for the same index (shortened S)."""
    from oracle import make_sequence

    for b in (0, 5, 31):
        assert torch.equal(bench.synthetic_sequence(b, 300, 64), make_sequence(b, 300, 64)[0])


def test_long_cpu_baseline_scales_a_bounded_sample():
    """The S = 1e5 CPU baseline times a bounded sample and reports a labelled x32
    extrapolation; run here at a tiny budget (it stops after the first block)."""
    out = bench.cpu_baseline_long(budget_s=0.0)
    assert out["kind"] == "port" and out["cores"] == torch.get_num_threads()
    assert out["s_per_forward_x32_extrapolated"] == pytest.approx(32 * out["s_per_sequence"])
    assert "1 of 784 attention blocks" in out["sample"]
    assert out["cpu_model"] and out["os_cpu_count"] == os.cpu_count()


def test_long_traffic_file_is_consistent():
    """The long leg's committed traffic: fetch and write counters scaled as the file says,
    per sequence, and at least the algorithmic bytes bench.py's roofline uses."""
    fields = {}
    with open(bench.LONG_TRAFFIC_FILE) as f:
        for line in f:
            if "=" in line and not line.startswith("#"):
                k, v = line.strip().split("=", 1)
                fields[k] = float(v)
    S, D = 100000, 1024
    assert fields["algorithmic_bytes_per_sequence"] == 4 * S * D * 2
    want = (fields["kernel_fetch_kib_per_dispatch"] * fields["fetch_scale"]
            + fields["kernel_write_kib_per_dispatch"] * fields["write_scale"]) * 1024 / fields["sequences_per_dispatch"]
    assert abs(want - fields["traffic_bytes_per_launch"]) <= 1e-4 * want
    assert bench.committed_traffic(bench.LONG_TRAFFIC_FILE) == fields["traffic_bytes_per_launch"]
