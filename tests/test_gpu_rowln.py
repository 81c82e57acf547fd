"""GPU parity of the out-projection with LayerNorm over whole rows in its epilogue.

At head_dim 256 and S <= 128 (the B64 d1024 config), fp16 activations and no stored
residual, the staged sublayer ends in one kernel: the out-projection's column tiles of
a 256-row block each reduce their rows to (mean, M2), exchange them through the
workspace and normalise their own columns (LN2 without the branch in memory).  The
cases cover every row width it takes (2, 4, 8 and 16 column tiles per row), token
masks, the full 256-tile grid of B64 d1024, a grid below the plan's threshold and the
batch one row block past the chip (both take the GEMM + LayerNorm pass instead), random
LayerNorm / bias parameters, inputs
whose rows have a mean of hundreds of standard deviations (the exchange combines the
tiles' statistics without cancellation), repeated calls with different batch sizes on
one workspace, and replays of a captured graph.

Reference: the fp32 oracle (TTB:60-173) on the same fp16-rounded weights and inputs,
gate of `compare_outputs` (TTB:1630-1697): zero failing elements.
"""

import pytest
import torch

from oracle import compare_outputs, make_input

from _gpu_util import DEV, build_pair, log, oracle_on, randomise_affine

pytestmark = pytest.mark.gpu


def _pair(D, H, seed=0, graph=None):
    ref, mod = build_pair(D, H, seed=seed, graph=graph)
    randomise_affine(ref, seed + 100)
    mod.load_state_dict(ref.state_dict(), strict=True)
    return ref, mod


def _mask(B, S, seed):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, S, generator=g) > 0.25
    m[:, 0] = True
    return m


def _check(ref, mod, x, causal, m, rows, tag):
    with torch.inference_mode():
        y = mod(x.to(DEV), valid_token_mask=None if m is None else m.to(DEV), causal=causal)
        torch.cuda.synchronize()
    want = oracle_on(ref, x[rows].float(), causal, "cpu", mask=None if m is None else m[rows])
    res = compare_outputs(want, y.float().cpu()[rows])
    log(f"[rowln] {tag} max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
    assert torch.isfinite(y).all(), tag
    assert res.passed, (tag, res)
    return y


# (B, S, D, H, causal, masked, compared sequences).  The plan takes the kernel when its
# grid covers at least three quarters of the chip (half of it at K <= 512) and fits it
# whole; the other batches run the GEMM + LayerNorm pass.
CASES = [
    (128, 128, 256, 1, False, True, [0, 127]),    # 2 column tiles per row (128 tiles, K = 256)
    (82, 100, 512, 2, True, False, [0, 81]),      # 4 (132 tiles, K = 512; last row block 8 rows)
    (32, 128, 2048, 8, True, True, [0, 31]),      # 16 (256 tiles)
    (64, 128, 1024, 4, False, True, [0, 31, 63]),  # 8: the full 256-tile grid, masked
    (48, 77, 1024, 4, True, True, [0, 47]),       # 8 (120 tiles, below the threshold: GEMM + LN pass)
    (65, 128, 1024, 4, True, False, [0, 64]),     # 264 tiles: the GEMM + LayerNorm pass
]


@pytest.mark.parametrize("B,S,D,H,causal,masked,rows", CASES,
                         ids=[f"B{c[0]}-S{c[1]}-D{c[2]}-H{c[3]}-{'c' if c[4] else 'n'}{'m' if c[5] else ''}"
                              for c in CASES])
def test_rowln_matches_oracle(B, S, D, H, causal, masked, rows):
    ref, mod = _pair(D, H, seed=D + H)
    x = make_input(B, S, D, seed=B + S).half()
    m = _mask(B, S, 3) if masked else None
    _check(ref, mod, x, causal, m, list(range(B)) if rows is None else rows, f"B{B} S{S} D{D} H{H}")


@pytest.mark.parametrize("B,D,H", [(64, 1024, 4), (32, 2048, 8)])
def test_rowln_large_row_mean(B, D, H):
    """Rows offset by ~300 standard deviations: LN2's statistics combine the tiles' means
    and squared deviations, never a raw sum of squares."""
    ref, mod = _pair(D, H, seed=7)
    S = 128
    g = torch.Generator().manual_seed(11)
    x = make_input(B, S, D, seed=4) + 300.0 * torch.randn(B, S, 1, generator=g)
    _check(ref, mod, x.half(), False, _mask(B, S, 5), [0, B - 1], f"large mean D{D}")


def test_rowln_repeated_calls_share_workspace():
    """Back-to-back calls of different batch sizes (different numbers of row blocks on the
    same statistics area): each call marks the area unwritten before its exchange, so
    every output equals a fresh call's, bit for bit."""
    ref, mod = _pair(1024, 4, seed=3)
    xs = [make_input(B, 128, 1024, seed=B).half().to(DEV) for B in (64, 9, 56, 1, 64)]
    with torch.inference_mode():
        first = [mod(x).clone() for x in xs]
        torch.cuda.synchronize()
        again = [mod(x).clone() for x in reversed(xs)][::-1]
        torch.cuda.synchronize()
    for a, b in zip(first, again):
        assert torch.equal(a, b)
    want = oracle_on(ref, xs[1].float().cpu(), False, "cpu")
    assert compare_outputs(want, first[1].float().cpu()).passed


def test_rowln_graph_replays_match_eager():
    """The sublayer captured in a graph (the fill of the statistics area is a kernel, not a
    memset) and replayed with fresh inputs, eager work between the replays, each replay
    equal to the eager call bit for bit."""
    ref, mod = _pair(1024, 4, seed=5, graph=True)
    xs = [make_input(64, 128, 1024, seed=s).half().to(DEV) for s in range(3)]
    with torch.inference_mode():
        outs = []
        for x in xs:  # the first call captures, later ones replay
            outs.append(mod(x).clone())
            torch.cuda.synchronize()
            (x.float() * 2).sum().item()
        assert mod._graph is not None
        mod._graph_ok = False
        eager = [mod(x).clone() for x in xs]
        torch.cuda.synchronize()
    for o, e in zip(outs, eager):
        assert torch.equal(o, e)
    want = oracle_on(ref, xs[2].float().cpu()[:2], False, "cpu")
    assert compare_outputs(want, outs[2].float().cpu()[:2]).passed
