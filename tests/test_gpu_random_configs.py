"""Seeded random sublayer configurations against the fp32 oracle.

Each case draws the batch, sequence length, d_model / head_dim, causality, a token
mask, the activation dtype and non-trivial LayerNorm / bias parameters from a fixed
seed, so the set is the same on every run; together they cross the plan boundaries
(query-split, persistent and staged kernels) in combinations the hand-picked cases
do not.  Sizes stay small enough for the oracle on the CPU.
"""

import random

import pytest
import torch

from oracle import compare_outputs, make_input

from _gpu_util import DEV, build_pair, log, oracle_on, randomise_affine

pytestmark = pytest.mark.gpu

# (d_model, heads) pairs the library accepts, head_dim 8 .. 256
GEOMETRIES = [(64, 2), (64, 8), (96, 3), (128, 1), (128, 2), (128, 4), (128, 16), (128, 8), (256, 2), (256, 16),
              (512, 8), (1024, 4)]


def _cases(n=24, seed=20261202):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        D, H = rng.choice(GEOMETRIES)
        S = rng.choice([1, 7, 32, 33, 64, 100, 127, 128, 129, 200])
        B = rng.choice([1, 2, 3, 5, 8, 17]) if D <= 256 else rng.choice([1, 2])
        causal = rng.random() < 0.4
        masked = rng.random() < 0.4
        dtype = torch.float32 if rng.random() < 0.2 else torch.float16
        out.append((i, B, S, D, H, causal, masked, dtype))
    return out


@pytest.mark.parametrize("i,B,S,D,H,causal,masked,dtype", _cases(),
                         ids=[f"{c[0]:02d}-B{c[1]}-S{c[2]}-D{c[3]}-H{c[4]}-{'c' if c[5] else 'n'}"
                              f"{'m' if c[6] else ''}-{'f32' if c[7] == torch.float32 else 'f16'}" for c in _cases()])
def test_random_config_matches_oracle(i, B, S, D, H, causal, masked, dtype):
    log(f"[random {i:02d}] B{B} S{S} D{D} H{H} causal={causal} masked={masked} {dtype}")
    ref, mod = build_pair(D, H, seed=i, dtype=dtype)
    randomise_affine(ref, 1000 + i)
    mod.load_state_dict(ref.state_dict(), strict=True)
    x = make_input(B, S, D, seed=i)
    if dtype == torch.float16:
        x = x.half()
    m = None
    if masked:
        g = torch.Generator().manual_seed(2000 + i)
        m = torch.rand(B, S, generator=g) > 0.3
        m[:, 0] = True  # every sequence keeps a valid key
    with torch.inference_mode():
        y = mod(x.to(DEV), valid_token_mask=None if m is None else m.to(DEV), causal=causal)
        torch.cuda.synchronize()
    want = oracle_on(ref, x.float(), causal, "cpu", mask=m)
    res = compare_outputs(want, y.float().cpu())
    log(f"[random {i:02d}] plan={'fused' if mod.plan == 0 else 'staged'} max_abs={res.max_abs_error:.3e} "
        f"failed={res.failed_elements}/{res.total_elements}")
    assert res.passed, res
