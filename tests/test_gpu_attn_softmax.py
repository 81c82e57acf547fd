"""GPU checks of the flash attention's online softmax on score patterns that move the running max.

After the first key block the kernel forms each 32-key tile's probabilities against the
running max without a block maximum, and accepts the tile when every lane's tile sum is at
most 2^16; a tile that fails rescales over the block's remaining tiles and is exponentiated
again.  Random N(0, 1) inputs (the other attention tests) never fail the check, so these
cases build the scores to make it fail:

* "ramp": key j's score grows by ~0.58 per key (log2 units), so every later block's first
  tile exceeds the running max by up to ~18 -- a failed check and a rescale per block;
* "spike": N(0, 1) scores plus one key per sequence ~58 above them, placed in the third
  32-key tile of a later block -- the check fails in the middle of a block, after two
  tiles have already been accumulated under the old max;
* "fall": the largest scores in the first block, then ~-60 -- later probabilities
  underflow to zero, no rescale.

Reference: fp32 torch softmax attention on the same fp16 (bf16) values (the restatement of
TTB:98-113), gate `allclose(atol=2e-3, rtol=1e-2)` as the other attention op tests (bf16:
atol 1.6e-2, rtol 2e-2).
"""

import pytest
import torch

from _gpu_util import DEV

pytestmark = pytest.mark.gpu


def _qkv(pattern, B, S, H, hd, seed):
    g = torch.Generator().manual_seed(seed)
    D = H * hd
    q = torch.randn(B, S, H, hd, generator=g)
    k = torch.randn(B, S, H, hd, generator=g)
    v = torch.randn(B, S, H, hd, generator=g)
    # Scores q.k * hd^-0.5: dimension 0 carries the pattern (q[..., 0] = hd^0.5, so that
    # k[..., 0] is the score it adds in natural-log units); the other dimensions add N(0, 1).
    q[..., 0] = hd ** 0.5
    j = torch.arange(S, dtype=torch.float32)
    if pattern == "ramp":
        k[..., 0] = (0.4 * j)[None, :, None]
    elif pattern == "spike":
        k[..., 0] = 0.0
        pos = min(S - 1, 128 + 64 + 5) if S > 200 else S - 1  # tile 2 of the second 128-key block
        k[:, pos, :, 0] = 40.0
    elif pattern == "fall":
        k[..., 0] = torch.where(j < 16, 0.0, -40.0)[None, :, None]
    qkv = torch.stack([q, k, v], 2).reshape(B * S, 3 * D)
    return qkv


def _reference(qkv, B, S, H, hd, causal, mask):
    D = H * hd
    q, k, v = qkv.float().view(B, S, 3, H, hd).permute(2, 0, 3, 1, 4)
    s = (q @ k.transpose(-2, -1).contiguous()) * hd ** -0.5
    dead = torch.zeros(B, 1, S, S, dtype=torch.bool, device=qkv.device)
    if mask is not None:
        dead = dead | ~mask[:, None, None, :]
    if causal:
        dead = dead | torch.ones(S, S, dtype=torch.bool, device=qkv.device).triu(1)
    s = s.masked_fill(dead, float("-inf"))
    p = torch.softmax(s, -1).nan_to_num(0.0)
    return (p @ v).transpose(1, 2).reshape(B * S, D)


@pytest.mark.parametrize("pattern", ["ramp", "spike", "fall"])
@pytest.mark.parametrize("hd", [16, 32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_attn_running_max_moves(pattern, hd, causal, masked):
    from cobra_amd import ops

    B, H = 2, 2
    for S in (100, 300, 1000):
        qkv = _qkv(pattern, B, S, H, hd, seed=S + hd).half().to(DEV)
        mask = None
        if masked:
            g = torch.Generator().manual_seed(S)
            mask = torch.rand(B, S, generator=g) < 0.7
            mask[:, 0] = True
            mask = mask.to(DEV)
        got = ops.attn(qkv, B, S, H, hd, hd ** -0.5, causal=causal, key_mask=mask).float()
        want = _reference(qkv, B, S, H, hd, causal, mask)
        err = (got - want).abs().max().item()
        print(f"[attn-softmax] {pattern} hd{hd} S{S} causal={causal} masked={masked} max_abs={err:.2e}", flush=True)
        assert torch.isfinite(got).all(), (pattern, hd, S, causal, masked)
        assert torch.allclose(got, want, atol=2e-3, rtol=1e-2), (pattern, hd, S, causal, masked, err)


@pytest.mark.parametrize("pattern", ["ramp", "spike"])
def test_attn_running_max_moves_bf16(pattern):
    from cobra_amd import ops

    B, H, hd = 2, 4, 32
    for S in (300, 1000):
        qkv = _qkv(pattern, B, S, H, hd, seed=S).to(torch.bfloat16).to(DEV)
        got = ops.attn(qkv, B, S, H, hd, hd ** -0.5, causal=False).float()
        want = _reference(qkv, B, S, H, hd, False, None)
        err = (got - want).abs().max().item()
        print(f"[attn-softmax] bf16 {pattern} S{S} max_abs={err:.2e}", flush=True)
        assert torch.allclose(got, want, atol=1.6e-2, rtol=2e-2), (pattern, S, err)
