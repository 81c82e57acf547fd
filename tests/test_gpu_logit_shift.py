"""GPU parity with logits far outside fp16's exponent range.

Every fused softmax here (query-split, persistent, fused QKV + attention, flash)
subtracts a row maximum before ``exp2``.  The other parity cases draw logits of a
few log2 units, where ``exp2`` of the raw logit would still fit fp16, so dropping
the subtraction (or taking it from the wrong row or tile) would pass them.  Here
the Q and K biases get a constant ``b`` in every dimension: each logit gains
``head_dim * b^2 * scale * log2(e)`` = ``SHIFT`` log2 units (b is chosen per head_dim
for that), a per-row constant the softmax ignores, plus per-key terms that widen
the logit spread to 5-10 log2 units.  Without the subtraction every row's largest
probability would overflow fp16 (2^16); the precondition below checks that on
the oracle's own q and k, and the sublayer must still match the oracle.
"""

import math

import pytest
import torch

from oracle import compare_outputs, make_input

from _gpu_util import DEV, build_pair, log, oracle_on

pytestmark = pytest.mark.gpu

SHIFT = 24.0  # log2 units added to every logit


def _pair(D, H, dtype=torch.float16, seed=0):
    ref, mod = build_pair(D, H, seed=seed, dtype=dtype)
    hd = D // H
    with torch.no_grad():
        b = math.sqrt(SHIFT / math.log2(math.e) / math.sqrt(hd))  # hd * b^2 / sqrt(hd) * log2(e) = SHIFT
        beta = torch.full((D,), b).half().float()  # fp16-representable
        ref.attention.q_proj.bias.add_(beta)
        ref.attention.k_proj.bias.add_(beta)
        ref.attention.q_proj.bias.copy_(ref.attention.q_proj.bias.half().float())
        ref.attention.k_proj.bias.copy_(ref.attention.k_proj.bias.half().float())
    mod.load_state_dict(ref.state_dict(), strict=True)
    return ref, mod


def _row_max_log2(ref, x: torch.Tensor, H: int, causal: bool, keys=None) -> torch.Tensor:
    """Per (head, query) maximum of q k^T * scale * log2(e) over the keys the query
    attends to (causal order, key mask), for one sequence, fp32."""
    with torch.no_grad():
        h = ref.norm1(x.float())
        q = ref.attention.q_proj(h)
        k = ref.attention.k_proj(h)
        S, D = h.shape
        hd = D // H
        q = q.view(S, H, hd).transpose(0, 1)
        k = k.view(S, H, hd).transpose(0, 1)
        s = torch.matmul(q, k.transpose(1, 2).contiguous()) * (hd ** -0.5) * math.log2(math.e)
        allowed = torch.ones(S, S, dtype=torch.bool)
        if causal:
            allowed = allowed.tril()
        if keys is not None:
            allowed = allowed & keys.view(1, S)
        s = s.masked_fill(~allowed, float("-inf"))
    return s.amax(dim=-1)


# (B, S, D, H, causal, masked, x dtype, expected plan, compared sequences)
CASES = [
    (4, 128, 128, 4, False, False, torch.float16, "fused", None),     # query-split, head_dim 32
    (4, 128, 128, 4, True, True, torch.float16, "fused", None),       # query-split, causal + mask
    (4, 128, 128, 16, False, False, torch.float16, "fused", None),    # query-split, head_dim 8
    (4, 128, 128, 1, False, True, torch.float16, "fused", None),      # query-split, one 128-dim head
    (1100, 100, 128, 4, False, True, torch.float16, "fused", [0, 549, 1099]),  # persistent, masked
    (8, 128, 128, 4, True, False, torch.float32, "fused", None),      # persistent, fp32 activations
    (2, 1024, 128, 4, True, False, torch.float16, "staged", None),    # flash attention, head_dim 32
    (2, 128, 1024, 16, False, True, torch.float16, "staged", None),   # staged GEMMs, head_dim 64
    (2, 128, 1024, 4, False, True, torch.float16, "staged", None),    # fused QKV + attention, head_dim 256
]


def _mask(B, S, seed):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, S, generator=g) > 0.2
    m[:, 0] = True
    return m


@pytest.mark.parametrize("B,S,D,H,causal,masked,dtype,plan,rows", CASES,
                         ids=[f"B{c[0]}-S{c[1]}-D{c[2]}-H{c[3]}-{'c' if c[4] else 'n'}{'m' if c[5] else ''}-"
                              f"{'f32' if c[6] == torch.float32 else 'f16'}" for c in CASES])
def test_shifted_logits_match_oracle(B, S, D, H, causal, masked, dtype, plan, rows):
    ref, mod = _pair(D, H, dtype=dtype)
    x = make_input(B, S, D, seed=7)
    if dtype == torch.float16:
        x = x.half()
    m = _mask(B, S, 11) if masked else None
    # Precondition: exp2 of every row's largest logit would overflow fp16.
    lo = _row_max_log2(ref, x[0], H, causal, None if m is None else m[0]).min().item()
    assert lo > 17.0, lo
    log(f"[logit shift] B{B} S{S} D{D} H{H} causal={causal} masked={masked} {dtype} min row max {lo:.1f}")
    with torch.inference_mode():
        y = mod(x.to(DEV), valid_token_mask=None if m is None else m.to(DEV), causal=causal)
        torch.cuda.synchronize()
    assert mod.plan == (0 if plan == "fused" else 1)
    sel = list(range(B)) if rows is None else rows
    want = oracle_on(ref, x[sel].float(), causal, "cpu", mask=None if m is None else m[sel])
    res = compare_outputs(want, y.float().cpu()[sel])
    log(f"[logit shift] plan={plan} max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
    assert res.passed, res
