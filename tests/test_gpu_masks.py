"""GPU parity of token masks (``valid_token_mask``) and the GEMM / LayerNorm epilogue options.

Masks follow ``BaselineSelfAttention`` (TTB:106-109, 121-122): padded keys are
``-inf`` before the softmax, padded rows get a zero attention output (so the
residual equals x there and y = LN2(x)).  The oracle is the fp32 restatement
with the same mask; the gate is the reference's (abs <= 2e-3 or rel <= 2e-2,
zero failures).  Masks are left-aligned like the reference harness's padding
(TTB:1602-1612) or scattered (any pattern, including padded first tokens and
whole padded 64-key blocks); one sequence per batch is fully padded.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import compare_outputs, make_input

from _gpu_util import DEV, build_pair, log, oracle_on

pytestmark = pytest.mark.gpu


def token_mask(B, S, seed, left_aligned):
    g = torch.Generator().manual_seed(seed)
    if left_aligned:
        lengths = torch.randint(1, S + 1, (B,), generator=g)
        m = torch.arange(S)[None, :] < lengths[:, None]
    else:
        m = torch.rand(B, S, generator=g) < 0.6
        if S > 80:
            m[0, :70] = False  # the first key block (64 keys) holds no valid key
        if S > 1:
            m[-1, 0] = False  # padded first token
    m[0, -1] = True if not left_aligned else m[0, -1]
    if B > 2:
        m[1] = False  # a fully padded sequence
    return m


@pytest.mark.parametrize(
    "B,S,D,H",
    [
        (16, 128, 128, 4),   # the headline geometry: query-split fused kernel
        (5, 80, 128, 2),     # query-split, head_dim 64, ragged S
        (4, 128, 64, 2),     # query-split, d_model 64
        (5, 100, 128, 1),    # query-split, one head of 128 dims over four waves, ragged S
        (5, 100, 128, 16),   # query-split, four 8-dim heads per wave, ragged S
        (300, 128, 128, 4),  # persistent fused kernel (more than two rounds of slices)
        (601, 96, 128, 4),   # persistent fused kernel, odd batch, ragged S
        (3, 17, 96, 3),      # persistent fused kernel, d_model 96
        (301, 96, 64, 2),    # persistent, d_model 64: two sequences per workgroup, odd batch
        (3, 333, 128, 2),    # hd 64, several key blocks, 8-wave attention
        (3, 100, 256, 2),    # hd 128, D > 128 (separate LN2 pass)
        (3, 40, 512, 2),     # hd 256 (32-key blocks)
        (3, 300, 32, 4),     # hd 8 -> 16-wide heads, 128-key blocks
    ],
)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("left", [True, False])
def test_layer_masked(B, S, D, H, causal, left):
    ref, mod = build_pair(D, H)
    x = make_input(B, S, D, seed=21).half()
    m = token_mask(B, S, seed=B * S + D, left_aligned=left)
    if left:
        x = x.masked_fill(~m[..., None], 0)  # the harness zero-fills padded tokens (TTB:1612)
    log(f"[mask] B{B} S{S} D{D} H{H} causal={causal} left={left} valid={int(m.sum())}/{m.numel()}")
    with torch.inference_mode():
        r, y = mod(x.to(DEV), m.to(DEV), causal=causal, return_residual=True)
        torch.cuda.synchronize()
    want_r, want_y = oracle_on(ref, x.float(), causal, "cpu", return_residual=True, mask=m)
    res = compare_outputs(want_y, y.float().cpu())
    log(f"[mask] max_abs={res.max_abs_error:.3e} failed={res.failed_elements}/{res.total_elements}")
    assert res.passed, res
    assert compare_outputs(want_r, r.cpu()).passed
    # padded rows: the attention branch is exactly zero, so r == x bit for bit
    assert torch.equal(r.cpu()[~m], x.float()[~m])


def test_masked_graph_replays_with_new_masks():
    """Staged plan under hipGraph: the mask is copied into the graph's static buffer per call."""
    ref, mod = build_pair(128, 4, graph=True)
    B, S, D = 8, 128, 128
    x = make_input(B, S, D, seed=4).half()
    xd = x.to(DEV)
    for seed in range(3):
        m = token_mask(B, S, seed=seed, left_aligned=seed % 2 == 0)
        with torch.inference_mode():
            y = mod(xd, m.to(DEV)).float().cpu()
            torch.cuda.synchronize()
        res = compare_outputs(oracle_on(ref, x.float(), False, "cpu", mask=m), y)
        log(f"[mask graph {seed}] max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
        assert res.passed, res
    assert mod._graph is not None


@pytest.mark.parametrize("B,S,D,H", [(8, 128, 128, 4), (300, 128, 128, 4), (4, 200, 128, 4), (8, 128, 128, 1),
                                     (8, 128, 128, 16)])
def test_all_valid_mask_equals_no_mask(B, S, D, H):
    """An all-true mask gives the unmasked result bit for bit (fused kernels, both
    variants, and the staged plan)."""
    ref, mod = build_pair(D, H)
    x = make_input(B, S, D, seed=5).half().to(DEV)
    with torch.inference_mode():
        a = mod(x).clone()
        b = mod(x, torch.ones(B, S, dtype=torch.bool, device=DEV))
        torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_fused_masked_fp32_io():
    """fp32 activations run the persistent fused kernel; masked against the masked oracle."""
    from cobra_amd import CobraAttentionSublayer
    from oracle import make_sublayer
    from oracle.cases import oracle_forward

    ref = make_sublayer(128, 4, seed=0)
    mod = CobraAttentionSublayer(128, 4)
    mod.load_state_dict(ref.state_dict())
    mod = mod.to(DEV).eval()
    x = make_input(6, 128, 128, seed=8)
    m = token_mask(6, 128, seed=3, left_aligned=False)
    with torch.inference_mode():
        y = mod(x.to(DEV), m.to(DEV), causal=True)
        torch.cuda.synchronize()
    assert mod.plan == 0
    res = compare_outputs(oracle_forward(ref, x, causal=True, valid_token_mask=m), y.cpu())
    log(f"[mask fp32] max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
    assert res.passed, res


def test_mask_bits_exact():
    from cobra_amd import ops

    for B, S in [(1, 1), (3, 63), (2, 64), (4, 65), (5, 1000)]:
        m = torch.rand(B, S, generator=torch.Generator().manual_seed(S)) < 0.5
        bits = ops.mask_bits(m.to(DEV)).cpu().numpy().view(np.uint64)
        nw = (S + 63) // 64
        want = np.zeros((B, nw), dtype=np.uint64)
        mn = m.numpy()
        for b in range(B):
            for j in range(S):
                if mn[b, j]:
                    want[b, j // 64] |= np.uint64(1) << np.uint64(j % 64)
        assert np.array_equal(bits, want), (B, S)


@pytest.mark.parametrize("hd", [8, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_attn_op_key_mask(hd, causal):
    from cobra_amd import ops

    torch.manual_seed(hd + 1)
    B, H = 3, 2
    for S in (1, 31, 64, 128, 130, 300):
        D = H * hd
        qkv = torch.randn(B * S, 3 * D, device=DEV).half()
        m = token_mask(B, S, seed=S, left_aligned=False).to(DEV)
        got = ops.attn(qkv, B, S, H, hd, hd ** -0.5, causal=causal, key_mask=m).float()
        q, k, v = qkv.float().view(B, S, 3, H, hd).permute(2, 0, 3, 1, 4)
        s = (q @ k.transpose(-2, -1).contiguous()) * hd ** -0.5
        dead = ~m[:, None, None, :]
        if causal:
            dead = dead | torch.ones(S, S, dtype=torch.bool, device=DEV).triu(1)
        s = s.masked_fill(dead, float("-inf"))
        p = torch.softmax(s, -1).nan_to_num(0.0)  # a query without a valid key: zero row
        want = (p @ v).transpose(1, 2).reshape(B * S, D)
        err = (got - want).abs().max().item()
        assert torch.allclose(got, want, atol=2e-3, rtol=1e-2), (hd, S, causal, err)


@pytest.mark.parametrize("M,N,K", [(8192, 1024, 1024), (300, 96, 40), (4096, 256, 128)])
def test_linear_epilogue_flags(M, N, K):
    """GELU, branch mask and residual mask against fp32 torch, on both GEMM kernels."""
    from cobra_amd import ops

    torch.manual_seed(M + N)
    a = (torch.randn(M, K, device=DEV) * 0.5).half()
    w = (torch.randn(N, K, device=DEV) / K ** 0.5).half()
    b = torch.randn(N, device=DEV)
    r = torch.randn(M, N, device=DEV)
    m = torch.rand(M, device=DEV) < 0.7
    prod = a.float() @ w.float().t() + b
    mf = m.float()[:, None]

    got = ops.linear(a, w, b, gelu=True, out_fp32=True)
    assert torch.allclose(got, F.gelu(prod), atol=1e-3, rtol=1e-3), (got - F.gelu(prod)).abs().max()
    got = ops.linear(a, w, b, out_fp32=True, resid=r, rmask=m)
    assert torch.allclose(got, (prod + r) * mf, atol=1e-3, rtol=1e-3)
    assert torch.equal(got[~m], torch.zeros_like(got[~m]))
    got = ops.linear(a, w, b, out_fp32=True, resid=r, rmask=m, mask_branch=True)
    assert torch.allclose(got, prod * mf + r, atol=1e-3, rtol=1e-3)
    assert torch.equal(got[~m], r[~m])
    got = ops.linear(a, w, b, gelu=True, resid=r.half(), rmask=m, mask_branch=True)
    assert torch.allclose(got.float(), F.gelu(prod) * mf + r.half().float(), atol=1e-2, rtol=1e-2)


def test_linear_ln_and_add_ln_masks():
    from cobra_amd import ops

    torch.manual_seed(9)
    for M, N, K in [(2048, 128, 128), (40000, 64, 64), (999, 96, 128)]:
        _check_linear_ln_masks(ops, M, N, K)

    M, N = 2048, 128
    g, be = torch.rand(N, device=DEV) + 0.5, torch.randn(N, device=DEV)
    m = torch.rand(M, device=DEV) < 0.7
    mf = m.float()[:, None]
    ln = lambda t: F.layer_norm(t, (N,), g, be, 1e-5)  # noqa: E731
    x = torch.randn(M, N, device=DEV)
    br = torch.randn(M, N, device=DEV).half()
    r, y = ops.add_ln(x, br, m, g, be, cast_fp16=False, store_resid=True, mask_out=True)
    want_r = (x + br.float()) * mf
    assert torch.equal(r, want_r)
    assert torch.allclose(y, ln(want_r) * mf, atol=2e-5, rtol=1e-4)
    r, y = ops.add_ln(x, None, m, g, be, cast_fp16=False, store_resid=False, mask_out=False)
    assert r is None
    assert torch.allclose(y, ln(x), atol=2e-5, rtol=1e-4)  # no store, no mask_out: the mask is unused


def _check_linear_ln_masks(ops, M, N, K):
    a = (torch.randn(M, K, device=DEV) * 0.5).half()
    w = (torch.randn(N, K, device=DEV) / K ** 0.5).half()
    b = torch.randn(N, device=DEV)
    res = torch.randn(M, N, device=DEV)
    g, be = torch.rand(N, device=DEV) + 0.5, torch.randn(N, device=DEV)
    m = torch.rand(M, device=DEV) < 0.7
    mf = m.float()[:, None]
    prod = a.float() @ w.float().t() + b
    ln = lambda t: F.layer_norm(t, (N,), g, be, 1e-5)  # noqa: E731

    r, y = ops.linear_ln(a, w, b, res, g, be, rmask=m, norm_fp16=False, mask_out=True)
    want_r = (prod + res) * mf
    assert torch.allclose(r, want_r, atol=1e-3, rtol=1e-3)
    assert torch.allclose(y, ln(want_r) * mf, atol=2e-3, rtol=1e-3)
    r, y = ops.linear_ln(a, w, b, res, g, be, rmask=m, norm_fp16=False, mask_branch=True)
    want_r = prod * mf + res
    assert torch.equal(r[~m], res[~m])
    assert torch.allclose(y, ln(want_r), atol=2e-3, rtol=1e-3)
