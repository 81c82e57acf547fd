"""GPU parity of the padded staged plan: head_dim or d_model not a multiple of 8.

The reference runs every shape its config validation accepts (d_model % heads == 0):
its attention kernel pads head_dim to HD_PAD = max(16, next_pow2(head_dim)) with masked
loads (torch_transformer_benchmark.py:578, 763-765) and its GEMMs mask their loads.
Here the library lays the weights out zero-padded (each head's rows to a multiple of
8 dimensions, d_model likewise) and runs the staged plan's vector kernels on them;
LayerNorm runs element-wise over the true width.  Every case goes through the drop-in
module against the fp32 oracle with the reference's gate (abs <= 2e-3 or rel <= 2e-2,
zero failing elements), causal or not, with token masks, fp16 and fp32 activations,
the residual output, random LayerNorm parameters and a large input mean.
"""

import pytest
import torch

from oracle import compare_outputs, make_input

from _gpu_util import DEV, build_pair, log, oracle_on, randomise_affine

pytestmark = pytest.mark.gpu

# (B, S, D, H): head_dim 12, 25, 12, 4, 9, 65, 3; d_model 96, 100, 36, 20, 9, 260, 24
SHAPES = [(3, 50, 96, 8), (2, 77, 100, 4), (4, 33, 36, 3), (2, 40, 20, 5), (3, 19, 9, 1), (2, 130, 260, 4),
          (5, 128, 24, 8)]


def _mask(B, S, seed):
    m = torch.rand(B, S, generator=torch.Generator().manual_seed(seed)) > 0.25
    m[:, 0] = True
    return m


@pytest.mark.parametrize("B,S,D,H", SHAPES)
@pytest.mark.parametrize("causal,masked", [(False, False), (True, False), (False, True), (True, True)])
def test_padded_plan_matches_oracle(B, S, D, H, causal, masked):
    from cobra_amd import ops

    assert ops.layer_plan(B, S, D, H, masked) == ops.PLAN_PADDED
    ref, mod = build_pair(D, H, seed=1)
    x = make_input(B, S, D, seed=2).half()
    m = _mask(B, S, 3) if masked else None
    log(f"[padded] B{B} S{S} D{D} H{H} hd{D // H} causal={causal} masked={masked}")
    with torch.inference_mode():
        r, y = mod(x.to(DEV), valid_token_mask=None if m is None else m.to(DEV), causal=causal, return_residual=True)
        torch.cuda.synchronize()
    assert mod.plan == ops.PLAN_PADDED
    want_r, want_y = oracle_on(ref, x.float(), causal, "cpu", return_residual=True, mask=m)
    res = compare_outputs(want_y, y.float().cpu())
    log(f"[padded] max_abs={res.max_abs_error:.3e} max_rel={res.max_relative_error:.3e} failed={res.failed_elements}")
    assert res.passed, res
    assert compare_outputs(want_r, r.cpu()).passed
    if masked:  # padded rows: the attention branch is zeroed, r = x
        pad = ~m
        assert torch.equal(r.cpu()[pad], x.float()[pad])


@pytest.mark.parametrize("B,S,D,H", [(3, 50, 96, 8), (2, 77, 100, 4), (4, 33, 36, 3)])
def test_padded_plan_fp32_random_affine_large_mean(B, S, D, H):
    """fp32 activations against the unrounded oracle, random LayerNorm / bias parameters,
    and an input whose mean is six standard deviations off zero."""
    ref, mod = build_pair(D, H, seed=4, dtype=torch.float32)
    randomise_affine(ref, 5)
    mod.load_state_dict(ref.state_dict(), strict=True)
    x = 3.0 + 0.5 * make_input(B, S, D, seed=6)
    with torch.inference_mode():
        y = mod(x.to(DEV))
        torch.cuda.synchronize()
    want = oracle_on(ref, x, False, "cpu")
    res = compare_outputs(want, y.cpu())
    log(f"[padded fp32] B{B} S{S} D{D} H{H} max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
    assert res.passed, res


@pytest.mark.parametrize("d", [9, 36, 100, 260, 1000])
@pytest.mark.parametrize("branch", [False, True])
def test_add_ln_any_width(d, branch):
    """cobra_ln_fwd at widths that are not a multiple of 8 (the element-wise kernel)."""
    from cobra_amd import ops

    torch.manual_seed(d)
    M = 37
    x = torch.randn(M, d, device=DEV).half()
    br = torch.randn(M, d, device=DEV) if branch else None
    w = torch.rand(d, device=DEV) + 0.5
    b = torch.randn(d, device=DEV) * 0.1
    r, y = ops.add_ln(x, br, None, w, b, True, 1e-5, True)
    rr = x.float() + (br if branch else 0)
    want = torch.nn.functional.layer_norm(rr, (d,), w, b, 1e-5)
    assert torch.allclose(r, rr, atol=1e-6, rtol=0)
    assert torch.allclose(y.float(), want, atol=2e-3, rtol=1e-3), (d, (y.float() - want).abs().max())


@pytest.mark.parametrize("B,S,D,H,masked", [(3, 50, 96, 8, True), (2, 130, 260, 4, False)])
def test_module_padding_once_equals_the_abi_padded_plan(B, S, D, H, masked):
    """The module pads its weights once per parameter version and runs the chain of op
    calls; cobra_layer_fwd's padded plan (the C ABI, which takes the unpadded weights)
    lays them out on every call and runs the same kernels: y and r equal bit for bit."""
    from cobra_amd import ops

    _, mod = build_pair(D, H, seed=4)
    x = make_input(B, S, D, seed=5).half().to(DEV)
    m = _mask(B, S, 6).to(DEV) if masked else None
    with torch.inference_mode():
        r1, y1 = mod(x, valid_token_mask=m, return_residual=True)
        p = mod._packed()
        assert p.pad is not None
        mb = None if m is None else m.view(torch.uint8)
        ws = torch.empty(ops.layer_workspace_bytes(B, S, D, H, masked, x.dtype), dtype=torch.uint8, device=DEV)
        y2 = torch.empty_like(x)
        r2 = torch.empty(B, S, D, dtype=torch.float32, device=DEV)
        ops.layer_fwd(x, p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln1_w, p.ln1_b, p.ln2_w, p.ln2_b, y2, ws, H, False,
                      resid_out=r2, valid_mask=mb)
        torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(r1, r2)
