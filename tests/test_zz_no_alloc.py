"""The allocation-free entry point ``cobra_layer_fwd_noalloc`` against ``cobra_layer_fwd``.

Both run the same kernels; the only difference is where the STAGED plan's
intermediates live (the library's per-device scratch instead of a caller
workspace), so y and the residual must be equal bit for bit.  Calls run in a
row on one stream, each followed by a smaller one, because every call shares
the device's scratch and finds the previous call's contents there.
"""

import pytest
import torch

from oracle import compare_outputs, make_input

from _gpu_util import DEV, build_pair, log, oracle_on

pytestmark = pytest.mark.gpu


def _packed(mod, dtype=torch.float16):
    return mod._packed(dtype)


def _run_both(mod, B, S, causal, masked, seed, resid, dtype=torch.float16):
    from cobra_amd import ops

    D = mod.attention.d_model
    H = mod.attention.num_heads
    p = _packed(mod, dtype)
    x = make_input(B, S, D, seed=seed).to(dtype).to(DEV)
    m = None
    if masked:
        m = torch.rand(B, S, generator=torch.Generator().manual_seed(seed)) < 0.8
        m[:, 0] = True
        m = m.to(DEV).view(torch.uint8)
    ws = torch.empty(ops.layer_workspace_bytes(B, S, D, H, masked, x.dtype), dtype=torch.uint8, device=DEV)
    y_ws, y_na = torch.empty_like(x), torch.full_like(x, float("nan"))
    r_ws = torch.empty(B, S, D, dtype=torch.float32, device=DEV) if resid else None
    r_na = torch.full_like(r_ws, float("nan")) if resid else None
    log(f"[noalloc] B{B} S{S} D{D} H{H} causal={causal} masked={masked} {dtype} "
        f"plan={ops.layer_plan(B, S, D, H, masked, dtype)} scratch={ws.numel()} bytes")
    with torch.inference_mode():
        ops.layer_fwd(x, p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln1_w, p.ln1_b, p.ln2_w, p.ln2_b, y_ws, ws, H, causal,
                      resid_out=r_ws, valid_mask=m)
        ops.layer_fwd_noalloc(x, p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln1_w, p.ln1_b, p.ln2_w, p.ln2_b, y_na, H,
                              causal, resid_out=r_na, valid_mask=m)
        torch.cuda.synchronize()
    return x, m, y_ws, y_na, r_ws, r_na


@pytest.mark.parametrize(
    "first,second",
    [
        ((8, 1024, 128, 4), (3, 300, 128, 4)),    # ln_gemm + flash attention + GEMM/LN epilogue
        ((4, 128, 1024, 4), (2, 77, 256, 2)),     # d_model > 128: residual through the scratch, LN pass
        ((2, 128, 128, 4), (1, 50, 128, 4)),      # FUSED plan: no scratch used at all
        # PADDED plan (head_dim 12): the padded weight copies live in the scratch too, and
        # LN1 must zero the pad columns that the larger first call left behind
        ((4, 200, 120, 4), (3, 50, 96, 8)),
    ],
)
@pytest.mark.parametrize("causal,masked", [(False, False), (True, True)])
def test_noalloc_equals_workspace_entry_point(first, second, causal, masked):
    for i, (B, S, D, H) in enumerate((first, second)):
        ref, mod = build_pair(D, H, seed=i)
        # first call without the residual output (at d_model > 128 the residual then
        # goes through the scratch), the second with it
        x, m, y_ws, y_na, r_ws, r_na = _run_both(mod, B, S, causal, masked, seed=40 + i, resid=i == 1)
        assert torch.equal(y_ws, y_na), (B, S, D, H)
        if i == 1:  # the smaller second call: residual too, and against the oracle
            assert torch.equal(r_ws, r_na), (B, S, D, H)
            want = oracle_on(ref, x.float().cpu(), causal, "cpu", mask=None if m is None else m.bool().cpu())
            res = compare_outputs(want, y_na.float().cpu())
            log(f"[noalloc] second call vs oracle: max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
            assert res.passed, res


@pytest.mark.parametrize("first,second", [((8, 256, 128, 4), (3, 100, 256, 4)), ((4, 100, 120, 4), (2, 50, 96, 8))])
def test_noalloc_bf16(first, second):
    """bf16 activations (the staged and padded plans with bf16 operands) through the
    scratch: bit-equal to the workspace entry point, and within the bf16 gate (the
    reference's scaled by bf16's unit roundoff over fp16's: abs 1.6e-2 or rel 2e-2) of the
    oracle on the same bf16-rounded weights."""
    for i, (B, S, D, H) in enumerate((first, second)):
        ref, mod = build_pair(D, H, seed=i, dtype=torch.bfloat16)
        x, m, y_ws, y_na, r_ws, r_na = _run_both(mod, B, S, True, True, seed=50 + i, resid=i == 1,
                                                 dtype=torch.bfloat16)
        assert torch.equal(y_ws, y_na), (B, S, D, H)
        if i == 1:
            assert torch.equal(r_ws, r_na), (B, S, D, H)
            want = oracle_on(ref, x.float().cpu(), True, "cpu", mask=m.bool().cpu())
            res = compare_outputs(want, y_na.float().cpu(), rtol=2e-2, atol=1.6e-2)
            log(f"[noalloc] bf16 second call vs oracle: max_abs={res.max_abs_error:.3e} "
                f"failed={res.failed_elements}")
            assert res.passed, res


def test_noalloc_rejects_shapes_beyond_its_scratch():
    """A shape whose workspace exceeds the scratch is refused before anything is
    enqueued: by the wrapper with a message, and by the C entry point with a code."""
    from cobra_amd import _lib, ops

    B, S, D, H = 200, 1024, 128, 4
    assert ops.layer_workspace_bytes(B, S, D, H) > ops.NOALLOC_MAX_BYTES
    _, mod = build_pair(D, H)
    p = _packed(mod)
    x = torch.zeros(B, S, D, dtype=torch.float16, device=DEV)
    y = torch.empty_like(x)
    with pytest.raises(ValueError, match="scratch"):
        ops.layer_fwd_noalloc(x, p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln1_w, p.ln1_b, p.ln2_w, p.ln2_b, y, H, False)
    code = _lib.lib().cobra_layer_fwd_noalloc(
        x.data_ptr(), _lib.F16, None, p.w_qkv.data_ptr(), p.b_qkv.data_ptr(), p.w_o.data_ptr(), p.b_o.data_ptr(),
        None, None, p.ln2_w.data_ptr(), p.ln2_b.data_ptr(), y.data_ptr(), None, B, S, D, H, 0, 1e-5, None)
    assert code != 0
    # the largest batch that fits still runs
    B_fit = max(b for b in range(1, B) if ops.layer_workspace_bytes(b, S, D, H) <= ops.NOALLOC_MAX_BYTES)
    xs = make_input(B_fit, S, D, seed=7).half().to(DEV)
    ya, yb = torch.empty_like(xs), torch.empty_like(xs)
    ws = torch.empty(ops.layer_workspace_bytes(B_fit, S, D, H), dtype=torch.uint8, device=DEV)
    with torch.inference_mode():
        ops.layer_fwd(xs, p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln1_w, p.ln1_b, p.ln2_w, p.ln2_b, ya, ws, H, False)
        ops.layer_fwd_noalloc(xs, p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln1_w, p.ln1_b, p.ln2_w, p.ln2_b, yb, H, False)
        torch.cuda.synchronize()
    log(f"[noalloc] largest batch at S{S} D{D}: {B_fit}")
    assert torch.equal(ya, yb)
