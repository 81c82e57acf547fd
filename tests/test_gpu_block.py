"""GPU parity of the whole-block launch (``cobra_block_fwd``): one transformer block of
the reference's fused stack (TTB:1216-1267) in one kernel.

The block gets h = norm1(r) rounded to fp16 (what the previous block's epilogue hands
it) and the fp32 residual r.  The expected values come from the oracle's own block
modules (``oracle/model.py``: attention, norm2, ffn_in, GELU, ffn_out, the block row
mask, then the next norm) applied in fp32 to the same fp16 h and fp32 r, with
fp16-rounded weights; gate: the reference's (abs <= 2e-3 or rel <= 2e-2, zero failing
elements).  Also: in-place residual update == out-of-place bit for bit, fp32 output ==
fp16 output before rounding, and argument checks.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import OracleTransformerConfig, compare_outputs, make_input, make_model, quantize_like

from _gpu_util import DEV, log

pytestmark = pytest.mark.gpu

D = FF = 128


def _mask(B, S, seed):
    m = torch.rand(B, S, generator=torch.Generator().manual_seed(seed)) > 0.3
    m[:, 0] = True
    return m


class Case:
    def __init__(self, B, S, H, causal, masked, seed=0, last=False, affine_seed=None, offset=0.0):
        self.B, self.S, self.H, self.causal, self.masked, self.last = B, S, H, causal, masked, last
        ref = make_model(OracleTransformerConfig(B, S, D, H, FF, 2, causal), seed=seed)
        if affine_seed is not None:  # non-trivial LayerNorm parameters
            g = torch.Generator().manual_seed(affine_seed)
            with torch.no_grad():
                for ln in (ref.layers[0].norm1, ref.layers[0].norm2, ref.layers[1].norm1, ref.final_norm):
                    ln.weight.copy_(torch.rand(D, generator=g) + 0.5)
                    ln.bias.copy_((torch.rand(D, generator=g) - 0.5) * 0.6)
        quantize_like(ref, torch.float16)
        self.ref = ref
        blk = ref.layers[0]
        self.nxt = ref.final_norm if last else ref.layers[1].norm1
        self.r = make_input(B, S, D, seed=seed + 1) + offset
        self.m = _mask(B, S, seed + 2) if masked else None
        with torch.no_grad():
            self.h = F.layer_norm(self.r, (D,), blk.norm1.weight, blk.norm1.bias, 1e-5).half()

    def expected(self):
        """(r2, out) in fp32 from the oracle's modules."""
        blk = self.ref.layers[0]
        with torch.inference_mode():
            r1 = self.r + blk.attention(self.h.float(), self.m, self.causal)
            r2 = r1 + blk.ffn_out(F.gelu(blk.ffn_in(blk.norm2(r1)), approximate="none"))
            if self.m is not None:
                r2 = r2.masked_fill(~self.m[..., None], 0)
            out = self.nxt(r2)
            if self.last and self.m is not None:
                out = out.masked_fill(~self.m[..., None], 0)
        return r2, out

    def run(self, out_dtype=torch.float16, in_place=False):
        from cobra_amd import ops

        blk = self.ref.layers[0]
        T = self.B * self.S

        def w16(t):
            return t.detach().to(DEV, torch.float16).contiguous()

        def f32(t):
            return t.detach().to(DEV, torch.float32).contiguous()

        att = blk.attention
        w_qkv = w16(torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight]))
        b_qkv = f32(torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias]))
        h = self.h.reshape(T, D).to(DEV).contiguous()
        r = self.r.reshape(T, D).to(DEV).contiguous()
        r_out = r if in_place else torch.empty_like(r)
        out = torch.empty(T, D, device=DEV, dtype=out_dtype)
        m = None if self.m is None else self.m.reshape(T).to(DEV).view(torch.uint8).contiguous()
        ops.block_fwd(h, r, w_qkv, b_qkv, w16(att.out_proj.weight), f32(att.out_proj.bias), f32(blk.norm2.weight),
                      f32(blk.norm2.bias), w16(blk.ffn_in.weight), f32(blk.ffn_in.bias), w16(blk.ffn_out.weight),
                      f32(blk.ffn_out.bias), f32(self.nxt.weight), f32(self.nxt.bias), r_out, out, self.B, self.S,
                      self.H, self.causal, valid_mask=m, mask_out=self.last and m is not None)
        torch.cuda.synchronize()
        return r_out.view(self.B, self.S, D).cpu(), out.view(self.B, self.S, D).float().cpu()


# (B, S, H): head_dim 128 / 64 / 32 / 8; full, ragged and single-token sequences; up to
# the largest batch the plan prefers at S 128 (two rounds of workgroups on 256 CUs).
SHAPES = [(3, 128, 4), (2, 77, 2), (4, 32, 1), (3, 100, 16), (2, 1, 4), (64, 128, 4)]


@pytest.mark.parametrize("B,S,H", SHAPES)
@pytest.mark.parametrize("causal,masked", [(False, False), (True, False), (False, True), (True, True)])
def test_block_matches_oracle(B, S, H, causal, masked):
    from cobra_amd import ops

    assert ops.block_plan(B, S, D, H, FF) >= 0
    c = Case(B, S, H, causal, masked, seed=B + S + H)
    log(f"[block] B{B} S{S} H{H} causal={causal} masked={masked}")
    r2, out = c.run()
    want_r, want_o = c.expected()
    rr = compare_outputs(want_r, r2)
    ro = compare_outputs(want_o, out)
    log(f"[block] r: max_abs={rr.max_abs_error:.3e} failed={rr.failed_elements}; "
        f"out: max_abs={ro.max_abs_error:.3e} max_rel={ro.max_relative_error:.3e} failed={ro.failed_elements}")
    assert rr.passed, rr
    assert ro.passed, ro
    if masked:  # padded rows: the block's residual is zero
        assert torch.equal(r2[~c.m], torch.zeros_like(r2[~c.m]))


@pytest.mark.parametrize("H", [1, 4, 16])
def test_block_last_fp32_output_and_in_place(H):
    """The last block: final_norm with the output row mask, fp32 output; the residual
    updated in place; random LayerNorm parameters."""
    c = Case(5, 96, H, True, True, seed=7, last=True, affine_seed=11)
    r_a, out16 = c.run(torch.float16)
    r_b, out32 = c.run(torch.float32, in_place=True)
    assert torch.equal(r_a, r_b)
    assert torch.equal(out32.half().float(), out16)
    want_r, want_o = c.expected()
    res = compare_outputs(want_o, out32)
    log(f"[block last] H{H} max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
    assert res.passed, res
    assert compare_outputs(want_r, r_b).passed
    pad = ~c.m
    assert torch.equal(out32[pad], torch.zeros_like(out32[pad]))


@pytest.mark.parametrize("offset", [300.0, 1000.0])
@pytest.mark.parametrize("H,causal,masked,last", [(4, False, False, False), (16, True, True, False),
                                                  (1, True, True, True)])
def test_block_residual_mean_hundreds_of_deviations(H, causal, masked, last, offset):
    """r = offset + N(0, 1): LN2 and the next norm see rows whose mean is hundreds of
    standard deviations off zero (their statistics are shifted by one element of the
    residual row); padded rows still come out exactly zero in r."""
    c = Case(4, 100, H, causal, masked, seed=21, last=last, affine_seed=5, offset=offset)
    log(f"[block offset {offset:g}] H{H} causal={causal} masked={masked} last={last}")
    r2, out = c.run(torch.float32 if last else torch.float16)
    want_r, want_o = c.expected()
    rr = compare_outputs(want_r, r2)
    ro = compare_outputs(want_o, out)
    log(f"[block offset {offset:g}] r failed={rr.failed_elements}; out max_abs={ro.max_abs_error:.3e} "
        f"failed={ro.failed_elements}")
    assert rr.passed, rr
    assert ro.passed, ro
    if masked:
        assert torch.equal(r2[~c.m], torch.zeros_like(r2[~c.m]))


def test_block_rejects_bad_arguments():
    from cobra_amd import ops
    from cobra_amd._lib import CobraError

    assert ops.block_plan(2, 128, 64, 2, 64) == -1   # d_model 64: not taken
    assert ops.block_plan(2, 129, 128, 4, 128) == -1  # more than 128 tokens
    assert ops.block_plan(2, 128, 128, 4, 512) == -1  # ffn_dim != d_model
    assert ops.block_plan(4096, 128, 128, 4, 128) == 0  # taken, not preferred
    c = Case(2, 16, 4, False, False)
    T = 32
    h = c.h.reshape(T, D).to(DEV)
    r = c.r.reshape(T, D).to(DEV)
    w = torch.zeros(3 * D, D, device=DEV, dtype=torch.float16)
    v = torch.zeros(3 * D, device=DEV)
    wd = torch.zeros(D, D, device=DEV, dtype=torch.float16)
    vd = torch.zeros(D, device=DEV)
    out = torch.empty(T, D, device=DEV, dtype=torch.float16)
    with pytest.raises(CobraError):  # out aliasing h
        ops.block_fwd(h, r, w, v, wd, vd, vd, vd, wd, vd, wd, vd, vd, vd, r, h, 2, 16, 4, False)
    with pytest.raises(CobraError):  # mask_out without a mask
        ops.block_fwd(h, r, w, v, wd, vd, vd, vd, wd, vd, wd, vd, vd, vd, r, out, 2, 16, 4, False, mask_out=True)
    torch.cuda.synchronize()
