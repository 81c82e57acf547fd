"""Pins the fp32 oracle (oracle/layer.py) without importing the reference.

The reference holds no golden vectors for this path, so each check below is a
closed form, an invariant, or agreement with an independent library routine,
chosen so that a plausible transcription mistake fails at least one of them.
``test_planted_mistakes_are_caught`` plants such mistakes in copies of the
oracle and asserts that the checks notice.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import OracleAttentionSublayer, make_input, make_sublayer
from oracle.cases import CONFIGS, make_sequence, oracle_forward, quantize_like


def _layer64(d=16, h=4, seed=0):
    torch.manual_seed(seed)
    layer = OracleAttentionSublayer(d, h).double().eval()
    with torch.no_grad():  # non-trivial LayerNorm affine so gamma/beta are exercised
        for ln in (layer.norm1, layer.norm2):
            ln.weight.uniform_(0.5, 1.5)
            ln.bias.uniform_(-0.5, 0.5)
    return layer


def _mha_reference(layer, h_in, causal):
    """Attention via torch's own multi-head attention routine (fp64).

    ``F.multi_head_attention_forward`` is an independent implementation with
    packed in-projection and (seq, batch, embed) layout.
    """
    att = layer.attention
    b, s, d = h_in.shape
    w_in = torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight])
    b_in = torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias])
    mask = None
    if causal:
        mask = torch.ones(s, s, dtype=torch.bool).triu(1)
    t = h_in.transpose(0, 1)
    out, _ = F.multi_head_attention_forward(
        t, t, t, d, att.num_heads, w_in, b_in, None, None, False, 0.0,
        att.out_proj.weight, att.out_proj.bias, training=False,
        need_weights=False, attn_mask=mask,
    )
    return out.transpose(0, 1)


# The oracle keeps the reference's ``softmax(scores.float())`` (TTB:112), so an
# fp64 run still takes its softmax in fp32: comparisons that pass through the
# softmax carry fp32-level error.  Every planted mistake below moves outputs by
# more than 1e-3.
SOFTMAX_TOL = 1e-6


def _mha_mismatch(layer, x, causal):
    with torch.no_grad():
        h_in = layer.norm1(x)
        ours = layer.attention(h_in, None, causal)
        ref = _mha_reference(layer, h_in, causal)
    return (ours - ref).abs().max().item()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d,h", [(16, 4), (24, 3), (32, 1), (32, 8)])
def test_attention_matches_library_mha(d, h, causal):
    """Head split/merge order, W vs W^T, biases, scale, softmax axis, mask side."""
    layer = _layer64(d, h)
    x = torch.randn(3, 7, d, dtype=torch.float64)
    assert _mha_mismatch(layer, x, causal) < SOFTMAX_TOL


def test_layernorm_closed_form():
    """Row c + [a, -a, a, -a, ...]: biased variance a^2, eps inside the sqrt."""
    d, a, c, eps = 8, 0.75, 3.0, 1e-5
    layer = OracleAttentionSublayer(d, 2).double()
    row = torch.tensor([a if i % 2 == 0 else -a for i in range(d)], dtype=torch.float64)
    y = layer.norm1((row + c)[None, None, :])[0, 0]
    want = row / math.sqrt(a * a + eps)
    assert torch.allclose(y, want, atol=1e-14, rtol=0)


def test_layernorm_moments():
    layer = _layer64()
    with torch.no_grad():
        layer.norm2.weight.fill_(1.0)
        layer.norm2.bias.fill_(0.0)
    x = torch.randn(2, 5, 16, dtype=torch.float64) * 3 + 1
    r, y = layer(x, return_residual=True)
    assert torch.allclose(y.mean(-1), torch.zeros(2, 5, dtype=torch.float64), atol=1e-12)
    var = r.var(-1, unbiased=False)
    assert torch.allclose(y.pow(2).mean(-1), var / (var + 1e-5), atol=1e-12)


def _np_linear(lin, t):
    return t @ lin.weight.detach().numpy().T + lin.bias.detach().numpy()


def _np_layernorm(ln, t, eps=1e-5):
    mu = t.mean(-1, keepdims=True)
    var = ((t - mu) ** 2).mean(-1, keepdims=True)
    return (t - mu) / np.sqrt(var + eps) * ln.weight.detach().numpy() + ln.bias.detach().numpy()


def test_single_token_is_value_path():
    """S=1: softmax over one key is 1, so ctx = v and the whole sublayer is
    y = LN2(x + out(v(LN1(x)))) -- catches a dropped residual or bias."""
    layer = _layer64(16, 4)
    x = torch.randn(4, 1, 16, dtype=torch.float64)
    with torch.no_grad():
        r, y = layer(x, return_residual=True)
    xn = x.numpy()
    att = layer.attention
    want_r = xn + _np_linear(att.out_proj, _np_linear(att.v_proj, _np_layernorm(layer.norm1, xn)))
    want_y = _np_layernorm(layer.norm2, want_r)
    assert np.abs(r.numpy() - want_r).max() < 1e-12
    assert np.abs(y.numpy() - want_y).max() < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_zero_query_gives_uniform_attention(causal):
    """W_q = b_q = 0 makes every score 0: ctx is the key-mean of v
    (non-causal) or the running prefix mean (causal)."""
    layer = _layer64(16, 4)
    with torch.no_grad():
        layer.attention.q_proj.weight.zero_()
        layer.attention.q_proj.bias.zero_()
    x = torch.randn(2, 6, 16, dtype=torch.float64)
    with torch.no_grad():
        out = layer.attention(layer.norm1(x), None, causal).numpy()
    att = layer.attention
    v = _np_linear(att.v_proj, _np_layernorm(layer.norm1, x.numpy()))
    if causal:
        ctx = np.cumsum(v, axis=1) / np.arange(1, 7)[None, :, None]
    else:
        ctx = np.repeat(v.mean(axis=1, keepdims=True), 6, axis=1)
    want = _np_linear(att.out_proj, ctx)
    assert np.abs(out - want).max() < SOFTMAX_TOL


def test_causal_prefix_invariance():
    """Under causality row i depends only on rows <= i (mask side check)."""
    layer = _layer64(16, 4)
    x = torch.randn(2, 9, 16, dtype=torch.float64)
    with torch.no_grad():
        full = layer(x, causal=True)
        for k in (1, 4, 9):
            assert torch.allclose(layer(x[:, :k], causal=True), full[:, :k], atol=SOFTMAX_TOL, rtol=0)
        # row 0 attends only to key 0: equal to the S=1 computation
        assert torch.allclose(layer(x[:, :1], causal=False), full[:, :1], atol=SOFTMAX_TOL, rtol=0)
        # non-causal rows do see the future
        assert not torch.allclose(layer(x[:, :4]), layer(x)[:, :4], atol=1e-6)


def test_noncausal_permutation_equivariance():
    layer = _layer64(16, 4)
    x = torch.randn(2, 8, 16, dtype=torch.float64)
    perm = torch.randperm(8)
    with torch.no_grad():
        assert torch.allclose(layer(x)[:, perm], layer(x[:, perm]), atol=SOFTMAX_TOL, rtol=0)


def test_batch_independence():
    layer = _layer64(16, 4)
    x = torch.randn(5, 7, 16, dtype=torch.float64)
    with torch.no_grad():
        full = layer(x)
        for b in range(5):
            assert torch.allclose(layer(x[b : b + 1]), full[b : b + 1], atol=SOFTMAX_TOL, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape,block", [((2, 128, 32, 4), 32), ((3, 333, 96, 3), 128), ((1, 64, 16, 2), 7)])
def test_query_blocked_equals_full(shape, block, causal):
    """The blocked oracle (reference_chunked.py:73-128) equals the full one."""
    b, s, d, h = shape
    torch.manual_seed(1234)
    layer = OracleAttentionSublayer(d, h).eval()
    x = make_input(b, s, d, seed=1234)
    with torch.no_grad():
        a = layer(x, causal=causal)
        c = layer(x, causal=causal, block_q=block)
    assert (a - c).abs().max().item() <= 1e-5


def test_seeded_construction_draw_order():
    """manual_seed then norm1, q, k, v, out, norm2 (TTB:129-131, 73-76)."""
    layer = make_sublayer(32, 4, seed=0)
    torch.manual_seed(0)
    torch.nn.LayerNorm(32)
    draws = [torch.nn.Linear(32, 32) for _ in range(4)]
    att = layer.attention
    for got, ref in zip((att.q_proj, att.k_proj, att.v_proj, att.out_proj), draws):
        assert torch.equal(got.weight, ref.weight) and torch.equal(got.bias, ref.bias)
    bound = 1 / math.sqrt(32)
    assert att.q_proj.weight.abs().max() <= bound
    assert torch.equal(layer.norm1.weight, torch.ones(32)) and torch.equal(layer.norm2.bias, torch.zeros(32))


def test_inputs_are_seeded_and_per_sequence_independent():
    a = make_input(2, 4, 8, seed=0)
    assert torch.equal(a, make_input(2, 4, 8, seed=0))
    assert not torch.equal(a, make_input(2, 4, 8, seed=1))
    s3 = make_sequence(3, 16, 8)
    assert torch.equal(s3, make_sequence(3, 16, 8))
    assert not torch.equal(s3, make_sequence(4, 16, 8))


def test_quantize_like_rounds_to_fp16_grid():
    layer = make_sublayer(16, 4)
    quantize_like(layer, torch.float16)
    for p in layer.parameters():
        assert torch.equal(p, p.half().float())


def test_config_matrix_flops():
    base = CONFIGS["base"]
    assert base.flops() == 8 * 8192 * 128 * 128 + 4 * 64 * 128 * 128 * 128
    assert abs(base.flops() / 1e9 - 1.611) < 1e-3
    assert abs(CONFIGS["gemm"].flops() / 1e9 - 73.0) < 0.1
    assert abs(CONFIGS["long"].flops() / 1e15 - 1.338) < 1e-3


def test_plumbing_config_runs_on_cpu():
    """Config 0: B1 d128 H4 S128, fp32, seed 0, non-causal, on the host."""
    c = CONFIGS["plumbing"]
    layer = make_sublayer(c.d_model, c.heads, seed=0)
    x = make_input(c.batch, c.seq_len, c.d_model, seed=0)
    y = oracle_forward(layer, x)
    assert y.shape == (1, 128, 128) and torch.isfinite(y).all()
    assert abs(y.mean().item()) < 1e-5


def _ragged_mask(b, s, seed=0, left_aligned=False):
    """[b, s] bool: each sequence has 1..s valid tokens, left-aligned (the
    reference harness's padding, TTB:1602-1612) or scattered."""
    g = torch.Generator().manual_seed(seed)
    if left_aligned:
        lengths = torch.randint(1, s + 1, (b,), generator=g)
        return torch.arange(s)[None, :] < lengths[:, None]
    m = torch.rand(b, s, generator=g) < 0.6
    m[:, 0] = True  # at least one valid token per sequence
    return m


def _key_mask_mismatch(layer, x, mask, causal):
    """Oracle attention under a token mask vs torch's multi-head attention with
    key_padding_mask (an independent implementation), on the valid query rows;
    plus the largest magnitude on the padded rows, which must be exactly 0."""
    att = layer.attention
    b, s, d = x.shape
    with torch.no_grad():
        h_in = layer.norm1(x)
        ours = att(h_in, mask, causal)
        w_in = torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight])
        b_in = torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias])
        t = h_in.transpose(0, 1)
        ref, _ = F.multi_head_attention_forward(
            t, t, t, d, att.num_heads, w_in, b_in, None, None, False, 0.0,
            att.out_proj.weight, att.out_proj.bias, training=False, need_weights=False,
            key_padding_mask=~mask, attn_mask=torch.ones(s, s, dtype=torch.bool).triu(1) if causal else None,
        )
        ref = ref.transpose(0, 1)
    valid_err = (ours - ref)[mask].abs().max().item()
    padded = ours[~mask].abs().max().item() if (~mask).any() else 0.0
    return valid_err, padded


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("left_aligned", [False, True])
def test_key_mask_matches_library_mha(causal, left_aligned):
    """Padded keys get -inf (TTB:106-109), padded rows a zero output (TTB:121-122)."""
    layer = _layer64(16, 4)
    x = torch.randn(4, 9, 16, dtype=torch.float64)
    mask = _ragged_mask(4, 9, seed=1, left_aligned=left_aligned)
    valid_err, padded = _key_mask_mismatch(layer, x, mask, causal)
    assert valid_err < SOFTMAX_TOL
    assert padded == 0.0


def _compaction_mismatch(layer, x, mask):
    """Non-causal: a sequence's valid rows equal the sublayer run on its valid
    tokens alone (padded keys are as good as absent); padded rows equal
    LN2(x), since their attention output is zero."""
    worst = 0.0
    with torch.no_grad():
        y = layer(x, mask)
        for bi in range(x.shape[0]):
            keep = mask[bi]
            alone = layer(x[bi : bi + 1, keep])
            worst = max(worst, (y[bi, keep] - alone[0]).abs().max().item())
            if (~keep).any():
                worst = max(worst, (y[bi, ~keep] - layer.norm2(x[bi, ~keep])).abs().max().item())
    return worst


def test_key_mask_equals_dropping_padded_tokens():
    layer = _layer64(16, 4)
    x = torch.randn(5, 11, 16, dtype=torch.float64)
    assert _compaction_mismatch(layer, x, _ragged_mask(5, 11, seed=2)) < SOFTMAX_TOL


def test_left_padding_is_a_no_op_for_valid_rows_under_causality():
    """The reference's elision argument (TTB:1110-1115): with left-aligned
    padding a valid causal query only sees valid keys, so its row equals the
    unmasked causal row."""
    layer = _layer64(16, 4)
    x = torch.randn(4, 10, 16, dtype=torch.float64)
    mask = _ragged_mask(4, 10, seed=3, left_aligned=True)
    with torch.no_grad():
        masked = layer(x, mask, causal=True)
        plain = layer(x, None, causal=True)
    assert (masked - plain)[mask].abs().max().item() < SOFTMAX_TOL


@pytest.mark.parametrize(
    "mistake",
    ["no_v_bias", "scale_sqrt_d", "heads_interleaved", "softmax_axis", "causal_lower", "no_residual", "unbiased_var",
     "mask_on_queries", "no_output_zeroing"],
)
def test_planted_mistakes_are_caught(mistake, monkeypatch):
    """Each mistake is planted in the oracle (CPU only); some check above must fail."""
    from oracle import layer as L

    layer = _layer64(16, 4)
    x = torch.randn(2, 6, 16, dtype=torch.float64)
    att = layer.attention

    if mistake == "no_v_bias":
        monkeypatch.setattr(att.v_proj, "forward", lambda t: t @ att.v_proj.weight.t())
    elif mistake == "scale_sqrt_d":
        att.scale = att.d_model ** -0.5
    elif mistake == "heads_interleaved":
        def bad_heads(t, _a=att):
            b, s, _ = t.shape
            return t.view(b, s, _a.head_dim, _a.num_heads).permute(0, 3, 1, 2).contiguous()
        monkeypatch.setattr(att, "_heads", bad_heads)
    elif mistake == "softmax_axis":
        orig = torch.softmax
        monkeypatch.setattr(L.torch, "softmax", lambda t, dim: orig(t, dim=-2))
    elif mistake == "causal_lower":
        orig_fill = torch.Tensor.masked_fill
        monkeypatch.setattr(
            L.OracleSelfAttention, "_probs_times_v",
            lambda self, q, k, v, q0, m, causal, od: (
                torch.matmul(
                    torch.softmax(
                        orig_fill(
                            torch.matmul(q, k.transpose(-2, -1)) * self.scale,
                            torch.ones(q.shape[-2], k.shape[-2], dtype=torch.bool).tril(-1) if causal
                            else torch.zeros(q.shape[-2], k.shape[-2], dtype=torch.bool),
                            float("-inf"),
                        ).float(), dim=-1,
                    ).to(od), v,
                )
            ),
        )
    elif mistake == "mask_on_queries":
        orig_pv = L.OracleSelfAttention._probs_times_v

        def rows_masked(self, q, k, v, q0, m, causal, od):
            # masks score rows (queries) instead of columns (keys)
            if m is None:
                return orig_pv(self, q, k, v, q0, m, causal, od)
            out = orig_pv(self, q, k, v, q0, None, causal, od)
            return out.masked_fill(~m[:, None, q0 : q0 + q.shape[-2], None], 0)

        monkeypatch.setattr(L.OracleSelfAttention, "_probs_times_v", rows_masked)
    elif mistake == "no_output_zeroing":
        orig_fwd = L.OracleSelfAttention.forward
        monkeypatch.setattr(
            L.OracleSelfAttention, "forward",
            lambda self, x, m=None, causal=False, block_q=None: orig_fwd(self, x, m, causal, block_q)
            + (0.0 if m is None else (~m[..., None]).to(x.dtype) * self.out_proj.bias),
        )
    caught = False
    if mistake in ("mask_on_queries", "no_output_zeroing"):
        mask = _ragged_mask(2, 6, seed=4)
        valid_err, padded = _key_mask_mismatch(layer, x, mask, False)
        caught = valid_err > 1e-3 or padded > 1e-3
    elif mistake in ("no_v_bias", "scale_sqrt_d", "heads_interleaved", "softmax_axis"):
        caught = _mha_mismatch(layer, x, False) > 1e-3
    elif mistake == "causal_lower":
        caught = _mha_mismatch(layer, x, True) > 1e-3
    elif mistake == "no_residual":
        def no_residual(self, x, valid_token_mask=None, causal=False, return_residual=False, block_q=None):
            r = self.attention(self.norm1(x), valid_token_mask, causal, block_q)
            return (r, self.norm2(r)) if return_residual else self.norm2(r)

        monkeypatch.setattr(OracleAttentionSublayer, "forward", no_residual)
        try:
            test_single_token_is_value_path()
        except AssertionError:
            caught = True
    elif mistake == "unbiased_var":
        def bad_ln(t, _ln=layer.norm1):
            mu = t.mean(-1, keepdim=True)
            var = t.var(-1, keepdim=True, unbiased=True)
            return (t - mu) / torch.sqrt(var + _ln.eps) * _ln.weight + _ln.bias
        monkeypatch.setattr(torch.nn.LayerNorm, "forward", lambda self, t: bad_ln(t, self))
        try:
            test_layernorm_closed_form()
        except AssertionError:
            caught = True
    assert caught, f"planted mistake '{mistake}' went unnoticed"


# ---------------------------------------------------------------------------
# The whole stack (oracle/model.py, TTB:126-173)
# ---------------------------------------------------------------------------

from oracle import OracleTransformerConfig, make_model  # noqa: E402


def _model64(b, s, d, h, f, n, causal, seed=0):
    cfg = OracleTransformerConfig(b, s, d, h, f, n, causal)
    model = make_model(cfg, seed=seed).double()
    with torch.no_grad():  # non-trivial LayerNorm affine so gamma/beta are exercised
        for name, p in model.named_parameters():
            if "norm" in name:
                p.uniform_(0.5, 1.5) if name.endswith("weight") else p.uniform_(-0.5, 0.5)
    return model


def _np_gelu_erf(t):
    return 0.5 * t * (1.0 + np.vectorize(math.erf)(t / math.sqrt(2.0)))


def _np_block_s1(blk, x):
    """One block at S = 1 in fp64 numpy: attention reduces to the value path (ctx = v)."""
    h = _np_layernorm(blk.norm1, x)
    att = blk.attention
    x1 = x + _np_linear(att.out_proj, _np_linear(att.v_proj, h))
    f = _np_gelu_erf(_np_linear(blk.ffn_in, _np_layernorm(blk.norm2, x1)))
    return x1 + _np_linear(blk.ffn_out, f)


def test_model_single_token_closed_form():
    """S = 1: the stack is LN -> v -> out -> +x -> LN -> W1 -> exact GELU -> W2 -> +x per
    block, then final_norm; restated in numpy fp64 with math.erf."""
    model = _model64(3, 1, 16, 4, 24, 3, causal=True)
    x = torch.randn(3, 1, 16, dtype=torch.float64)
    with torch.no_grad():
        got = model(x).numpy()
    want = x.numpy()
    for blk in model.layers:
        want = _np_block_s1(blk, want)
    want = _np_layernorm(model.final_norm, want)
    assert np.abs(got - want).max() < 1e-10


def test_gelu_is_the_exact_erf_form():
    """The oracle's FFN activation (oracle.model.F.gelu, as the stack calls it) is
    the exact erf GELU; the tanh form differs by more than any rounding would hide."""
    from oracle import model as M

    t = torch.linspace(-6, 6, 241, dtype=torch.float64)
    got = M.F.gelu(t, approximate="none").numpy()
    assert np.abs(got - _np_gelu_erf(t.numpy())).max() < 1e-14


def test_model_attention_half_is_the_sublayer():
    """Each block's first half is the (separately pinned) attention sublayer's residual."""
    model = _model64(2, 7, 16, 4, 32, 1, causal=False)
    sub = OracleAttentionSublayer(16, 4).double()
    blk = model.layers[0]
    sub.norm1.load_state_dict(blk.norm1.state_dict())
    sub.attention.load_state_dict(blk.attention.state_dict())
    sub.norm2.load_state_dict(blk.norm2.state_dict())
    x = torch.randn(2, 7, 16, dtype=torch.float64)
    with torch.no_grad():
        r, _ = sub(x, return_residual=True)
        x1 = x + blk.attention(blk.norm1(x), None, False)
    assert (r - x1).abs().max().item() == 0.0


def _model_mask_checks(model, x, mask):
    """(padded-row max |y|, causal: valid rows vs the unmasked run;
    non-causal: valid rows vs each sequence's valid tokens alone)."""
    with torch.no_grad():
        y = model(x, mask)
        padded = y[~mask].abs().max().item() if (~mask).any() else 0.0
        worst = 0.0
        if model.config.causal:
            plain = model(x)
            worst = (y - plain)[mask].abs().max().item()
        else:
            for bi in range(x.shape[0]):
                keep = mask[bi]
                alone = model(x[bi : bi + 1, keep])
                worst = max(worst, (y[bi, keep] - alone[0]).abs().max().item())
    return padded, worst


@pytest.mark.parametrize("causal", [False, True])
def test_model_masks(causal):
    """Padded rows are exactly 0 (TTB:144-145, 171-172); under causality with
    left-aligned padding the valid rows equal the unmasked run (TTB:1110-1115);
    without causality they equal the model run on the valid tokens alone."""
    model = _model64(4, 9, 16, 4, 24, 2, causal=causal)
    x = torch.randn(4, 9, 16, dtype=torch.float64)
    mask = _ragged_mask(4, 9, seed=7, left_aligned=True)
    x = x.masked_fill(~mask[..., None], 0)
    padded, worst = _model_mask_checks(model, x, mask)
    assert padded == 0.0
    assert worst < SOFTMAX_TOL


# The per-block row mask (TTB:144-145) is not among the plants: with padded keys
# masked and the output rows masked at the end, no output element depends on
# it (the reference's fused path likewise skips the attention output's row
# mask, TTB:1255-1268).
@pytest.mark.parametrize("mistake", ["gelu_tanh", "norm2_after_add", "no_final_norm", "no_output_mask"])
def test_model_planted_mistakes_are_caught(mistake, monkeypatch):
    from oracle import model as M

    if mistake == "gelu_tanh":
        orig_gelu = F.gelu
        monkeypatch.setattr(M.F, "gelu", lambda t, approximate="none": orig_gelu(t, approximate="tanh"))
    elif mistake == "norm2_after_add":
        def bad_block(self, x, m, causal, block_q=None):
            x = x + self.attention(self.norm1(x), m, causal, block_q)
            return self.norm2(x + self.ffn_out(F.gelu(self.ffn_in(x))))
        monkeypatch.setattr(M.OracleTransformerBlock, "forward", bad_block)
    elif mistake == "no_final_norm":
        monkeypatch.setattr(M.OracleTransformer, "forward",
                            lambda self, x, m=None, block_q=None: self.layers[0](x, m, self.config.causal, block_q)
                            if len(self.layers) == 1 else x)
    elif mistake == "no_output_mask":
        def unmasked_output(self, x, m=None, block_q=None):
            for layer in self.layers:
                x = layer(x, m, self.config.causal, block_q)
            return self.final_norm(x)
        monkeypatch.setattr(M.OracleTransformer, "forward", unmasked_output)
    caught = False
    try:
        test_model_single_token_closed_form()
        test_gelu_is_the_exact_erf_form()
        test_model_masks(False)
        test_model_masks(True)
    except AssertionError:
        caught = True
    assert caught, f"planted mistake '{mistake}' went unnoticed"
