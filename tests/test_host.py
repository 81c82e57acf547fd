"""CPU tests of the host side: C-ABI library, planner, drop-in contract."""

import ast
import os
import re

import pytest
import torch

from oracle import OracleAttentionSublayer, make_sublayer

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cobra_amd.h")
PKG = os.path.join(ROOT, "cobra-gpu-kernel_amd", "cobra_amd")


def _header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\*?\s+\*?(cobra_[a-z0-9_]+)\(", text, re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    from cobra_amd import _lib

    lib = _lib.lib()
    names = _header_functions()
    assert len(names) >= 8
    for n in names:
        assert hasattr(lib, n), f"{n} declared in cobra_amd.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert lib.cobra_version() == _lib.ABI_VERSION
    assert lib.cobra_error_string(0)


def test_argument_validation_rejects_before_any_launch():
    """Invalid arguments return an error without touching the GPU."""
    from cobra_amd import _lib

    lib = _lib.lib()
    bad = lib.cobra_ln_fwd(None, 0, None, 0, None, None, None, 0, None, None, 0, 8, 128, 1e-5, None)
    assert bad != 0
    # a mask flag without a mask, an unknown flag
    assert lib.cobra_ln_fwd(256, 0, None, 0, 256, 256, None, _lib.EPI_MASK_OUT, None, 256, 0, 8, 128, 1e-5,
                            None) != 0
    F16, BF16, F32 = _lib.F16, _lib.BF16, _lib.F32
    assert lib.cobra_linear_fwd(256, 256, F16, None, None, 0, 256, 64, 256, 0, 8, 8, 8, None) != 0
    assert lib.cobra_linear_fwd(256, 256, F16, None, None, 0, 256, _lib.EPI_MASK_OUT, 256, 0, 8, 8, 8, None) != 0
    assert lib.cobra_linear_fwd(256, 256, F16, None, None, 0, None, _lib.EPI_MASK_RESID, 256, 0, 8, 8, 8, None) != 0
    assert lib.cobra_linear_fwd(256, 256, F32, None, None, 0, None, 0, 256, F32, 8, 8, 8, None) != 0  # operand type
    assert lib.cobra_linear_fwd(256, 256, BF16, None, None, 0, None, 0, 256, F16, 8, 8, 8, None) != 0  # bf16 -> fp16
    assert lib.cobra_linear_fwd(256, 256, F16, None, None, 0, None, 0, 256, BF16, 8, 8, 8, None) != 0  # fp16 -> bf16
    assert lib.cobra_attn_fwd(16, 16, F16, None, 1, 4, 1, 12, 0.1, 0, None) != 0  # misaligned pointers
    assert lib.cobra_attn_fwd(256, 256, F16, 12, 1, 4, 1, 16, 0.1, 0, None) != 0  # misaligned key bits
    assert lib.cobra_attn_fwd(256, 256, F32, None, 1, 4, 1, 16, 0.1, 0, None) != 0  # operand type
    assert lib.cobra_ln_fwd(256, BF16, 256, BF16, 256, 256, None, 0, None, 256, BF16, 8, 128, 1e-5,
                            None) != 0  # bf16 branch
    assert lib.cobra_layer_plan(2, 16, 128, 4, 0, BF16) == _lib.PLAN_STAGED   # bf16: the staged kernels
    assert lib.cobra_layer_plan(2, 16, 100, 4, 0, BF16) == _lib.PLAN_PADDED
    assert lib.cobra_layer_workspace_bytes(2, 16, 128, 4, 0, BF16) == \
        lib.cobra_layer_workspace_bytes(2, 16, 128, 16, 0, F32)
    assert lib.cobra_mask_bits(256, 12, 1, 4, None) != 0                   # misaligned key bits
    assert lib.cobra_layer_workspace_bytes(2, 16, 528, 2, 0, _lib.F16) == -1       # head_dim 264
    assert lib.cobra_layer_workspace_bytes(2, 16, 100, 3, 0, _lib.F16) == -1       # d_model % heads
    assert lib.cobra_layer_plan(2, 16, 120, 10, 0, _lib.F16) == _lib.PLAN_PADDED   # head_dim 12
    assert lib.cobra_layer_plan(2, 16, 100, 4, 0, _lib.F16) == _lib.PLAN_PADDED    # d_model 100
    assert lib.cobra_layer_workspace_bytes(2, 16, 128, 16, 0, _lib.F32) > 0     # staged plan (head_dim 8, fp32)
    assert lib.cobra_layer_workspace_bytes(2, 16, 128, 4, 0, 7) == -1           # dtype code
    assert lib.cobra_layer_plan(2, 16, 128, 4, 0, _lib.F16) == _lib.PLAN_FUSED
    assert lib.cobra_layer_plan(2, 16, 128, 4, 1, _lib.F16) == _lib.PLAN_FUSED  # the fused kernels take token masks
    assert lib.cobra_layer_plan(2, 16, 128, 4, 0, 7) == -1


def test_empty_calls_return_before_reading_pointers():
    """A call with no rows checks its shape and dtype arguments and returns 0 with NULL
    pointers (the data pointers of empty tensors), before any GPU call; a bad shape or
    dtype is still rejected."""
    from cobra_amd import _lib

    lib = _lib.lib()
    F16, F32 = _lib.F16, _lib.F32
    assert lib.cobra_ln_fwd(None, F16, None, 0, None, None, None, 0, None, None, F16, 0, 128, 1e-5, None) == 0
    assert lib.cobra_ln_fwd(None, 7, None, 0, None, None, None, 0, None, None, F16, 0, 128, 1e-5, None) != 0
    assert lib.cobra_ln_fwd_strided(None, F32, 0, None, 0, 0, None, None, None, 0, None, 0, None, F16, 0, 0, 96,
                                    1e-5, None) == 0
    assert lib.cobra_linear_fwd(None, None, F16, None, None, 0, None, 0, None, F16, 0, 64, 64, None) == 0
    assert lib.cobra_linear_fwd(None, None, F16, None, None, 0, None, 0, None, F16, 0, 0, 64, None) != 0  # N = 0
    assert lib.cobra_linear_ln_fwd(None, None, None, None, 0, None, 0, None, None, None, None, F16, 0, 128, 64,
                                   1e-5, None) == 0
    assert lib.cobra_attn_fwd(None, None, F16, None, 0, 128, 4, 32, 0.1, 0, None) == 0
    assert lib.cobra_attn_fwd(None, None, F16, None, 3, 0, 4, 32, 0.1, 0, None) == 0
    assert lib.cobra_attn_fwd(None, None, F16, None, 0, 128, 4, 264, 0.1, 0, None) != 0  # head_dim
    assert lib.cobra_mask_bits(None, None, 0, 128, None) == 0
    layer_args = [None] * 12 + [None, None, 0]  # x .. resid_out, workspace, workspace bytes
    for B, S, D, H, dt in [(0, 128, 128, 4, F16), (3, 0, 128, 4, F16), (0, 1024, 128, 4, F16),
                           (0, 128, 1024, 4, F16), (2, 0, 1024, 16, F32), (0, 50, 96, 8, F16)]:
        a = list(layer_args)
        a[1] = dt
        assert lib.cobra_layer_fwd(*a, B, S, D, H, 0, 1e-5, None) == 0, (B, S, D, H)
        assert lib.cobra_layer_fwd_noalloc(*a[:13], B, S, D, H, 0, 1e-5, None) == 0, (B, S, D, H)
    a = list(layer_args)
    a[1] = F16
    assert lib.cobra_layer_fwd(*a, 0, 16, 528, 2, 0, 1e-5, None) != 0  # head_dim 264
    a[1] = 7
    assert lib.cobra_layer_fwd(*a, 0, 16, 128, 4, 0, 1e-5, None) != 0  # dtype code


def test_layer_bind_validates_and_releases():
    """cobra_layer_bind checks what cobra_layer_fwd would check, once; run rejects a
    mask on a handle bound without one, before any launch."""
    from cobra_amd import _lib

    lib = _lib.lib()
    w = [256 * (i + 1) for i in range(8)]  # aligned stand-in addresses: bind dereferences nothing
    assert not lib.cobra_layer_bind(0, 0, 12, *w[1:], None, 0, 2, 16, 128, 4, 0, 1e-5)   # misaligned w_qkv
    assert not lib.cobra_layer_bind(0, 0, *w, None, 0, 2, 16, 120, 10, 0, 1e-5)          # padded: needs workspace
    assert not lib.cobra_layer_bind(0, 0, *w, None, 0, 2, 16, 528, 2, 0, 1e-5)           # head_dim 264
    assert not lib.cobra_layer_bind(1, 0, *w, None, 0, 2, 16, 128, 16, 0, 1e-5)          # staged: needs workspace
    assert not lib.cobra_layer_bind(5, 0, *w, None, 0, 2, 16, 128, 4, 0, 1e-5)           # dtype code
    h = lib.cobra_layer_bind(0, 0, *w, None, 0, 2, 16, 128, 4, 0, 1e-5)                  # fused: no workspace
    assert h
    assert lib.cobra_layer_run(h, 256, 512, 768, None, None) != 0  # mask on an unmasked handle
    assert lib.cobra_layer_run(None, 256, None, 768, None, None) != 0
    lib.cobra_layer_unbind(h)
    lib.cobra_layer_unbind(None)
    ws = lib.cobra_layer_workspace_bytes(2, 16, 128, 16, 1, _lib.F32)
    h = lib.cobra_layer_bind(1, 1, *w, 4096, ws, 2, 16, 128, 16, 0, 1e-5)
    assert h
    lib.cobra_layer_unbind(h)
    assert not lib.cobra_layer_bind(1, 1, *w, 4096, ws - 1, 2, 16, 128, 16, 0, 1e-5)
    # LN1's affine: both parameters (w[4], w[5]) or neither; one alone, or misaligned, is rejected
    h = lib.cobra_layer_bind(0, 0, *w[:4], None, None, *w[6:], None, 0, 2, 16, 128, 4, 0, 1e-5)
    assert h
    lib.cobra_layer_unbind(h)
    assert not lib.cobra_layer_bind(0, 0, *w[:4], None, w[5], *w[6:], None, 0, 2, 16, 128, 4, 0, 1e-5)
    assert not lib.cobra_layer_bind(0, 0, *w[:4], w[4], None, *w[6:], None, 0, 2, 16, 128, 4, 0, 1e-5)
    assert not lib.cobra_layer_bind(0, 0, *w[:4], w[4] + 4, w[5], *w[6:], None, 0, 2, 16, 128, 4, 0, 1e-5)
    # the same check in cobra_layer_fwd, before any launch (x = 4096, y = 8192)
    assert lib.cobra_layer_fwd(4096, 0, None, *w[:4], None, w[5], *w[6:], 8192, None, None, 0, 2, 16, 128, 4, 0,
                               1e-5, None) != 0


def test_host_companion_loads_and_checks_its_arguments():
    """cobra_host.so (the module's native steady-state call, linked against the C ABI
    and torch) loads without a GPU and rejects a null launch handle, a host input and
    a parameter list without one snapshot value per tensor, before any launch."""
    from cobra_amd import _lib

    host = _lib.host()
    x = torch.zeros(2, 16, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="null launch handle"):
        host.BoundForward(0, x, [], [], None, 1e-5, False, None)
    with pytest.raises(RuntimeError, match="device tensor"):
        host.BoundForward(256, x, [], [], None, 1e-5, False, None)
    with pytest.raises(RuntimeError, match="one snapshot value"):
        host.BoundForward(256, x, [x], [], None, 1e-5, False, None)


def test_padded_block_weights_reproduce_the_block():
    """The stack's zero-padded weights (d_model 100 -> 104, head_dim 25 -> 32, ffn 50 -> 56)
    give, in fp64 on the CPU, each head's q / k / v and scores, the attention output, the
    out-projection and the FFN of the unpadded block in the true columns and exact zeros
    in every padded one: a head mapped to the wrong rows, a transposed W_o block or a
    shifted FFN column fails one of these."""
    import torch.nn.functional as F

    from cobra_amd.padding import PadGeometry, pad_block_weights

    D, H, FF, T = 100, 4, 50, 7
    g = PadGeometry(D, H, FF)
    assert (g.dp, g.hdp, g.fp, g.e) == (104, 32, 56, 128) and g.needed
    assert not PadGeometry(128, 4, 256).needed
    gen = torch.Generator().manual_seed(0)
    rnd = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)  # noqa: E731
    w_qkv, b_qkv, w_o, b_o = rnd(3 * D, D), rnd(3 * D), rnd(D, D), rnd(D)
    w1, b1, w2, b2 = rnd(FF, D), rnd(FF), rnd(D, FF), rnd(D)
    wq, bq, wo, bo, wi, bi, wu, bu = pad_block_weights(w_qkv, b_qkv, w_o, b_o, w1, b1, w2, b2, g)
    assert wq.shape == (3 * g.e, g.dp) and wo.shape == (g.dp, g.e) and wi.shape == (g.fp, g.dp)
    h = rnd(T, D)
    hp = torch.zeros(T, g.dp, dtype=torch.float64)
    hp[:, :D] = h
    qkv = (h @ w_qkv.T + b_qkv).view(T, 3, H, g.hd)
    qkvp = (hp @ wq.T + bq).view(T, 3, H, g.hdp)
    assert torch.allclose(qkvp[..., : g.hd], qkv, atol=1e-12)
    assert torch.equal(qkvp[..., g.hd:], torch.zeros_like(qkvp[..., g.hd:]))
    q, k, v = (qkv[:, i].transpose(0, 1) for i in range(3))      # [H, T, hd]
    qp, kp, vp = (qkvp[:, i].transpose(0, 1) for i in range(3))  # [H, T, hdp]
    s_true = (q @ k.transpose(1, 2)) * g.hd ** -0.5
    s_pad = (qp @ kp.transpose(1, 2)) * g.hd ** -0.5
    assert torch.allclose(s_pad, s_true, atol=1e-12)
    ctx = (torch.softmax(s_true, -1) @ v).transpose(0, 1).reshape(T, D)
    ctxp = (torch.softmax(s_pad, -1) @ vp).transpose(0, 1).reshape(T, g.e)
    out, outp = ctx @ w_o.T + b_o, ctxp @ wo.T + bo
    assert torch.allclose(outp[:, :D], out, atol=1e-10)
    assert torch.equal(outp[:, D:], torch.zeros_like(outp[:, D:]))
    hid, hidp = F.gelu(h @ w1.T + b1), F.gelu(hp @ wi.T + bi)
    assert torch.allclose(hidp[:, :FF], hid, atol=1e-12)
    assert torch.equal(hidp[:, FF:], torch.zeros_like(hidp[:, FF:]))
    y, yp = hid @ w2.T + b2, hidp @ wu.T + bu
    assert torch.allclose(yp[:, :D], y, atol=1e-10)
    assert torch.equal(yp[:, D:], torch.zeros_like(yp[:, D:]))


def test_ln1_fold_matches_layernorm_then_projection():
    """The module's packed QKV weights carry LN1's affine: LayerNorm without affine
    followed by the folded projection equals LayerNorm with affine followed by the
    original projection (fp64, up to the fp16 rounding of W diag(g1)).  Weights and
    LayerNorm parameters are non-uniform, so scaling the wrong axis of W, dropping
    the W b1 term or its sign fails."""
    from cobra_amd import CobraAttentionSublayer
    from cobra_amd.layer import _Pack

    torch.manual_seed(3)
    D = 64
    m = CobraAttentionSublayer(D, 4)
    with torch.no_grad():
        m.norm1.weight.uniform_(0.5, 1.5)
        m.norm1.bias.uniform_(-0.5, 0.5)
        for lin in (m.attention.q_proj, m.attention.k_proj, m.attention.v_proj):
            lin.bias.uniform_(-0.1, 0.1)
    p = _Pack(m, None)
    assert p.ln1_w is None and p.ln1_b is None
    assert p.w_qkv.dtype == torch.float16 and p.b_qkv.dtype == torch.float32
    x = torch.randn(32, D, dtype=torch.float64) * 2 + 0.3
    att = m.attention
    w = torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight]).double()
    b = torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias]).double()
    want = torch.nn.functional.layer_norm(x, (D,), m.norm1.weight.double(), m.norm1.bias.double()) @ w.T + b
    got = torch.nn.functional.layer_norm(x, (D,)) @ p.w_qkv.double().T + p.b_qkv.double()
    assert torch.allclose(got, want, rtol=0, atol=2e-3), (got - want).abs().max()
    assert (got - want).abs().max() > 0  # the fp16 rounding of W diag(g1) is visible, not skipped


def test_workspace_size_formula():
    from cobra_amd import ops

    # fused plan: no workspace
    assert ops.layer_workspace_bytes(64, 128, 128, 4) == 0
    # staged: h fp16 [T, D] + qkv fp16 [T, 3D], 256-B aligned (for D > 128 the out-projection's
    # fp16 branch reuses the qkv area; an fp32 residual goes only to a caller's resid_out)
    f32 = torch.float32
    assert ops.layer_workspace_bytes(64, 128, 128, 16, dtype=f32) == 8192 * 128 * 2 + 8192 * 384 * 2
    t, d = 32 * 100000, 1024
    assert ops.layer_workspace_bytes(32, 100000, 1024, 16) == t * d * 2 + t * 3 * d * 2
    # a token mask adds the packed key bits, [B][ceil(S/64)] u64, 256-B aligned
    bits = -(-(32 * 1563 * 8) // 256) * 256
    assert ops.layer_workspace_bytes(32, 100000, 1024, 16, masked=True) == t * d * 2 + t * 3 * d * 2 + bits
    assert ops.layer_workspace_bytes(64, 128, 128, 4, masked=True) == 0  # fused: the kernel reads the mask bytes
    assert ops.layer_workspace_bytes(64, 128, 128, 16, masked=True, dtype=f32) == 8192 * 128 * 2 + 8192 * 384 * 2 + 1024


def test_qkv_attn_workspace_and_fused_contract():
    """cobra_qkv_attn_fwd: head_dim 256 with seq_len <= 128 is one fused launch that needs no
    workspace (size 0, a null workspace accepted) but refuses ctx overlapping h; every other
    shape needs the q / k / v workspace and refuses a null one -- all decided before any launch."""
    from cobra_amd import _lib, ops

    lib = _lib.lib()
    assert lib.cobra_qkv_attn_workspace_bytes(64, 128, 4, 256) == 0
    assert lib.cobra_qkv_attn_workspace_bytes(2, 1, 1, 256) == 0
    assert lib.cobra_qkv_attn_workspace_bytes(64, 129, 4, 256) == round(64 * 129 * 3 * 1024 * 2 / 256 + 0.5) * 256
    assert lib.cobra_qkv_attn_workspace_bytes(64, 128, 8, 128) == 64 * 128 * 3 * 1024 * 2
    assert lib.cobra_qkv_attn_workspace_bytes(1, 16, 1, 264) == -1
    assert ops.qkv_attn_fused(64, 128, 4, 256) and not ops.qkv_attn_fused(64, 128, 16, 64)
    # ctx overlapping h on the fused shape; a null workspace on a two-launch shape
    assert lib.cobra_qkv_attn_fwd(1 << 20, 4096, None, (1 << 20) + 256, None, None, 0, 2, 16, 1, 256, 0.0625, 0,
                                  None) != 0
    assert lib.cobra_qkv_attn_fwd(1 << 20, 4096, None, 1 << 24, None, None, 0, 2, 16, 2, 64, 0.125, 0, None) != 0


def test_plan_selection_per_config():
    """One fused kernel for S <= 128 at d_model 128 with head_dim 32 or 64, and with
    head_dim 128 for fp16 batches the query-split kernel covers in two rounds of
    workgroups; staged otherwise."""
    import torch

    from cobra_amd import ops
    from oracle import CONFIGS

    fused = {"plumbing", "base", "b1", "b4", "b16", "b128", "b10000", "s32", "h1", "h2", "h16"}
    for name, c in CONFIGS.items():
        want = ops.PLAN_FUSED if name in fused else ops.PLAN_STAGED
        assert ops.layer_plan(c.batch, c.seq_len, c.d_model, c.heads) == want, name
    assert ops.layer_plan(2, 129, 128, 4) == ops.PLAN_STAGED
    assert ops.layer_plan(2, 17, 96, 3) == ops.PLAN_FUSED
    # head_dim 128: the query-split kernel only (fp16 activations, <= 2 rounds at 256 CUs)
    assert ops.layer_plan(128, 128, 128, 1) == ops.PLAN_FUSED
    assert ops.layer_plan(129, 128, 128, 1) == ops.PLAN_STAGED
    assert ops.layer_plan(64, 128, 128, 1, dtype=torch.float32) == ops.PLAN_STAGED
    assert ops.layer_plan(64, 128, 128, 16, dtype=torch.float32) == ops.PLAN_STAGED
    assert ops.layer_plan(129, 128, 128, 16) == ops.PLAN_STAGED
    assert ops.layer_plan(64, 128, 128, 4, dtype=torch.float32) == ops.PLAN_FUSED
    assert ops.layer_workspace_bytes(64, 128, 128, 1) == 0
    assert ops.layer_workspace_bytes(64, 128, 128, 1, dtype=torch.float32) == 8192 * 128 * 2 + 8192 * 384 * 2
    assert ops.layer_plan(2, 16, 128, 4, dtype=torch.bfloat16) == ops.PLAN_STAGED  # bf16: staged kernels
    assert ops.layer_plan(2, 16, 120, 10, dtype=torch.bfloat16) == ops.PLAN_PADDED
    with pytest.raises(TypeError):
        ops.layer_plan(2, 16, 128, 4, dtype=torch.float64)
    with pytest.raises(ValueError):
        ops.layer_plan(2, 16, 528, 2)  # head_dim 264
    assert ops.layer_plan(2, 16, 120, 10) == ops.PLAN_PADDED


def test_state_dict_identical_to_reference_sublayer():
    from cobra_amd import CobraAttentionSublayer

    ref = make_sublayer(128, 4, seed=0)
    torch.manual_seed(0)
    mod = CobraAttentionSublayer(128, 4)
    sd_r, sd_m = ref.state_dict(), mod.state_dict()
    assert list(sd_r) == list(sd_m)
    for k in sd_r:
        assert torch.equal(sd_r[k], sd_m[k]), k  # same seeded draws, same order
    mod.load_state_dict(sd_r, strict=True)
    ref.load_state_dict(sd_m, strict=True)


def test_module_refuses_to_run_without_gpu():
    from cobra_amd import CobraAttentionSublayer

    mod = CobraAttentionSublayer(128, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        mod(torch.zeros(1, 4, 128))


def test_ops_reject_host_tensors():
    from cobra_amd import ops

    with pytest.raises(ValueError, match="device"):
        ops.linear(torch.zeros(4, 8, dtype=torch.float16), torch.zeros(8, 8, dtype=torch.float16), None)
    with pytest.raises(ValueError, match="device"):
        ops.linear(torch.zeros(4, 8, dtype=torch.float16), torch.zeros(8, 8, dtype=torch.float16), None, gelu=True)
    with pytest.raises(ValueError, match="device"):
        ops.mask_bits(torch.ones(2, 8, dtype=torch.bool))


def test_product_never_imports_the_oracle():
    for root, _, files in os.walk(os.path.join(ROOT, "cobra-gpu-kernel_amd")):
        for f in files:
            if not f.endswith(".py"):
                continue
            tree = ast.parse(open(os.path.join(root, f)).read())
            for node in ast.walk(tree):
                if isinstance(node, ast.Import):
                    mods = [a.name for a in node.names]
                elif isinstance(node, ast.ImportFrom):
                    mods = [node.module or ""]
                else:
                    continue
                assert not any(m.split(".")[0] == "oracle" for m in mods), f"{f} imports the oracle"


# ---- streaming planner (TTB:1364-1508 restated as pure functions) ----------

def test_should_stream_rules():
    from cobra_amd.streaming import should_stream

    gib = 1 << 30
    assert should_stream(False, 10, 1, 0, 100 * gib)            # host input always streams
    assert not should_stream(True, gib - 1, 32, 10**15, gib)     # small input never
    assert not should_stream(True, 2 * gib, 1, 10**15, gib)      # one sequence: nothing to split
    assert should_stream(True, 2 * gib, 4, 61 * gib, 100 * gib)  # live set > 60 % of free
    assert not should_stream(True, 2 * gib, 4, 59 * gib, 100 * gib)


def test_plan_chunk():
    from cobra_amd.streaming import plan_chunk

    assert plan_chunk(32, 10, 1000) == 32
    assert plan_chunk(32, 100, 1000) == 6      # 600 // 100
    assert plan_chunk(32, 10**9, 1000) == 1    # never below one sequence


def test_long_config_fits_one_pass_on_288gb():
    """B32 S1e5 D1024 fp16 on a 288 GB device: one chunk, no streaming."""
    from cobra_amd import ops
    from cobra_amd.streaming import live_bytes_per_sequence, plan_chunk, should_stream

    per_seq = live_bytes_per_sequence(ops.layer_workspace_bytes(1, 100000, 1024, 16), 100000, 1024, 2)
    free = 280 * 10**9
    assert not should_stream(True, 32 * 100000 * 1024 * 2, 32, 32 * per_seq, free)
    assert plan_chunk(32, per_seq, free) == 32
    assert plan_chunk(32, per_seq, 16 * 10**9) < 32


class _FakeOOM(Exception):
    pass


def test_halve_on_oom_then_succeed():
    from cobra_amd.streaming import run_chunked

    calls, frees = [], []

    def run(b0, b1):
        calls.append((b0, b1))
        if b1 - b0 > 3:
            raise _FakeOOM()

    done = run_chunked(10, 8, run, lambda: frees.append(1), lambda e: isinstance(e, _FakeOOM))
    assert done == [(0, 2), (2, 4), (4, 6), (6, 8), (8, 10)]
    assert calls[:2] == [(0, 8), (0, 4)] and len(frees) == 2


def test_oom_at_step_one_propagates():
    from cobra_amd.streaming import run_chunked

    def run(b0, b1):
        raise _FakeOOM()

    with pytest.raises(_FakeOOM):
        run_chunked(4, 4, run, lambda: None, lambda e: isinstance(e, _FakeOOM))


def test_non_oom_errors_propagate_immediately():
    from cobra_amd.streaming import run_chunked

    def run(b0, b1):
        raise ValueError("boom")

    with pytest.raises(ValueError):
        run_chunked(4, 2, run, lambda: None, lambda e: isinstance(e, _FakeOOM))


def test_oracle_and_product_share_parameter_names():
    from cobra_amd import CobraAttentionSublayer

    a = dict(OracleAttentionSublayer(64, 2).named_parameters())
    b = dict(CobraAttentionSublayer(64, 2).named_parameters())
    assert {k: v.shape for k, v in a.items()} == {k: v.shape for k, v in b.items()}


def test_noalloc_scratch_size_matches_the_header():
    """The Python wrapper's size check uses the header's COBRA_NOALLOC_MAX_BYTES."""
    from cobra_amd import _lib, ops

    m = re.search(r"#define COBRA_NOALLOC_MAX_BYTES \((\d+)ll << (\d+)\)", open(HEADER).read())
    assert m, "COBRA_NOALLOC_MAX_BYTES not found"
    assert _lib.NOALLOC_MAX_BYTES == ops.NOALLOC_MAX_BYTES == int(m.group(1)) << int(m.group(2))
    lib = _lib.lib()
    # rejected on the host, before any device call: a shape beyond the scratch
    assert lib.cobra_layer_fwd_noalloc(256, _lib.F16, None, 256, 256, 256, 256, None, None, 256, 256, 256, None,
                                       200, 1024, 128, 4, 0, 1e-5, None) != 0


def _r256(n):
    return (n + 255) & ~255


@pytest.mark.parametrize("B,S,D,H,masked", [(2, 16, 120, 10, False), (3, 17, 100, 4, True), (1, 5, 36, 3, True),
                                            (2, 9, 9, 1, False), (4, 33, 260, 4, True)])
def test_padded_plan_workspace(B, S, D, H, masked):
    """The padded plan's workspace: padded W_qkv / b_qkv / W_o / b_o, h or ctx (the wider),
    qkv, the fp32 branch and the key bits, each 256-byte aligned (head_dim and d_model
    rounded up to multiples of 8)."""
    from cobra_amd import ops

    hdp = -(-(D // H) // 8) * 8
    dp = -(-D // 8) * 8
    e = H * hdp
    t = B * S
    want = (_r256(3 * e * dp * 2) + _r256(3 * e * 4) + _r256(dp * e * 2) + _r256(dp * 4) + _r256(t * max(dp, e) * 2)
            + _r256(t * 3 * e * 2) + _r256(t * dp * 4) + (_r256(B * -(-S // 64) * 8) if masked else 0))
    assert ops.layer_plan(B, S, D, H, masked) == ops.PLAN_PADDED
    assert ops.layer_workspace_bytes(B, S, D, H, masked) == want
