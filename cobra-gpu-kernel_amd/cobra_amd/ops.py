"""Tensor-level wrappers of the C ABI, mirroring the reference's kernel launchers.

Each function keeps the name stem, argument order and meaning of the
reference launcher it replaces (``torch_transformer_benchmark.py``, "TTB"),
allocates its outputs with ``torch.empty`` like the reference does, enqueues
on ``torch.cuda.current_stream()`` and never synchronises.  Differences:

* weights are nn.Linear's ``[N, K]`` layout; the reference passed a
  transposed ``[K, N]`` copy to its GEMMs (TTB:895-904).  No copy is needed here;
* attention takes ``causal`` (the reference kernel was causal-only) and an
  optional ``key_mask`` (the reference routed masked attention to SDPA with an
  additive -inf bias, TTB:1207-1213, 1240-1253);
* row masks (``mask_row`` / ``rmask``) are ``[M]`` bool or uint8 tensors
  (0 = padded row), applied with the reference kernels' MASK_RESID / MASK_OUT
  rules; ``mask_branch=True`` additionally offers the attention sublayer's own
  rule, zeroing the product rows *before* the residual add (TTB:121-122).

Argument errors raise ``ValueError``/``TypeError`` before anything is
enqueued; a non-zero code from the library raises ``CobraError``.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import BF16, F16, F32, call

_DT = {torch.float16: F16, torch.float32: F32, torch.bfloat16: BF16}


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: dtype {t.dtype} not supported (float16, bfloat16 or float32)") from None


def _dev(t: torch.Tensor, what: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{what} must be a device tensor (got {t.device}); the HIP path has no host fallback")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return t


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """The device's current stream handle.  The raw query costs ~0.1 us; building
    a Stream object (torch.cuda.current_stream) costs ~3 us, a quarter of a
    small forward's launch budget."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def _f32_param(t: torch.Tensor, n: int, what: str) -> torch.Tensor:
    if t.shape != (n,):
        raise ValueError(f"{what} must have shape ({n},), got {tuple(t.shape)}")
    return t.to(dtype=torch.float32).contiguous()


def _row_mask(m: Optional[torch.Tensor], rows: int, what: str) -> Optional[torch.Tensor]:
    """A [rows] (or [B, S] with B*S == rows) bool/uint8 device mask as a uint8 view."""
    if m is None:
        return None
    _dev(m, what)
    if m.dtype not in (torch.bool, torch.uint8):
        raise TypeError(f"{what} must be bool or uint8, got {m.dtype}")
    if m.numel() != rows:
        raise ValueError(f"{what} must hold {rows} rows, got shape {tuple(m.shape)}")
    # bool -> uint8 is a reinterpretation of the same bytes (0x00 / 0x01), not a copy.
    return m.reshape(rows).view(torch.uint8)


def add_ln(
    resid: torch.Tensor,
    branch: Optional[torch.Tensor],
    mask_row: Optional[torch.Tensor],
    w: Optional[torch.Tensor],
    b: Optional[torch.Tensor],
    cast_fp16: bool = True,
    eps: float = 1e-5,
    store_resid: bool = True,
    mask_out: bool = False,
) -> Tuple[Optional[torch.Tensor], torch.Tensor]:
    """``(resid + branch)`` then LayerNorm -> ``(new_resid | None, normed)``.

    Mirrors ``_tl_add_ln`` (TTB:539-569), including its mask rule: with a
    ``mask_row``, the residual is multiplied by the mask whenever it is stored
    or the output is masked, and ``mask_out`` also masks the normalised output.
    The stored residual is always fp32.  ``w = b = None``: no elementwise affine
    (weight 1, bias 0, which leaves the normalised value exact).
    """
    _dev(resid, "resid")
    if resid.dim() != 2:
        raise ValueError("resid must be [M, N]")
    M, N = resid.shape
    mrow = _row_mask(mask_row, M, "mask_row")
    flags = 0
    if mrow is not None:
        if store_resid or mask_out:
            flags |= _lib.EPI_MASK_RESID
        if mask_out:
            flags |= _lib.EPI_MASK_OUT
    if branch is not None:
        _dev(branch, "branch")
        if branch.shape != resid.shape:
            raise ValueError("branch must match resid")
    if (w is None) != (b is None):
        raise ValueError("w and b must both be given or both be None")
    if w is None:
        gw = torch.ones(N, device=resid.device, dtype=torch.float32)
        gb = torch.zeros(N, device=resid.device, dtype=torch.float32)
    else:
        gw, gb = _f32_param(w, N, "w"), _f32_param(b, N, "b")
    out_r = torch.empty((M, N), device=resid.device, dtype=torch.float32) if store_resid else None
    out_n = torch.empty((M, N), device=resid.device, dtype=torch.float16 if cast_fp16 else torch.float32)
    call(
        "cobra_ln_fwd", resid.data_ptr(), _dtype_code(resid, "resid"), _ptr(branch),
        _dtype_code(branch, "branch") if branch is not None else 0, gw.data_ptr(), gb.data_ptr(), _ptr(mrow),
        flags, _ptr(out_r), out_n.data_ptr(), _dtype_code(out_n, "normed"), M, N, float(eps), _stream(resid),
    )
    return out_r, out_n


def ln_strided(
    x: torch.Tensor,
    d: int,
    w: torch.Tensor,
    b: torch.Tensor,
    out_cols: Optional[int] = None,
    out_dtype: Optional[torch.dtype] = None,
    branch: Optional[torch.Tensor] = None,
    mask_row: Optional[torch.Tensor] = None,
    resid_out: Optional[torch.Tensor] = None,
    mask_resid: bool = False,
    mask_out: bool = False,
    eps: float = 1e-5,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """LayerNorm over the first ``d`` columns of each row of ``x`` [M, ldx] (+ ``branch``
    [M, ldb] in its first d columns) -> ``y`` [M, out_cols] with columns d .. out_cols-1
    zero (a zero-padded GEMM operand).  The counterpart of ``_tl_add_ln`` (TTB:539-569)
    for rows padded past their true width; ``resid_out`` [M, ldr] fp32 receives the first
    d columns of x (+ branch) (after the row mask with ``mask_resid``), its other
    columns are left as they are.  ``mask_out`` zeroes padded rows' output.  ``out``:
    a caller-provided y (contiguous [M, out_cols]) instead of a new tensor."""
    _dev(x, "x")
    if x.dim() != 2 or x.shape[1] < d or d <= 0:
        raise ValueError(f"x must be [M, >= {d}]")
    M = x.shape[0]
    out_cols = d if out_cols is None else int(out_cols)
    if out_cols < d:
        raise ValueError("out_cols must be >= d")
    w32, b32 = _f32_param(w, d, "w"), _f32_param(b, d, "b")
    flags = 0
    mrow = _row_mask(mask_row, M, "mask_row")
    if mrow is not None:
        flags |= (_lib.EPI_MASK_RESID if mask_resid else 0) | (_lib.EPI_MASK_OUT if mask_out else 0)
    elif mask_resid or mask_out:
        raise ValueError("mask_resid / mask_out need mask_row")
    if branch is not None:
        _dev(branch, "branch")
        if branch.dim() != 2 or branch.shape[0] != M or branch.shape[1] < d:
            raise ValueError("branch must be [M, >= d]")
    if resid_out is not None:
        _dev(resid_out, "resid_out")
        if resid_out.dtype != torch.float32 or resid_out.dim() != 2 or resid_out.shape[0] != M or \
                resid_out.shape[1] < d:
            raise ValueError("resid_out must be fp32 [M, >= d]")
    if out is None:
        y = torch.empty((M, out_cols), device=x.device, dtype=out_dtype or x.dtype)
    else:
        y = _dev(out, "out")
        if tuple(y.shape) != (M, out_cols) or (out_dtype is not None and y.dtype != out_dtype):
            raise ValueError(f"out must be [{M}, {out_cols}]" + (f" {out_dtype}" if out_dtype else ""))
    call(
        "cobra_ln_fwd_strided", x.data_ptr(), _dtype_code(x, "x"), x.shape[1], _ptr(branch),
        _dtype_code(branch, "branch") if branch is not None else 0, branch.shape[1] if branch is not None else 0,
        w32.data_ptr(), b32.data_ptr(), _ptr(mrow), flags, _ptr(resid_out),
        resid_out.shape[1] if resid_out is not None else 0, y.data_ptr(), _dtype_code(y, "y"), out_cols, M, d,
        float(eps), _stream(x),
    )
    return y


def linear(
    a: torch.Tensor,
    w: torch.Tensor,
    bias: Optional[torch.Tensor],
    gelu: bool = False,
    out_fp32: bool = False,
    resid: Optional[torch.Tensor] = None,
    rmask: Optional[torch.Tensor] = None,
    mask_branch: bool = False,
) -> torch.Tensor:
    """``a @ w.T + bias`` (GELU) ``(+ resid)`` with fp32 accumulate.  Mirrors ``_tl_linear`` (TTB:355-381).

    a: [M, K] and w: [N, K] both fp16 or both bf16 (bf16 MFMA operands); bias: [N];
    resid: [M, N] in a's dtype or fp32.  The output is fp32 with ``out_fp32``, else a's dtype.
    ``gelu`` is the exact erf GELU after the bias (TTB:326-328).  ``rmask``
    multiplies ``(product + resid)`` of padded rows by 0 when there is a
    residual (the reference kernel applies it only then, TTB:343-348); with
    ``mask_branch=True`` it instead zeroes the padded rows' product before the
    residual add, so those rows come out equal to ``resid``.
    """
    _dev(a, "a")
    _dev(w, "w")
    if a.dtype not in (torch.float16, torch.bfloat16) or w.dtype != a.dtype:
        raise TypeError("a and w must be both float16 or both bfloat16 (fp32 accumulate)")
    M, K = a.shape
    N, K2 = w.shape
    if K2 != K:
        raise ValueError(f"inner dimensions differ: a {tuple(a.shape)}, w {tuple(w.shape)}")
    b32 = _f32_param(bias, N, "bias") if bias is not None else None
    if resid is not None:
        _dev(resid, "resid")
        if resid.shape != (M, N):
            raise ValueError("resid must be [M, N]")
        if resid.dtype not in (a.dtype, torch.float32):
            raise TypeError(f"resid must be {a.dtype} or float32, got {resid.dtype}")
    mrow = _row_mask(rmask, M, "rmask")
    epi = _lib.EPI_GELU if gelu else 0
    if mrow is not None:
        if mask_branch:
            epi |= _lib.EPI_MASK_BRANCH
        elif resid is not None:
            epi |= _lib.EPI_MASK_RESID
        else:
            mrow = None
    out = torch.empty((M, N), device=a.device, dtype=torch.float32 if out_fp32 else a.dtype)
    call(
        "cobra_linear_fwd", a.data_ptr(), w.data_ptr(), _dtype_code(a, "a"), _ptr(b32), _ptr(resid),
        _dtype_code(resid, "resid") if resid is not None else 0, _ptr(mrow), epi, out.data_ptr(),
        _dtype_code(out, "out"), M, N, K, _stream(a),
    )
    return out


def linear_ln(
    a: torch.Tensor,
    w: torch.Tensor,
    bias: torch.Tensor,
    resid: torch.Tensor,
    nw: torch.Tensor,
    nb: torch.Tensor,
    rmask: Optional[torch.Tensor] = None,
    norm_fp16: bool = True,
    mask_out: bool = False,
    eps: float = 1e-5,
    mask_branch: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """``r = a @ w.T + bias + resid``; ``(r fp32, LayerNorm(r))``.  Mirrors ``_tl_linear_ln`` (TTB:465-488).

    Requires N <= 128, like the reference (TTB:471).  ``rmask`` multiplies the
    padded rows of ``r`` by 0 and, with ``mask_out``, of the normalised output
    (TTB:436-458); ``mask_branch=True`` zeroes the padded rows' product before
    the residual add instead (the attention sublayer's rule, TTB:121-122).
    """
    _dev(a, "a")
    _dev(w, "w")
    _dev(resid, "resid")
    if a.dtype != torch.float16 or w.dtype != torch.float16:
        raise TypeError("a and w must be float16")
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K or resid.shape != (M, N):
        raise ValueError("shape mismatch")
    if N > 128:
        raise ValueError("fused-LN GEMM requires N <= 128 (one workgroup owns a whole row)")
    b32 = _f32_param(bias, N, "bias")
    gw, gb = _f32_param(nw, N, "nw"), _f32_param(nb, N, "nb")
    mrow = _row_mask(rmask, M, "rmask")
    epi = 0
    if mrow is not None:
        epi |= _lib.EPI_MASK_BRANCH if mask_branch else _lib.EPI_MASK_RESID
        if mask_out:
            epi |= _lib.EPI_MASK_OUT
    out = torch.empty((M, N), device=a.device, dtype=torch.float32)
    normed = torch.empty((M, N), device=a.device, dtype=torch.float16 if norm_fp16 else torch.float32)
    call(
        "cobra_linear_ln_fwd", a.data_ptr(), w.data_ptr(), b32.data_ptr(), resid.data_ptr(),
        _dtype_code(resid, "resid"), _ptr(mrow), epi, out.data_ptr(), gw.data_ptr(), gb.data_ptr(),
        normed.data_ptr(), _dtype_code(normed, "normed"), M, N, K, float(eps), _stream(a),
    )
    return out, normed


def ln_linear_ok(d: int, x_dtype: torch.dtype) -> bool:
    """Whether ``ln_linear`` covers rows of width d (one k-tile per row)."""
    return d in (64, 128) and x_dtype in (torch.float16, torch.float32)


def ln_linear(x: torch.Tensor, w_ln: torch.Tensor, b_ln: torch.Tensor, w: torch.Tensor,
              bias: Optional[torch.Tensor], eps: float = 1e-5) -> torch.Tensor:
    """``LayerNorm(x) @ w.T + bias`` in one kernel, fp16 out; the normalised rows
    never reach memory.  Stands for ``_tl_add_ln`` followed by ``F.linear``
    (TTB:1216-1234).  x: [M, d] fp16/fp32 with d 64 or 128; w: [N, d] fp16 with
    N <= 3d (a QKV projection) and N % 8 == 0.
    """
    _dev(x, "x")
    _dev(w, "w")
    if x.dim() != 2:
        raise ValueError("x must be [M, d]")
    M, d = x.shape
    if not ln_linear_ok(d, x.dtype):
        raise ValueError(f"ln_linear needs d 64 or 128 and fp16/fp32 x, got d={d} {x.dtype}")
    if w.dtype != torch.float16 or w.dim() != 2 or w.shape[1] != d:
        raise ValueError(f"w must be fp16 [N, {d}]")
    N = w.shape[0]
    if N > 3 * d or N % 8:
        raise ValueError(f"ln_linear needs N <= {3 * d} and N % 8 == 0, got N={N}")
    gw, gb = _f32_param(w_ln, d, "w_ln"), _f32_param(b_ln, d, "b_ln")
    b32 = _f32_param(bias, N, "bias") if bias is not None else None
    out = torch.empty((M, N), device=x.device, dtype=torch.float16)
    call("cobra_ln_linear_fwd", x.data_ptr(), _dtype_code(x, "x"), gw.data_ptr(), gb.data_ptr(), w.data_ptr(),
         _ptr(b32), out.data_ptr(), M, N, d, float(eps), _stream(x))
    return out


def mask_bits(mask: torch.Tensor) -> torch.Tensor:
    """[B, S] bool/uint8 token mask -> packed key bits ``[B, ceil(S/64)]`` (int64 storage of u64 words)."""
    if mask.dim() != 2:
        raise ValueError(f"mask must be [B, S], got {tuple(mask.shape)}")
    B, S = mask.shape
    m = _row_mask(mask, B * S, "mask")
    bits = torch.empty((B, (S + 63) // 64), device=mask.device, dtype=torch.int64)
    call("cobra_mask_bits", m.data_ptr(), bits.data_ptr(), B, S, _stream(mask))
    return bits


def attn(
    qkv: torch.Tensor,
    batch: int,
    seq_len: int,
    heads: int,
    head_dim: int,
    scale: float,
    out_dtype: Optional[torch.dtype] = None,
    cfgs=None,
    causal: bool = True,
    key_mask: Optional[torch.Tensor] = None,
    key_bits: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention on packed ``qkv [B*S, 3*H*hd]`` -> ``ctx [B*S, H*hd]``.  Mirrors ``_tl_attn`` (TTB:828-854).

    qkv and ctx are fp16, or both bf16 (bf16 MFMA operands, the probabilities rounded to
    bf16 for the P.V product); ``out_dtype`` None means qkv's dtype.

    ``cfgs`` (the reference's tile ladder) is accepted and ignored: tiles are
    chosen inside the library from (seq_len, head_dim).  ``key_mask`` ([B, S]
    bool/uint8, 0 = padded) masks keys like TTB:106-109; a query with no valid
    key gets a zero row.  ``key_bits`` passes the packed form (``mask_bits``)
    instead, so a caller with several attention calls per mask packs it once.
    """
    _dev(qkv, "qkv")
    if qkv.dtype not in (torch.float16, torch.bfloat16) or (out_dtype is not None and out_dtype != qkv.dtype):
        raise TypeError("attention operands and output are float16, or both bfloat16")
    D = heads * head_dim
    if qkv.shape != (batch * seq_len, 3 * D):
        raise ValueError(f"qkv must be [{batch * seq_len}, {3 * D}], got {tuple(qkv.shape)}")
    bits = key_bits
    if key_mask is not None:
        if key_bits is not None:
            raise ValueError("pass key_mask or key_bits, not both")
        if tuple(key_mask.shape) != (batch, seq_len):
            raise ValueError(f"key_mask must be [{batch}, {seq_len}], got {tuple(key_mask.shape)}")
        bits = mask_bits(key_mask)
    elif bits is not None:
        _dev(bits, "key_bits")
        if bits.dtype != torch.int64 or tuple(bits.shape) != (batch, (seq_len + 63) // 64):
            raise ValueError(f"key_bits must be int64 [{batch}, {(seq_len + 63) // 64}]")
    out = torch.empty((batch * seq_len, D), device=qkv.device, dtype=qkv.dtype)
    call(
        "cobra_attn_fwd", qkv.data_ptr(), out.data_ptr(), _dtype_code(qkv, "qkv"), _ptr(bits), batch, seq_len, heads,
        head_dim,
        float(scale), 1 if causal else 0, _stream(qkv),
    )
    return out


def qkv_attn(
    h: torch.Tensor,
    w_qkv: torch.Tensor,
    b_qkv: Optional[torch.Tensor],
    batch: int,
    seq_len: int,
    heads: int,
    head_dim: int,
    scale: float,
    out_dtype: torch.dtype = torch.float16,
    cfgs=None,
    causal: bool = True,
    key_mask: Optional[torch.Tensor] = None,
    key_bits: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """QKV projection fused with attention: ``h [B*S, D]`` -> ``ctx [B*S, D]``.  Mirrors
    ``_tl_qkvattn`` (TTB:761-785).

    Differences from the reference launcher: ``w_qkv`` is the nn.Linear-layout ``[3D, D]``
    q | k | v weight (the reference passes the transposed ``[D, 3D]``), and attention may be
    non-causal and masked (``key_mask`` / ``key_bits`` as in ``attn``).  For head_dim 256
    and seq_len <= 128 the projection runs inside the attention kernel, one workgroup per
    (sequence, head), as the reference's fused kernel does; otherwise the projected q / k / v
    go through a workspace allocated here (``torch.empty``) between the GEMM and the
    attention kernel.  ``cfgs`` is accepted and ignored.
    """
    _dev(h, "h")
    _dev(w_qkv, "w_qkv")
    if h.dtype != torch.float16 or w_qkv.dtype != torch.float16 or out_dtype != torch.float16:
        raise TypeError("h, w_qkv and ctx are float16")
    D = heads * head_dim
    if h.shape != (batch * seq_len, D) or w_qkv.shape != (3 * D, D):
        raise ValueError(f"h must be [{batch * seq_len}, {D}] and w_qkv [{3 * D}, {D}]")
    bias = None if b_qkv is None else _f32_param(b_qkv, 3 * D, "b_qkv")
    bits = key_bits
    if key_mask is not None:
        if key_bits is not None:
            raise ValueError("pass key_mask or key_bits, not both")
        if tuple(key_mask.shape) != (batch, seq_len):
            raise ValueError(f"key_mask must be [{batch}, {seq_len}], got {tuple(key_mask.shape)}")
        bits = mask_bits(key_mask)
    elif bits is not None:
        _dev(bits, "key_bits")
        if bits.dtype != torch.int64 or tuple(bits.shape) != (batch, (seq_len + 63) // 64):
            raise ValueError(f"key_bits must be int64 [{batch}, {(seq_len + 63) // 64}]")
    need = _lib.lib().cobra_qkv_attn_workspace_bytes(batch, seq_len, heads, head_dim)
    if need < 0:
        raise ValueError(f"unsupported attention shape heads={heads} head_dim={head_dim}")
    ws = torch.empty(int(need), dtype=torch.uint8, device=h.device) if need > 0 else None
    out = torch.empty((batch * seq_len, D), device=h.device, dtype=torch.float16)
    call(
        "cobra_qkv_attn_fwd", h.data_ptr(), w_qkv.data_ptr(), _ptr(bias), out.data_ptr(), _ptr(bits), _ptr(ws),
        0 if ws is None else ws.numel(), batch, seq_len, heads, head_dim, float(scale), 1 if causal else 0,
        _stream(h),
    )
    return out


def qkv_attn_fused(batch: int, seq_len: int, heads: int, head_dim: int) -> bool:
    """Whether ``qkv_attn`` runs as one launch (the projection inside the attention kernel,
    no q / k / v buffer) for this shape (host-only query)."""
    return _lib.lib().cobra_qkv_attn_workspace_bytes(batch, seq_len, heads, head_dim) == 0


PLAN_FUSED = _lib.PLAN_FUSED
PLAN_STAGED = _lib.PLAN_STAGED
PLAN_PADDED = _lib.PLAN_PADDED


def _dt_of(dtype: torch.dtype) -> int:
    try:
        return _DT[dtype]
    except KeyError:
        raise TypeError(f"dtype {dtype} not supported (float16, bfloat16 or float32)") from None


def layer_plan(batch: int, seq_len: int, d_model: int, heads: int, masked: bool = False,
               dtype: torch.dtype = torch.float16) -> int:
    """PLAN_FUSED (one kernel), PLAN_STAGED, or PLAN_PADDED (head_dim or d_model not a
    multiple of 8: the staged plan on zero-padded copies) for this shape and activation
    dtype (host-only query)."""
    p = _lib.lib().cobra_layer_plan(batch, seq_len, d_model, heads, 1 if masked else 0, _dt_of(dtype))
    if p < 0:
        raise ValueError(f"unsupported sublayer shape B={batch} S={seq_len} D={d_model} H={heads}")
    return int(p)


def layer_workspace_bytes(batch: int, seq_len: int, d_model: int, heads: int, masked: bool = False,
                          dtype: torch.dtype = torch.float16) -> int:
    n = _lib.lib().cobra_layer_workspace_bytes(batch, seq_len, d_model, heads, 1 if masked else 0, _dt_of(dtype))
    if n < 0:
        raise ValueError(f"unsupported sublayer shape B={batch} S={seq_len} D={d_model} H={heads}")
    return int(n)


def layer_fwd(
    x: torch.Tensor,
    w_qkv: torch.Tensor,
    b_qkv: torch.Tensor,
    w_o: torch.Tensor,
    b_o: torch.Tensor,
    ln1_w: Optional[torch.Tensor],
    ln1_b: Optional[torch.Tensor],
    ln2_w: torch.Tensor,
    ln2_b: torch.Tensor,
    y: torch.Tensor,
    workspace: torch.Tensor,
    heads: int,
    causal: bool,
    eps: float = 1e-5,
    resid_out: Optional[torch.Tensor] = None,
    valid_mask: Optional[torch.Tensor] = None,
) -> None:
    """Enqueue the whole sublayer into caller-provided buffers (no allocation).

    x, y: [B, S, D] (same dtype); packed weights as produced by ``CobraAttentionSublayer``;
    ln1_w = ln1_b = None: LN1 without elementwise affine (already folded into w_qkv / b_qkv);
    valid_mask: optional [B, S] uint8 (0 = padded token) -- the workspace must then be
    sized with ``masked=True``.
    """
    call("cobra_layer_fwd", *layer_fwd_args(x, w_qkv, b_qkv, w_o, b_o, ln1_w, ln1_b, ln2_w, ln2_b, y, workspace,
                                            heads, causal, eps, resid_out, valid_mask))


def layer_fwd_args(x, w_qkv, b_qkv, w_o, b_o, ln1_w, ln1_b, ln2_w, ln2_b, y, workspace, heads, causal, eps=1e-5,
                   resid_out=None, valid_mask=None) -> list:
    """The argument list of ``cobra_layer_fwd``."""
    B, S, D = x.shape
    return [x.data_ptr(), _dtype_code(x, "x"), _ptr(valid_mask), w_qkv.data_ptr(), b_qkv.data_ptr(),
            w_o.data_ptr(), b_o.data_ptr(), _ptr(ln1_w), _ptr(ln1_b), ln2_w.data_ptr(),
            ln2_b.data_ptr(), y.data_ptr(), _ptr(resid_out), workspace.data_ptr(), workspace.numel(),
            B, S, D, heads, 1 if causal else 0, float(eps), _stream(x)]


def block_plan(batch: int, seq_len: int, d_model: int, heads: int, ffn_dim: int) -> int:
    """``cobra_block_plan``: -1 the whole-block kernel does not take the shape, 0 it does
    but composing the per-op kernels is expected to be faster, 1 it does and is preferred."""
    return int(_lib.lib().cobra_block_plan(batch, seq_len, d_model, heads, ffn_dim))


def block_fwd(
    h: torch.Tensor,
    r: torch.Tensor,
    w_qkv: torch.Tensor,
    b_qkv: torch.Tensor,
    w_o: torch.Tensor,
    b_o: torch.Tensor,
    ln2_w: torch.Tensor,
    ln2_b: torch.Tensor,
    w1: torch.Tensor,
    b1: torch.Tensor,
    w2: torch.Tensor,
    b2: torch.Tensor,
    lnn_w: torch.Tensor,
    lnn_b: torch.Tensor,
    r_out: torch.Tensor,
    out: torch.Tensor,
    batch: int,
    seq_len: int,
    heads: int,
    causal: bool,
    eps: float = 1e-5,
    valid_mask: Optional[torch.Tensor] = None,
    mask_out: bool = False,
) -> None:
    """One transformer block of the fused stack in one launch (``cobra_block_fwd``; the
    loop body of the reference's ``_run_fused``, TTB:1216-1267): ``h = norm1(r)`` fp16
    and the fp32 residual ``r`` in; the block's residual to ``r_out`` (may be ``r``) and
    the next norm's output (``lnn``; ``final_norm`` with ``mask_out`` on the last block)
    to ``out`` (fp16 or fp32).  ``valid_mask``: optional [B, S] uint8, 0 = padded token.
    """
    T, D = h.shape
    F = w1.shape[0]
    if h.dtype != torch.float16 or r.dtype != torch.float32 or r_out.dtype != torch.float32:
        raise TypeError("h is float16, r and r_out float32")
    if T != batch * seq_len or r.shape != (T, D) or r_out.shape != (T, D) or out.shape != (T, D):
        raise ValueError("h, r, r_out and out must be [batch * seq_len, d_model]")
    if tuple(w1.shape) != (F, D) or tuple(w2.shape) != (D, F):
        raise ValueError(f"w1 must be [F, {D}] and w2 [{D}, F]")
    for name, t in (("h", h), ("r", r), ("r_out", r_out), ("out", out)):
        _dev(t, name)
    if valid_mask is not None:
        _dev(valid_mask, "valid_mask")
        if valid_mask.dtype != torch.uint8 or valid_mask.numel() != T:
            raise ValueError("valid_mask must be uint8 with batch * seq_len elements")
    call("cobra_block_fwd", h.data_ptr(), r.data_ptr(), _ptr(valid_mask), w_qkv.data_ptr(), b_qkv.data_ptr(),
         w_o.data_ptr(), b_o.data_ptr(), ln2_w.data_ptr(), ln2_b.data_ptr(), w1.data_ptr(), b1.data_ptr(),
         w2.data_ptr(), b2.data_ptr(), lnn_w.data_ptr(), lnn_b.data_ptr(), r_out.data_ptr(), out.data_ptr(),
         _dtype_code(out, "out"), 1 if mask_out else 0, batch, seq_len, D, heads, F, 1 if causal else 0, float(eps),
         _stream(h))


NOALLOC_MAX_BYTES = _lib.NOALLOC_MAX_BYTES


def layer_fwd_noalloc(
    x: torch.Tensor,
    w_qkv: torch.Tensor,
    b_qkv: torch.Tensor,
    w_o: torch.Tensor,
    b_o: torch.Tensor,
    ln1_w: Optional[torch.Tensor],
    ln1_b: Optional[torch.Tensor],
    ln2_w: torch.Tensor,
    ln2_b: torch.Tensor,
    y: torch.Tensor,
    heads: int,
    causal: bool,
    eps: float = 1e-5,
    resid_out: Optional[torch.Tensor] = None,
    valid_mask: Optional[torch.Tensor] = None,
) -> None:
    """``layer_fwd`` without a workspace (``cobra_layer_fwd_noalloc``): the library's
    per-device scratch of ``NOALLOC_MAX_BYTES`` holds the intermediates, so nothing is
    allocated.  Calls that overlap on one GPU (several streams or threads) race."""
    B, S, D = x.shape
    need = layer_workspace_bytes(B, S, D, heads, valid_mask is not None, x.dtype)
    if need > NOALLOC_MAX_BYTES:
        raise ValueError(f"B={B} S={S} D={D} H={heads} needs {need} bytes of scratch; the allocation-free "
                         f"entry point holds {NOALLOC_MAX_BYTES}: use layer_fwd with a workspace")
    args = layer_fwd_args(x, w_qkv, b_qkv, w_o, b_o, ln1_w, ln1_b, ln2_w, ln2_b, y, x, heads, causal, eps,
                          resid_out, valid_mask)
    del args[13:15]  # no workspace pointer / size
    call("cobra_layer_fwd_noalloc", *args)


class LayerLaunch:
    """A bound ``cobra_layer_fwd`` (``cobra_layer_bind``): ``run(x, y, stream)``
    launches with every other argument fixed.  Keeps the buffers it names alive."""

    __slots__ = ("handle", "run_fn", "_keep", "_unbind")

    def __init__(self, x_dtype, masked, w_qkv, b_qkv, w_o, b_o, ln1_w, ln1_b, ln2_w, ln2_b, workspace, batch,
                 seq_len, d_model, heads, causal, eps):
        lib = _lib.lib()
        self.handle = None
        h = lib.cobra_layer_bind(_DT[x_dtype], 1 if masked else 0, w_qkv.data_ptr(), b_qkv.data_ptr(),
                                 w_o.data_ptr(), b_o.data_ptr(), _ptr(ln1_w), _ptr(ln1_b),
                                 ln2_w.data_ptr(), ln2_b.data_ptr(), workspace.data_ptr(), workspace.numel(),
                                 batch, seq_len, d_model, heads, 1 if causal else 0, float(eps))
        if not h:
            raise ValueError("cobra_layer_bind rejected the arguments")
        self.handle = h
        self.run_fn = lib.cobra_layer_run
        self._unbind = lib.cobra_layer_unbind
        self._keep = (w_qkv, b_qkv, w_o, b_o, ln1_w, ln1_b, ln2_w, ln2_b, workspace)

    def __del__(self):
        if self.handle:
            self._unbind(self.handle)
            self.handle = None


def check_code(fn: str, code: int) -> None:
    _lib.check(fn, code)


def raw_stream(device_index: int) -> int:
    """The current stream handle of a device, by index."""
    if _raw_stream is not None:
        return _raw_stream(device_index)
    return torch.cuda.current_stream(device_index).cuda_stream
