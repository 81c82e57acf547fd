"""Zero-padded weight layouts for shapes whose d_model, ffn_dim or head_dim is not a
multiple of 8.

The kernels move 16-byte chunks (8 fp16 values) of every operand row; the reference
accepts any ``d_model % heads == 0`` (torch_transformer_benchmark.py:30-57, "TTB") and
sends such shapes to SDPA / ``F.linear`` (TTB:1030-1071).  Here they run on the same
kernels with weights padded once per parameter version: every padded q / k / v
dimension, attention-output column, FFN activation and residual column is exactly 0,
and LayerNorms run over the true width alone (``ops.ln_strided``).
"""

from __future__ import annotations


def _round8(n: int) -> int:
    return (n + 7) // 8 * 8


class PadGeometry:
    """Widths the kernels run a block at: d_model, ffn_dim and head_dim rounded up to
    multiples of 8 (16-byte rows for the GEMMs' LDS-DMA tiles and the attention's
    operand fragments).  The reference's stack accepts any ``d_model % heads == 0``
    (TTB:30-57) and sends such shapes to SDPA / ``F.linear`` (TTB:1030-1071); here they
    run on the same kernels with zero-padded weights."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        self.d, self.heads, self.f = d_model, num_heads, ffn_dim
        self.hd = d_model // num_heads
        self.hdp = _round8(self.hd)
        self.e = num_heads * self.hdp  # padded width of q, k, v and of the attention output
        self.dp = _round8(d_model)
        self.fp = _round8(ffn_dim)

    @property
    def needed(self) -> bool:
        return (self.dp, self.hdp, self.fp) != (self.d, self.hd, self.f)


def pad_attention_weights(w_qkv, b_qkv, w_o, b_o, g: PadGeometry):
    """Zero-padded copies of the attention weights for the padded widths of ``g``: every
    head of q, k, v gets hdp - hd zero rows (and W_o the matching zero columns), d_model
    gets dp - d zero columns (and zero output rows).  The padded q . k terms and
    attention-output columns are exactly 0, as are the out-projection's pad columns."""
    H, hd, hdp, D, Dp = g.heads, g.hd, g.hdp, g.d, g.dp
    wq = w_qkv.new_zeros(3, H, hdp, Dp)
    wq[:, :, :hd, :D] = w_qkv.view(3, H, hd, D)
    bq = b_qkv.new_zeros(3, H, hdp)
    bq[:, :, :hd] = b_qkv.view(3, H, hd)
    wo = w_o.new_zeros(Dp, H, hdp)
    wo[:D, :, :hd] = w_o.view(D, H, hd)
    bo = b_o.new_zeros(Dp)
    bo[:D] = b_o
    return wq.view(3 * H * hdp, Dp), bq.view(-1), wo.view(Dp, H * hdp), bo


def pad_block_weights(w_qkv, b_qkv, w_o, b_o, w1, b1, w2, b2, g: PadGeometry):
    """The attention weights as ``pad_attention_weights``, and the FFN's: ffn_dim gets
    fp - f zero rows / columns, d_model dp - d zero columns / output rows.  The padded
    FFN activations are gelu(0) = 0 and the padded residual columns stay 0, so the first
    d columns are the unpadded block's."""
    H, hd, hdp, D, Dp, F, Fp = g.heads, g.hd, g.hdp, g.d, g.dp, g.f, g.fp
    wq, bq, wo, bo = pad_attention_weights(w_qkv, b_qkv, w_o, b_o, g)
    wi = w1.new_zeros(Fp, Dp)
    wi[:F, :D] = w1
    bi = b1.new_zeros(Fp)
    bi[:F] = b1
    wu = w2.new_zeros(Dp, Fp)
    wu[:D, :F] = w2
    bu = b2.new_zeros(Dp)
    bu[:D] = b2
    return (wq, bq, wo, bo, wi, bi, wu, bu)
