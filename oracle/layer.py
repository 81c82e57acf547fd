"""fp32 restatement of the reference attention sublayer (test infrastructure).

The sublayer is the attention half of the reference block
(``torch_transformer_benchmark.py:135-142``)::

    r = x + attention(norm1(x), valid_token_mask, causal)     # TTB:141
    y = norm2(r)                                               # feeds the FFN, TTB:142

``attention`` restates ``BaselineSelfAttention.forward`` (TTB:88-123) step by
step, calling the same library routines in the same order: three ``nn.Linear``
projections, a head split to ``[B, H, S, hd]``, ``(q @ k^T) * scale`` (the scale
is applied after the product, TTB:98), ``-inf`` fills for the causal upper
triangle (TTB:100-104) and for invalid keys (TTB:106-109), softmax in fp32 cast
back to the activation dtype (TTB:112), ``probs @ v`` (TTB:113), head merge,
``out_proj`` (TTB:119) and the output row mask (TTB:121-122).

``block_q`` visits the query axis in blocks, which is how
``tools/reference_chunked.py:73-128`` makes S = 100000 checkable: softmax runs
along keys, so blocking queries changes no arithmetic, and under causality the
keys past the block's last query are never formed (``kv_end``,
reference_chunked.py:103).
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch
import torch.nn as nn


class OracleSelfAttention(nn.Module):
    """Restates ``BaselineSelfAttention`` (TTB:60-123).

    Parameter names, shapes and the construction order of the four projections
    (q, k, v, out -- TTB:73-76) match the reference, so a state_dict loads in
    either direction and seeded construction draws the same weights.
    """

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:  # TTB:65-66
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5  # TTB:71
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)

    def _heads(self, t: torch.Tensor) -> torch.Tensor:
        """[B, S, D] -> [B, H, S, hd], materialised (TTB:78-84)."""
        b, s, _ = t.shape
        t = t.view(b, s, self.num_heads, self.head_dim)
        return t.transpose(1, 2).contiguous()

    def _probs_times_v(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        q0: int,
        valid_token_mask: Optional[torch.Tensor],
        causal: bool,
        out_dtype: torch.dtype,
    ) -> torch.Tensor:
        """Scores, masks, fp32 softmax and PV for queries ``q0 .. q0+len(q)``.

        ``k``/``v`` hold keys ``0 .. kv_end``; ``kv_end`` is S, or the block's
        last query + 1 under causality (the keys beyond it would be -inf).
        """
        kv_end = k.shape[-2]
        # k^T made contiguous: bf16 batched products with a transposed right operand have
        # faulted this GPU, so no reference ever passes one.
        scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) * self.scale  # TTB:98
        if causal:  # TTB:100-104 (triu(diagonal=1) -> -inf)
            rows = torch.arange(q0, q0 + q.shape[-2], device=q.device)
            cols = torch.arange(kv_end, device=q.device)
            future = cols[None, :] > rows[:, None]
            scores = scores.masked_fill(future, float("-inf"))
        if valid_token_mask is not None:  # TTB:106-109, keys only
            bad_key = ~valid_token_mask[:, None, None, :kv_end]
            scores = scores.masked_fill(bad_key, float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(dtype=out_dtype)  # TTB:112
        return torch.matmul(probs, v)  # TTB:113

    def forward(
        self,
        x: torch.Tensor,
        valid_token_mask: Optional[torch.Tensor] = None,
        causal: bool = False,
        block_q: Optional[int] = None,
    ) -> torch.Tensor:
        b, s, _ = x.shape
        q = self._heads(self.q_proj(x))  # TTB:94-96
        k = self._heads(self.k_proj(x))
        v = self._heads(self.v_proj(x))

        if block_q is None or block_q >= s:
            ctx = self._probs_times_v(q, k, v, 0, valid_token_mask, causal, x.dtype)
        else:
            # tools/reference_chunked.py:94-121: heads one at a time, queries in
            # blocks of block_q; identical arithmetic per query row.
            ctx = torch.empty_like(q)
            for h in range(self.num_heads):
                for q0 in range(0, s, block_q):
                    q1 = min(q0 + block_q, s)
                    kv_end = q1 if causal else s
                    ctx[:, h : h + 1, q0:q1] = self._probs_times_v(
                        q[:, h : h + 1, q0:q1],
                        k[:, h : h + 1, :kv_end],
                        v[:, h : h + 1, :kv_end],
                        q0,
                        valid_token_mask,
                        causal,
                        x.dtype,
                    )

        merged = ctx.transpose(1, 2).contiguous().view(b, s, self.d_model)  # TTB:114-118
        out = self.out_proj(merged)  # TTB:119
        if valid_token_mask is not None:  # TTB:121-122
            out = out.masked_fill(~valid_token_mask[..., None], 0)
        return out


class OracleAttentionSublayer(nn.Module):
    """norm1 -> attention -> residual add -> norm2 (TTB:129-131, 141-142).

    Module and parameter names equal the reference block's (``norm1.*``,
    ``attention.{q,k,v,out}_proj.*``, ``norm2.*``), and the construction order
    norm1, attention, norm2 equals the first three members of
    ``BaselineTransformerBlock.__init__`` (TTB:129-131).  LayerNorm draws no
    random numbers, so ``torch.manual_seed(s)`` followed by this constructor
    draws exactly the attention weights of layer 0 of a reference model built
    under the same seed.
    """

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)  # eps 1e-5, biased variance
        self.attention = OracleSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)

    def forward(
        self,
        x: torch.Tensor,
        valid_token_mask: Optional[torch.Tensor] = None,
        causal: bool = False,
        return_residual: bool = False,
        block_q: Optional[int] = None,
    ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
        r = x + self.attention(self.norm1(x), valid_token_mask, causal, block_q)
        y = self.norm2(r)
        return (r, y) if return_residual else y
