"""fp32 restatement of the reference transformer stack (test infrastructure).

Restates, step by step and with the same library routines:

* ``TransformerConfig`` (TTB:28-57): fields and ``validate``;
* ``BaselineTransformerBlock`` (TTB:126-146)::

      x = x + attention(norm1(x), valid_token_mask, causal)          # TTB:141
      x = x + ffn_out(gelu(ffn_in(norm2(x)), approximate="none"))    # TTB:142
      x = x.masked_fill(~valid_token_mask[..., None], 0)             # TTB:144-145

* ``BaselineTransformer`` (TTB:149-173): the blocks in order, ``final_norm``,
  and the output row mask.

The attention is ``OracleSelfAttention`` (TTB:60-123), whose own checks live in
``tests/test_oracle.py``; construction order (norm1, attention, norm2, ffn_in,
ffn_out per block; final_norm last, TTB:129-133, 153-161) equals the
reference's, so a seeded build draws the reference's weights and a state_dict
loads in either direction.  ``block_q`` forwards to the attention's
query-blocked evaluation for sequences whose [S, S] scores cannot be formed.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .layer import OracleSelfAttention


@dataclass(frozen=True)
class OracleTransformerConfig:
    """Restates ``TransformerConfig`` (TTB:28-57)."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads", "ffn_dim", "num_layers"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(f"d_model ({self.d_model}) must be divisible by num_heads ({self.num_heads})")


class OracleTransformerBlock(nn.Module):
    """Restates ``BaselineTransformerBlock`` (TTB:126-146)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = OracleSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor], causal: bool,
                block_q: Optional[int] = None) -> torch.Tensor:
        x = x + self.attention(self.norm1(x), valid_token_mask, causal, block_q)  # TTB:141
        x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))  # TTB:142
        if valid_token_mask is not None:  # TTB:144-145
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


class OracleTransformer(nn.Module):
    """Restates ``BaselineTransformer`` (TTB:149-173)."""

    def __init__(self, config: OracleTransformerConfig) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            [OracleTransformerBlock(config.d_model, config.num_heads, config.ffn_dim) for _ in range(config.num_layers)]
        )
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None,
                block_q: Optional[int] = None) -> torch.Tensor:
        for layer in self.layers:
            x = layer(x, valid_token_mask, self.config.causal, block_q)
        x = self.final_norm(x)
        if valid_token_mask is not None:  # TTB:171-172
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


def make_model(config: OracleTransformerConfig, seed: int = 0) -> OracleTransformer:
    """Seeded fp32 model on the CPU (the harness seeds, then constructs; TTB:2024-2031)."""
    torch.manual_seed(seed)
    return OracleTransformer(config).eval()


def model_forward(model: OracleTransformer, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None,
                  block_q: Optional[int] = None) -> torch.Tensor:
    """fp32 output for ``x`` (any dtype / device); TF32 disabled."""
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    if valid_token_mask is not None:
        valid_token_mask = valid_token_mask.to(x.device, torch.bool)
    try:
        with torch.inference_mode():
            return model(x.float(), valid_token_mask, block_q)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
