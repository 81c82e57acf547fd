"""Seeded construction, inputs and the configuration matrix (test infrastructure).

* Weights: ``torch.manual_seed(seed)`` on the CPU, then the sublayer is built in
  the reference block's order (norm1, q, k, v, out, norm2; TTB:129-131,
  73-76).  nn.Linear default init U(+-1/sqrt(d_model)); LayerNorm gamma=1,
  beta=0.  Mirrors the harness's seeding before construction (TTB:2024-2031).
* Inputs: ``randn(B, S, D)`` from a generator seeded with ``seed``, times
  ``input_scale`` (TTB:1583-1594).  The reference draws on the *device*
  generator; here the draw is always on the CPU so that the GPU path, the
  oracle and the CPU baseline see identical values, then copied over.
* Long sequences draw one generator per sequence, seeded ``(seed << 32) | b``,
  so any sampled sequence regenerates alone without a 13 GB host tensor.
* fp16 configurations: the oracle runs in fp32 on the *same* fp16-rounded
  inputs and weights (``quantize_like``), which is the reference's own scored
  practice of an fp32 layer against fp16-operand kernels (tools/sweep.py:238,
  TTB:960-1004).

The matrix is the benchmark's case list (tools/sweep.py:31-47) restricted to
the attention sublayer and to BASELINE's configurations.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import torch

from .layer import OracleAttentionSublayer


@dataclass(frozen=True)
class LayerCase:
    name: str
    batch: int
    seq_len: int
    d_model: int
    heads: int
    causal: bool = False
    dtype: str = "float16"

    @property
    def head_dim(self) -> int:
        return self.d_model // self.heads

    @property
    def tokens(self) -> int:
        return self.batch * self.seq_len

    def flops(self) -> int:
        """Algorithmic FLOPs of one sublayer forward.

        Projections ``8*T*D^2`` (q, k, v, out), attention ``4*B*S^2*D``
        non-causal (QK^T and PV), halved under causality -- the reference's
        convention (tools/time_case14.py:18).  LayerNorm / softmax / bias work
        is not counted.
        """
        t, d, s = self.tokens, self.d_model, self.seq_len
        attn = 4 * self.batch * s * s * d
        if self.causal:
            attn //= 2
        return 8 * t * d * d + attn

    def hbm_bytes(self, io_bytes: int = 2, weight_bytes: int = 2, residual_out: bool = False) -> int:
        """Algorithmic HBM bytes: x in, y out, packed weights, biases + LN params."""
        t, d = self.tokens, self.d_model
        b = t * d * (io_bytes + io_bytes) + 4 * d * d * weight_bytes + (4 * d + 4 * d) * 4
        if residual_out:
            b += 4 * t * d
        return b


# name -> case.  Non-causal with no mask unless stated; the
# reference's own matrix is causal, so a causal twin of each is tested too.
CONFIGS: Dict[str, LayerCase] = {
    "plumbing": LayerCase("plumbing", 1, 128, 128, 4, dtype="float32"),
    "base": LayerCase("base", 64, 128, 128, 4),
    "b1": LayerCase("b1", 1, 128, 128, 4),
    "b4": LayerCase("b4", 4, 128, 128, 4),
    "b16": LayerCase("b16", 16, 128, 128, 4),
    "b128": LayerCase("b128", 128, 128, 128, 4),
    "b10000": LayerCase("b10000", 10000, 128, 128, 4),
    "s32": LayerCase("s32", 64, 32, 128, 4),
    "s1024": LayerCase("s1024", 64, 1024, 128, 4),
    "h1": LayerCase("h1", 64, 128, 128, 1),
    "h2": LayerCase("h2", 64, 128, 128, 2),
    "h16": LayerCase("h16", 64, 128, 128, 16),
    "gemm": LayerCase("gemm", 64, 128, 1024, 4),
    "long": LayerCase("long", 32, 100000, 1024, 16),
}


def make_sublayer(d_model: int, heads: int, seed: int = 0) -> OracleAttentionSublayer:
    """Seeded fp32 CPU sublayer (TTB:2024-2031 order: seed, then construct)."""
    torch.manual_seed(seed)
    return OracleAttentionSublayer(d_model, heads).eval()


def make_input(batch: int, seq_len: int, d_model: int, seed: int = 0, input_scale: float = 1.0) -> torch.Tensor:
    """x ~ N(0, 1) * input_scale, fp32, on the CPU (TTB:1583-1594)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    x = torch.randn(batch, seq_len, d_model, generator=g, dtype=torch.float32)
    return x * input_scale


def make_sequence(b: int, seq_len: int, d_model: int, seed: int = 0) -> torch.Tensor:
    """Sequence ``b`` of a per-sequence-seeded batch: [1, S, D] fp32."""
    g = torch.Generator(device="cpu")
    g.manual_seed((seed << 32) | b)
    return torch.randn(1, seq_len, d_model, generator=g, dtype=torch.float32)


def quantize_like(module: torch.nn.Module, dtype: torch.dtype) -> torch.nn.Module:
    """Round every parameter through ``dtype`` and back to fp32, in place."""
    with torch.no_grad():
        for p in module.parameters():
            p.copy_(p.to(dtype).float())
    return module


def oracle_forward(
    layer: OracleAttentionSublayer,
    x: torch.Tensor,
    causal: bool = False,
    block_q: Optional[int] = None,
    return_residual: bool = False,
    valid_token_mask: Optional[torch.Tensor] = None,
):
    """fp32 oracle output for ``x`` (any dtype / device); TF32 disabled."""
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    if valid_token_mask is not None:
        valid_token_mask = valid_token_mask.to(x.device, torch.bool)
    try:
        with torch.inference_mode():
            return layer(x.float(), valid_token_mask, causal, return_residual, block_q)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
