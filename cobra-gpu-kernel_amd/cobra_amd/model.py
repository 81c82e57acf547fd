"""Drop-in transformer stack: ``CobraTransformer`` for the reference's model.

``CobraTransformer(config)`` has the parameters, construction order and
``forward(x, valid_token_mask=None)`` surface of ``BaselineTransformer`` /
``UserOptimizedTransformer`` (torch_transformer_benchmark.py:149-173,
917-1541, "TTB"): ``layers[i].{norm1, attention.{q,k,v,out}_proj, norm2,
ffn_in, ffn_out}`` and ``final_norm``, so a reference state_dict loads with
``strict=True`` and a seeded construction draws the reference's weights.

Every op runs on this library's HIP kernels through ``ops`` (no PyTorch
compute fallback).  Per block, with the residual stream ``r`` kept in fp32
and GEMM operands in fp16 (the reference's fused policy, TTB:1170-1290):

    h    = LN1(r)                       layer 0: LayerNorm kernel; later layers:
                                        the previous block's FFN epilogue
    qkv  = h Wqkv^T + b                 one [3D, D] GEMM, q|k|v order (TTB:876-883)
    ctx  = attention(qkv)               flash attention, causal per config,
                                        padded keys masked (TTB:98-113)
    r    = r + (ctx Wo^T + bo)          fp32 epilogue; padded rows' branch = 0
    h2   = LN2(r)                       same kernel for d_model <= 128, else a
                                        LayerNorm pass (TTB:1255-1283)
    f    = gelu(h2 W1^T + b1)           exact erf GELU in the GEMM epilogue
    r    = (r + f W2^T + b2) * mask     block row mask (TTB:144-145)
    h    = LN1'(r)                      the NEXT block's norm1, or final_norm with
                                        the output row mask on the last block

The op order and roundings are the reference's; the output is x.dtype.  bf16
activations run the same per-op composition with bf16 weights and bf16 GEMM /
attention operands (the residual stream stays fp32).
At d_model 128, ffn_dim 128, seq_len <= 128 (head_dim 8 / 32 / 64 / 128) and
batches of at most two rounds of workgroups, each block is ONE launch
(``cobra_block_fwd``: the query-split kernel's whole-block mode) fed by one
LayerNorm launch for layer 0's norm1; the GELU there uses a branch-free erf
(Abramowitz & Stegun 7.1.26, |error| <= 1.5e-7).  Those forwards launch directly;
other shapes replay a captured hipGraph of the whole forward for small inputs
(<= 64 MiB, TTB:1077-1079) with static input / mask buffers (TTB:1331-1360);
inputs that do not fit one device pass stream in batch chunks (TTB:1364-1508).
"""

from __future__ import annotations

import gc
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn as nn

from . import ops, streaming
from .layer import CobraSelfAttention
from .padding import PadGeometry, pad_block_weights

GRAPH_MAX_INPUT_BYTES = 64 * 1024 * 1024


@dataclass(frozen=True)
class TransformerConfig:
    """Fields and validation of the reference's ``TransformerConfig`` (TTB:28-57)."""

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


class CobraTransformerBlock(nn.Module):
    """Parameters of ``BaselineTransformerBlock`` (TTB:126-133), same names and draw order."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = CobraSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)


class _BlockPack:
    """Kernel-ready copies of one block's parameters (plain attributes, so the
    state_dict is unchanged; TTB:857-914), zero-padded when the geometry needs it.  The
    weight matrices are in the MFMA operand type ``op``: fp16, or bf16 for bf16
    activations."""

    __slots__ = ("w_qkv", "b_qkv", "w_o", "b_o", "w1", "b1", "w2", "b2", "ln1_w", "ln1_b", "ln2_w", "ln2_b")

    def __init__(self, blk: CobraTransformerBlock, geom: PadGeometry, op: torch.dtype = torch.float16) -> None:
        att = blk.attention
        with torch.no_grad():
            w = (torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight]).to(op),
                 torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias]).float(),
                 att.out_proj.weight.to(op), att.out_proj.bias.float(),
                 blk.ffn_in.weight.to(op), blk.ffn_in.bias.float(),
                 blk.ffn_out.weight.to(op), blk.ffn_out.bias.float())
            if geom.needed:
                w = pad_block_weights(*w, geom)
            (self.w_qkv, self.b_qkv, self.w_o, self.b_o, self.w1, self.b1, self.w2,
             self.b2) = (t.contiguous() for t in w)
            self.ln1_w = blk.norm1.weight.float().contiguous()
            self.ln1_b = blk.norm1.bias.float().contiguous()
            self.ln2_w = blk.norm2.weight.float().contiguous()
            self.ln2_b = blk.norm2.bias.float().contiguous()


class CobraTransformer(nn.Module):
    def __init__(self, config: TransformerConfig, graph: Optional[bool] = None) -> None:
        super().__init__()
        config.validate()
        self.config = config
        self._geom = PadGeometry(config.d_model, config.num_heads, config.ffn_dim)
        # Construction order = BaselineTransformer's (TTB:153-161).
        self.layers = nn.ModuleList(
            [CobraTransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
             for _ in range(config.num_layers)]
        )
        self.final_norm = nn.LayerNorm(config.d_model)
        # hipGraph replay: None = automatic (inputs <= 64 MiB), True / False force it.
        self.graph = graph
        # Upper bound on sequences per device pass when a batch is streamed (None: from free memory).
        self.stream_chunk: Optional[int] = None
        self._params = list(self.parameters())
        self._versioned = [not p.is_inference() for p in self._params]
        self._packs: Optional[List[_BlockPack]] = None
        self._op = torch.float16  # operand type of the packs
        self._final = None
        self._versions = None
        self._sig = None
        self._graph_ok = False
        self._graph = None
        self._static_x = self._static_m = self._static_out = None
        self._blocks = False  # the signature runs one whole-block kernel per block
        self._fast = None     # native steady-state call (cobra_host.BoundStack) of that mode

    # -- parameters -----------------------------------------------------------

    def _apply(self, fn, *args, **kwargs):
        out = super()._apply(fn, *args, **kwargs)
        self._params = list(self.parameters())
        self._versioned = [not p.is_inference() for p in self._params]
        self._packs = None
        self._sig = None
        self._fast = None
        return out

    def _packed(self, x_dtype: torch.dtype = torch.float16) -> List[_BlockPack]:
        op = torch.bfloat16 if x_dtype == torch.bfloat16 else torch.float16
        versions = tuple([p._version if v else p.data_ptr() for p, v in zip(self._params, self._versioned)])
        if self._packs is None or self._versions != versions or self._op != op:
            if not self.final_norm.weight.is_cuda:
                raise RuntimeError("CobraTransformer runs on the GPU only: move it with .to('cuda')")
            self._packs = [_BlockPack(blk, self._geom, op) for blk in self.layers]
            self._op = op
            with torch.no_grad():
                self._final = (self.final_norm.weight.float().contiguous(), self.final_norm.bias.float().contiguous())
            self._versions = versions
            self._graph = None
            self._fast = None
        return self._packs

    # -- entry point ----------------------------------------------------------

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        # Steady state of the one-kernel-per-block mode (same input signature, no mask,
        # parameters and eps unchanged): the native call checks that, allocates and
        # launches; it returns None for any other call.
        f = self._fast
        if f is not None and valid_token_mask is None:
            y = f(x)
            if y is not None:
                return y
        self._validate(x)
        packs = self._packed(x.dtype)
        if not x.is_cuda or x.numel() * x.element_size() >= streaming.STREAM_MIN_BYTES:
            if self._stream_needed(x):
                return self._run_streamed(x, valid_token_mask)
        masked = valid_token_mask is not None
        sig = (tuple(x.shape), x.dtype, x.device, masked)
        if sig != self._sig:
            # Automatic: replay a hipGraph for the composed forward (five launches per
            # block); launch the one-kernel-per-block forward directly, which measured
            # faster than its graph replay at B >= 4 (56 vs 62 us at case 1).
            cfg = self.config
            blocks = x.dtype != torch.bfloat16 and \
                ops.block_plan(x.shape[0], x.shape[1], cfg.d_model, cfg.num_heads, cfg.ffn_dim) == 1
            self._graph_ok = (self.graph if self.graph is not None else not blocks) and \
                x.numel() * x.element_size() <= GRAPH_MAX_INPUT_BYTES
            self._blocks = blocks
            self._fast = None
            self._graph = None
            self._static_x = self._static_m = self._static_out = None
            self._sig = sig
        x = x.contiguous()
        m = self._mask_bytes(valid_token_mask, x) if masked else None
        if self._graph_ok:
            return self._run_graphed(x, m, packs)
        out = self._run(x, m, packs)
        if self._blocks and m is None and x.numel() * x.element_size() < streaming.STREAM_MIN_BYTES:
            self._fast = self._make_fast(x, packs)
        return out

    def _make_fast(self, x: torch.Tensor, packs: List[_BlockPack]):
        from . import _lib

        flat = []
        for i, p in enumerate(packs):
            nw, nb = self._final if i == len(packs) - 1 else (packs[i + 1].ln1_w, packs[i + 1].ln1_b)
            flat += [p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln2_w, p.ln2_b, p.w1, p.b1, p.w2, p.b2, nw, nb]
        cfg = self.config
        return _lib.host().BoundStack(x, self._params, list(self._versions), self.final_norm,
                                      float(self.final_norm.eps), packs[0].ln1_w, packs[0].ln1_b, flat,
                                      cfg.num_heads, cfg.ffn_dim, bool(cfg.causal), ops.check_code).__call__

    def _validate(self, x: torch.Tensor) -> None:
        if x.dim() != 3 or x.shape[-1] != self.config.d_model:
            raise ValueError(f"x must be [B, S, {self.config.d_model}], got {tuple(x.shape)}")
        if x.dtype not in (torch.float16, torch.float32, torch.bfloat16):
            raise TypeError(f"x dtype {x.dtype} not supported (float16, bfloat16 or float32)")
        g = self._geom
        if g.hdp > 256 or g.dp > 4096:
            raise ValueError("the HIP kernels take head_dim <= 256 and d_model <= 4096 (after rounding up to "
                             "multiples of 8)")

    @staticmethod
    def _mask_bytes(mask: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """[B, S] token mask as contiguous device bytes (0 = padded); applied whenever given."""
        if tuple(mask.shape) != tuple(x.shape[:2]):
            raise ValueError(f"valid_token_mask must be {tuple(x.shape[:2])}, got {tuple(mask.shape)}")
        if mask.dtype not in (torch.bool, torch.uint8):
            raise TypeError(f"valid_token_mask must be bool or uint8, got {mask.dtype}")
        mask = mask.to(x.device, non_blocking=True).contiguous()
        return mask.view(torch.uint8) if mask.dtype == torch.bool else mask

    # -- the forward, as a sequence of kernel launches ---------------------------

    def _run(self, x: torch.Tensor, m: Optional[torch.Tensor], packs: List[_BlockPack]) -> torch.Tensor:
        cfg = self.config
        B, S, D = x.shape
        T = B * S
        H = cfg.num_heads
        hd = D // H
        scale = hd ** -0.5
        eps = self.final_norm.eps
        xf = x.view(T, D)
        mrow = None if m is None else m.view(T)
        out16 = x.dtype == torch.float16
        n = len(packs)
        bf16 = x.dtype == torch.bfloat16
        if not bf16 and ops.block_plan(B, S, D, H, cfg.ffn_dim) == 1:
            return self._run_blocks(x, m, packs).view(B, S, D)
        bits = None if m is None else ops.mask_bits(m.view(B, S))
        if self._geom.needed or bf16:
            # bf16: the same per-op composition with bf16 operands (the LayerNorm-epilogue
            # GEMMs, LN1-in-prologue projection and fused kernels are fp16-operand)
            return self._run_padded(x, m, mrow, bits, packs).view(B, S, D)

        # Layer 0's LN1 rides in its QKV projection where the row fits one k-tile.
        fold_ln1 = ops.ln_linear_ok(D, x.dtype)
        h = None if fold_ln1 else ops.add_ln(xf, None, None, packs[0].ln1_w, packs[0].ln1_b, cast_fp16=True,
                                             eps=eps, store_resid=False)[1]
        fused_qkv = ops.qkv_attn_fused(B, S, H, hd)
        r = xf
        for i, p in enumerate(packs):
            last = i == n - 1
            nw, nb = self._final if last else (packs[i + 1].ln1_w, packs[i + 1].ln1_b)
            if i == 0 and fold_ln1:
                qkv = ops.ln_linear(xf, p.ln1_w, p.ln1_b, p.w_qkv, p.b_qkv, eps=eps)
                ctx = ops.attn(qkv, B, S, H, hd, scale, causal=cfg.causal, key_bits=bits)
            elif fused_qkv:  # the projection inside the attention kernel (head_dim 256, S <= 128)
                ctx = ops.qkv_attn(h, p.w_qkv, p.b_qkv, B, S, H, hd, scale, causal=cfg.causal, key_bits=bits)
            else:
                qkv = ops.linear(h, p.w_qkv, p.b_qkv)
                ctx = ops.attn(qkv, B, S, H, hd, scale, causal=cfg.causal, key_bits=bits)
            if D <= 128:
                r, h2 = ops.linear_ln(ctx, p.w_o, p.b_o, r, p.ln2_w, p.ln2_b, rmask=mrow, eps=eps, mask_branch=True)
            else:
                r = ops.linear(ctx, p.w_o, p.b_o, out_fp32=True, resid=r, rmask=mrow, mask_branch=True)
                _, h2 = ops.add_ln(r, None, None, p.ln2_w, p.ln2_b, cast_fp16=True, eps=eps, store_resid=False)
            hid = ops.linear(h2, p.w1, p.b1, gelu=True)
            norm16 = out16 or not last
            if D <= 128:
                r, h = ops.linear_ln(hid, p.w2, p.b2, r, nw, nb, rmask=mrow, norm_fp16=norm16, mask_out=last,
                                     eps=eps)
            else:
                r = ops.linear(hid, p.w2, p.b2, out_fp32=True, resid=r, rmask=mrow)
                _, h = ops.add_ln(r, None, mrow, nw, nb, cast_fp16=norm16, eps=eps, store_resid=False,
                                  mask_out=last)
        return h.view(B, S, D)

    def _run_padded(self, x: torch.Tensor, m: Optional[torch.Tensor], mrow: Optional[torch.Tensor],
                    bits: Optional[torch.Tensor], packs: List[_BlockPack]) -> torch.Tensor:
        """The composed forward at the padded widths (``PadGeometry``; equal to the true
        ones when nothing needs padding): the fp32 residual is [T, dp] with its pad columns
        0, every LayerNorm normalises the d true columns of its row and writes a
        zero-padded operand (fp16, or bf16 for bf16 activations), the attention runs at
        head_dim hdp with the true scale hd^-0.5, and the last norm writes [T, d] in x.dtype."""
        cfg, g = self.config, self._geom
        op = self._op
        B, S, D = x.shape
        T = B * S
        eps = self.final_norm.eps
        scale = g.hd ** -0.5
        r = torch.zeros((T, g.dp), device=x.device, dtype=torch.float32)
        h = ops.ln_strided(x.view(T, D), D, packs[0].ln1_w, packs[0].ln1_b, out_cols=g.dp,
                           out_dtype=op, resid_out=r, eps=eps)
        n = len(packs)
        for i, p in enumerate(packs):
            last = i == n - 1
            nw, nb = self._final if last else (packs[i + 1].ln1_w, packs[i + 1].ln1_b)
            qkv = ops.linear(h, p.w_qkv, p.b_qkv)
            ctx = ops.attn(qkv, B, S, cfg.num_heads, g.hdp, scale, causal=cfg.causal, key_bits=bits)
            r = ops.linear(ctx, p.w_o, p.b_o, out_fp32=True, resid=r, rmask=mrow, mask_branch=True)
            h2 = ops.ln_strided(r, D, p.ln2_w, p.ln2_b, out_cols=g.dp, out_dtype=op, eps=eps)
            hid = ops.linear(h2, p.w1, p.b1, gelu=True)
            r = ops.linear(hid, p.w2, p.b2, out_fp32=True, resid=r, rmask=mrow)
            if last:
                h = ops.ln_strided(r, D, nw, nb, out_cols=D, out_dtype=x.dtype, mask_row=mrow,
                                   mask_resid=mrow is not None, mask_out=mrow is not None, eps=eps)
            else:
                h = ops.ln_strided(r, D, nw, nb, out_cols=g.dp, out_dtype=op, eps=eps)
        return h

    def _run_blocks(self, x: torch.Tensor, m: Optional[torch.Tensor], packs: List[_BlockPack]) -> torch.Tensor:
        """One launch per block (``cobra_block_fwd``) for the shapes the whole-block kernel
        takes: layer 0's norm1 by the LayerNorm kernel (which also widens x into the fp32
        residual), then each block reads h = norm1(r) and r, updates r in place and writes
        the next block's h (ping-pong buffers: every workgroup of a sequence reads all of
        its h rows) or, on the last block, final_norm's output with the row mask."""
        cfg = self.config
        B, S, D = x.shape
        T = B * S
        eps = self.final_norm.eps
        r, h = ops.add_ln(x.view(T, D), None, None, packs[0].ln1_w, packs[0].ln1_b, cast_fp16=True, eps=eps,
                          store_resid=True)
        h_next = torch.empty_like(h) if len(packs) > 1 else None
        out = None
        for i, p in enumerate(packs):
            last = i == len(packs) - 1
            nw, nb = self._final if last else (packs[i + 1].ln1_w, packs[i + 1].ln1_b)
            out = torch.empty((T, D), device=x.device, dtype=x.dtype) if last else h_next
            ops.block_fwd(h, r, p.w_qkv, p.b_qkv, p.w_o, p.b_o, p.ln2_w, p.ln2_b, p.w1, p.b1, p.w2, p.b2, nw, nb,
                          r, out, B, S, cfg.num_heads, cfg.causal, eps=eps,
                          valid_mask=None if m is None else m.view(T), mask_out=last and m is not None)
            if not last:
                h, h_next = out, h
        return out

    def _run_graphed(self, x, m, packs):
        if self._graph is None:
            self._static_x = x.clone()
            self._static_m = None if m is None else m.clone()
            self._run(self._static_x, self._static_m, packs)  # loads every code object outside the capture
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._static_out = self._run(self._static_x, self._static_m, packs)
            self._graph = graph
        if x.data_ptr() != self._static_x.data_ptr():
            self._static_x.copy_(x)
        if m is not None and m.data_ptr() != self._static_m.data_ptr():
            self._static_m.copy_(m)
        self._graph.replay()
        # Returned without a clone, as the reference does (TTB:1356-1360).
        return self._static_out

    # -- streaming -----------------------------------------------------------------

    def _per_seq_bytes(self, x: torch.Tensor) -> int:
        """Device bytes one sequence holds at the peak of a block (this build's model):
        fp32 residual, fp16 h / qkv / ctx / h2 / FFN hidden, the input and the output."""
        S, D, F = x.shape[1], self._geom.dp, self._geom.fp
        per_tok = 4 * D + 2 * D + 6 * D + 2 * D + 2 * D + 2 * F + 2 * D * x.element_size() + 4 * D
        return S * per_tok

    def _stream_needed(self, x: torch.Tensor) -> bool:
        nbytes = x.numel() * x.element_size()
        if x.is_cuda and nbytes < streaming.STREAM_MIN_BYTES:
            return False
        free, _ = torch.cuda.mem_get_info(self.final_norm.weight.device)
        return streaming.should_stream(x.is_cuda, nbytes, x.shape[0], self._per_seq_bytes(x) * x.shape[0], free)

    def _run_streamed(self, x, valid_token_mask):
        dev = self.final_norm.weight.device
        packs = self._packed(x.dtype)
        B = x.shape[0]
        free, _ = torch.cuda.mem_get_info(dev)
        step = streaming.plan_chunk(B, self._per_seq_bytes(x), free)
        if self.stream_chunk:
            step = max(1, min(step, int(self.stream_chunk)))
        out = torch.empty_like(x)

        def on_oom() -> None:
            gc.collect()
            torch.cuda.empty_cache()

        def is_oom(e: BaseException) -> bool:
            return isinstance(e, torch.cuda.OutOfMemoryError)

        if not x.is_cuda:
            # Copies in and out overlap the compute of neighbouring chunks.
            def run(xd, md):
                return (self._run(xd, None if md is None else self._mask_bytes(md, xd), packs),)

            streaming.stream_host(x, valid_token_mask, [out], streaming.host_chunk(B, step), run, dev, is_oom,
                                  on_oom)
            return out

        def run_chunk(b0: int, b1: int) -> None:
            xc = x[b0:b1].contiguous()
            mc = None if valid_token_mask is None else self._mask_bytes(valid_token_mask[b0:b1], xc)
            out[b0:b1].copy_(self._run(xc, mc, packs))

        streaming.run_chunked(B, step, run_chunk, on_oom, is_oom)
        return out
