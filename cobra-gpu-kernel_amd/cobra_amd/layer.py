"""Drop-in attention sublayer: norm1 -> multi-head attention -> +residual -> norm2.

``CobraAttentionSublayer`` is the attention half of the reference block
(``torch_transformer_benchmark.py:135-142``) with the reference module's
parameter names, shapes and construction order, so ``load_state_dict`` works
in both directions and ``torch.manual_seed(s)`` draws the same weights.  Its
``forward(x, valid_token_mask=None)`` keeps the reference call surface
(TTB:1512-1516) and returns ``y = norm2(x + attention(norm1(x)))`` in x.dtype.

Every forward runs on hand-written HIP kernels through the C ABI
(``cobra_layer_fwd``): there is no PyTorch compute fallback.  The host side
mirrors the reference's orchestration (TTB:857-1541):

* weights are packed lazily on the first forward, as plain attributes so
  ``state_dict`` is unchanged (TTB:857-864): one fp16 ``[3D, D]`` q|k|v
  matrix in that order (TTB:876-883), fp16 ``W_o``, fp32 biases and LayerNorm
  parameters; for bf16 activations the two matrices are bf16 and the sublayer runs
  the staged kernels with bf16 MFMA operands.  The pack is rebuilt whenever a parameter changes (in-place
  updates bump its version), which the reference did only on shape changes;
* the library picks the plan: one fused kernel for the whole sublayer
  (S <= 128, d_model <= 128) or a staged pipeline of four kernels.  Either is
  launched directly by default: on this runtime a hipGraph replay carries
  ~13 us of fixed latency against ~2.5 us per direct launch, and the sublayer
  is one to five launches, so the reference's graph gate (small inputs,
  TTB:1077-1079) would cost 10-20 us per forward here.  ``graph=True``
  captures the forward once into a hipGraph (``torch.cuda.CUDAGraph`` on ROCm)
  for inputs <= 64 MiB and replays it, with the output buffer returned without
  a clone as the reference does (TTB:1356-1360);
* inputs that do not fit one device pass are streamed in batch chunks sized
  from ``hipMemGetInfo`` with halve-on-OOM (``streaming``, TTB:1364-1508);
* ``valid_token_mask`` ([B, S] bool) masks padded keys and zeroes the padded
  rows' attention output, as ``BaselineSelfAttention`` does (TTB:106-109,
  121-122), for any mask (not only left-aligned padding).  It is applied
  whenever given, without a host-side ``.all()`` test; the graph path copies
  it into a static buffer like the reference (TTB:1338, 1353-1354).
"""

from __future__ import annotations

import gc
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn

from . import ops, streaming
from .padding import PadGeometry, pad_attention_weights

GRAPH_MAX_INPUT_BYTES = 64 * 1024 * 1024


class CobraSelfAttention(nn.Module):
    """Parameters of ``BaselineSelfAttention`` (TTB:60-76): q, k, v, out projections.

    Only a container here -- the sublayer runs the whole attention in its
    kernels -- but with identical names, shapes, init and draw order.
    """

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)


class _Pack:
    """Kernel-ready copies of the parameters (never registered on the module).

    LN1's elementwise affine is folded into the QKV projection, which consumes
    nothing else of LN1's output:
        (n * g1 + b1) W^T + b = n (W diag(g1))^T + (b + W b1),   n = (x - mean) * rstd,
    so the kernels normalise without reading g1 / b1 (``ln1_w = ln1_b = None``
    selects that form of ``cobra_layer_fwd``).  W diag(g1) is rounded to the operand
    type (fp16, or bf16 for bf16 activations) once, as W itself is; the bias term is
    formed in fp64 and stored in fp32.
    """

    __slots__ = ("w_qkv", "b_qkv", "w_o", "b_o", "ln1_w", "ln1_b", "ln2_w", "ln2_b", "versions", "pad", "geom",
                 "one", "zero", "op")

    def __init__(self, m: "CobraAttentionSublayer", versions, op: torch.dtype = torch.float16) -> None:
        att = m.attention
        self.op = op
        with torch.no_grad():
            w = torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight]).float()
            b = torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias]).double()
            g1 = m.norm1.weight.float()
            self.w_qkv = (w * g1).to(op).contiguous()
            self.b_qkv = (b + w.double() @ m.norm1.bias.double()).float().contiguous()
            self.ln1_w = None
            self.ln1_b = None
            self.w_o = att.out_proj.weight.to(op).contiguous()
            self.b_o = att.out_proj.bias.float().contiguous()
            self.ln2_w = m.norm2.weight.float().contiguous()
            self.ln2_b = m.norm2.bias.float().contiguous()
            # d_model or head_dim not a multiple of 8: zero-padded copies made here, once
            # per parameter version (the C ABI's padded plan, which takes the unpadded
            # weights, lays them out again on every call).
            att_ = m.attention
            self.geom = PadGeometry(att_.d_model, att_.num_heads, att_.d_model)
            self.pad = None
            if self.geom.needed:
                self.pad = tuple(t.contiguous() for t in pad_attention_weights(self.w_qkv, self.b_qkv, self.w_o,
                                                                               self.b_o, self.geom))
                self.one = torch.ones(att_.d_model, device=self.w_o.device)
                self.zero = torch.zeros(att_.d_model, device=self.w_o.device)
        self.versions = versions


class _Fast:
    """The steady-state launch of one input signature: ``cobra_layer_fwd`` bound
    (``cobra_layer_bind``) with everything but x, y and the stream, and the native
    call around it (``cobra_host.BoundForward``: checks x's signature, the parameters'
    versions and norm1's eps, allocates y, launches on the current stream)."""

    __slots__ = ("launch", "call")


class CobraAttentionSublayer(nn.Module):
    def __init__(self, d_model: int, num_heads: int, causal: bool = False, eps: float = 1e-5,
                 graph: Optional[bool] = None) -> None:
        super().__init__()
        # Construction order = BaselineTransformerBlock's first members (TTB:129-131).
        self.norm1 = nn.LayerNorm(d_model, eps=eps)
        self.attention = CobraSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model, eps=eps)
        self._fast: Optional[_Fast] = None
        self.causal = causal
        # hipGraph replay: None / False = direct launches (cheaper for the one to five
        # launches of a sublayer on this runtime); True = replay a captured graph for
        # inputs <= 64 MiB.
        self.graph = graph
        # Upper bound on sequences per device pass when a batch is streamed (None: from free memory).
        self.stream_chunk: Optional[int] = None
        self.plan: Optional[int] = None
        self._params = list(self.parameters())
        self._versioned = [not p.is_inference() for p in self._params]
        self._pack: Optional[_Pack] = None
        self._sig = None
        self._ws: Optional[torch.Tensor] = None
        self._graph_ok = False
        self._graph = None
        self._static_x: Optional[torch.Tensor] = None
        self._static_y: Optional[torch.Tensor] = None
        self._static_r: Optional[torch.Tensor] = None
        self._static_m: Optional[torch.Tensor] = None

    @property
    def causal(self) -> bool:
        return self._causal

    @causal.setter
    def causal(self, value: bool) -> None:
        # The bound steady-state launch has the mode baked in.
        self._causal = bool(value)
        self._fast = None

    # -- parameters ---------------------------------------------------------

    def _apply(self, fn, *args, **kwargs):
        # .to() / .half() / .cuda() replace parameter storage: drop every cache.
        out = super()._apply(fn, *args, **kwargs)
        self._params = list(self.parameters())
        self._versioned = [not p.is_inference() for p in self._params]
        self._pack = None
        self._sig = None
        self._fast = None
        return out

    def _versions(self):
        # In-place updates (load_state_dict, optimiser-style edits) bump _version.
        # Inference tensors (made under torch.inference_mode) keep no version
        # counter; for those only a storage change is detected.
        return tuple([p._version if v else p.data_ptr() for p, v in zip(self._params, self._versioned)])

    def _packed(self, x_dtype: torch.dtype = torch.float16) -> _Pack:
        # MFMA operand type of the packed weights: bf16 for bf16 activations, else fp16.
        op = torch.bfloat16 if x_dtype == torch.bfloat16 else torch.float16
        versions = self._versions()
        if self._pack is None or self._pack.versions != versions or self._pack.op != op:
            if not self.norm1.weight.is_cuda:
                raise RuntimeError("CobraAttentionSublayer runs on the GPU only: move it with .to('cuda')")
            self._pack = _Pack(self, versions, op)
            self._graph = None  # the graph baked in the old buffers' addresses
            self._fast = None
        return self._pack

    # -- entry point ----------------------------------------------------------

    def forward(
        self,
        x: torch.Tensor,
        valid_token_mask: Optional[torch.Tensor] = None,
        causal: Optional[bool] = None,
        return_residual: bool = False,
    ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
        # Steady state of the common call (same input signature, a device mask or none as
        # bound, weights and eps unchanged): the native call checks all of that,
        # allocates y and launches; it returns None for any other call.  At the small
        # shapes the kernel takes ~7 us, as long as the checks, the allocation and the
        # launch took from Python, so this path is what back-to-back forwards are bound by.
        f = self._fast
        if f is not None and causal is None and not return_residual:
            y = f.call(x, valid_token_mask)
            if y is not None:
                return y
        fast_ok = causal is None and not return_residual
        causal = self.causal if causal is None else bool(causal)
        pack = self._packed(x.dtype)
        # Free memory moves between calls, so big or host-resident inputs are
        # re-checked every time (TTB:1402-1406); small ones never pay for it.
        if not x.is_cuda or x.numel() * x.element_size() >= streaming.STREAM_MIN_BYTES:
            self._validate(x)
            if self._stream_needed(x):
                return self._run_streamed(x, valid_token_mask, causal, return_residual)
        masked = valid_token_mask is not None
        sig = (x.shape, x.dtype, x.device, causal, return_residual, masked)
        if sig != self._sig:
            self._validate(x)
            self._prepare(sig, x, masked)
        if not x.is_contiguous():
            x = x.contiguous()
        m = self._mask_bytes(valid_token_mask, x) if masked else None
        if self._graph_ok:
            return self._run_graphed(x, m, pack, causal, return_residual)
        out = self._run_eager(x, m, pack, causal, return_residual)
        if fast_ok and pack.pad is None and x.is_cuda and x.numel() * x.element_size() < streaming.STREAM_MIN_BYTES:
            self._fast = self._make_fast(x, pack, masked)
        return out

    def _make_fast(self, x: torch.Tensor, pack: _Pack, masked: bool) -> _Fast:
        from . import _lib

        f = _Fast()
        B, S, D = x.shape
        f.launch = ops.LayerLaunch(x.dtype, masked, pack.w_qkv, pack.b_qkv, pack.w_o, pack.b_o, pack.ln1_w,
                                   pack.ln1_b, pack.ln2_w, pack.ln2_b, self._ws, B, S, D,
                                   self.attention.num_heads, self.causal, self.norm1.eps)
        f.call = _lib.host().BoundForward(f.launch.handle, x, self._params, list(pack.versions), self.norm1,
                                          float(self.norm1.eps), masked, ops.check_code).__call__
        return f

    # -- planning -------------------------------------------------------------

    def _validate(self, x: torch.Tensor) -> None:
        if x.dim() != 3 or x.shape[-1] != self.attention.d_model:
            raise ValueError(f"x must be [B, S, {self.attention.d_model}], got {tuple(x.shape)}")
        if x.dtype not in (torch.float16, torch.float32, torch.bfloat16):
            raise TypeError(f"x dtype {x.dtype} not supported (float16, bfloat16 or float32)")

    @staticmethod
    def _mask_bytes(mask: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """The [B, S] token mask as contiguous device bytes (0 = padded).

        A bool mask is reinterpreted, not converted (TTB:1203-1205).  The mask
        is always applied -- there is no ``.all()`` test, which would cost a
        device synchronisation per call.
        """
        if tuple(mask.shape) != tuple(x.shape[:2]):
            raise ValueError(f"valid_token_mask must be {tuple(x.shape[:2])}, got {tuple(mask.shape)}")
        if mask.dtype not in (torch.bool, torch.uint8):
            raise TypeError(f"valid_token_mask must be bool or uint8, got {mask.dtype}")
        if mask.device != x.device:
            mask = mask.to(x.device, non_blocking=True)
        mask = mask.contiguous()
        return mask.view(torch.uint8) if mask.dtype == torch.bool else mask

    def _prepare(self, sig, x: torch.Tensor, masked: bool) -> None:
        """Per-signature set-up (the reference's _prepare, TTB:948-1081): plan,
        workspace, graph gate.  Never runs on the steady-state path."""
        B, S, D = x.shape
        H = self.attention.num_heads
        self.plan = ops.layer_plan(B, S, D, H, masked, x.dtype)
        # The padded plan runs on the pack's padded weights with tensors of its own.
        nbytes = 0 if self.plan == ops.PLAN_PADDED else ops.layer_workspace_bytes(B, S, D, H, masked, x.dtype)
        self._ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        small = x.numel() * x.element_size() <= GRAPH_MAX_INPUT_BYTES
        self._graph_ok = bool(self.graph) and small
        self._graph = None
        self._static_x = self._static_y = self._static_r = self._static_m = None
        self._fast = None
        self._sig = sig

    def _launch(self, x, m, y, r, pack: _Pack, ws: torch.Tensor, causal: bool) -> None:
        if pack.pad is not None:
            self._launch_padded(x, m, y, r, pack, causal)
            return
        ops.layer_fwd(x, pack.w_qkv, pack.b_qkv, pack.w_o, pack.b_o, pack.ln1_w, pack.ln1_b, pack.ln2_w,
                      pack.ln2_b, y, ws, self.attention.num_heads, causal, self.norm1.eps, resid_out=r,
                      valid_mask=m)

    def _launch_padded(self, x, m, y, r, pack: _Pack, causal: bool) -> None:
        """The sublayer at the padded widths (d_model or head_dim not a multiple of 8) on
        the pack's padded weights: LN1 over the true width into a zero-padded operand, the
        QKV projection, attention at head_dim hdp with the true scale hd^-0.5, the fp32
        out-projection branch (padded rows' branch zeroed, TTB:121-122), and LN2 of
        x + branch over the true width into y (and r)."""
        wq, bq, wo, bo = pack.pad
        g = pack.geom
        B, S, D = x.shape
        T = B * S
        eps = self.norm1.eps
        xf = x.view(T, D)
        mrow = None if m is None else m.view(T)
        bits = None if m is None else ops.mask_bits(m.view(B, S))
        h = ops.ln_strided(xf, D, pack.one, pack.zero, out_cols=g.dp, out_dtype=pack.op, eps=eps)
        qkv = ops.linear(h, wq, bq)
        ctx = ops.attn(qkv, B, S, g.heads, g.hdp, g.hd ** -0.5, causal=causal, key_bits=bits)
        branch = ops.linear(ctx, wo, bo, out_fp32=True, rmask=mrow, mask_branch=True)
        ops.ln_strided(xf, D, pack.ln2_w, pack.ln2_b, branch=branch, resid_out=None if r is None else r.view(T, D),
                       eps=self.norm2.eps, out=y.view(T, D))

    def _run_eager(self, x, m, pack, causal, return_residual, ws=None):
        y = torch.empty_like(x)
        r = torch.empty(x.shape, dtype=torch.float32, device=x.device) if return_residual else None
        self._launch(x, m, y, r, pack, self._ws if ws is None else ws, causal)
        return (r, y) if return_residual else y

    def _run_graphed(self, x, m, pack, causal, return_residual):
        if self._graph is None:
            self._static_x = x.clone()
            self._static_m = None if m is None else m.clone()
            self._static_y = torch.empty_like(x)
            self._static_r = (torch.empty(x.shape, dtype=torch.float32, device=x.device)
                              if return_residual else None)
            # One eager pass first: loads the code objects outside the capture.
            self._launch(self._static_x, self._static_m, self._static_y, self._static_r, pack, self._ws, causal)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._launch(self._static_x, self._static_m, self._static_y, self._static_r, pack, self._ws,
                             causal)
            self._graph = graph
        if x.data_ptr() != self._static_x.data_ptr():
            self._static_x.copy_(x)
        if m is not None and m.data_ptr() != self._static_m.data_ptr():
            self._static_m.copy_(m)
        self._graph.replay()
        return (self._static_r, self._static_y) if return_residual else self._static_y

    def input_buffer(self) -> Optional[torch.Tensor]:
        """The captured graph's static input: writing into it and passing it
        back to ``forward`` skips the input copy."""
        return self._static_x

    # -- streaming ------------------------------------------------------------

    def _per_seq_bytes(self, x: torch.Tensor, return_residual: bool) -> int:
        B, S, D = x.shape
        # The staged plan's workspace, which is linear in the batch: chunks that
        # take the fused plan instead need less.
        ws = -(-ops.layer_workspace_bytes(B, S, D, self.attention.num_heads, True, torch.float32) // B) if B else 0
        return streaming.live_bytes_per_sequence(ws, S, D, x.element_size(), return_residual)

    def _stream_needed(self, x: torch.Tensor) -> bool:
        dev = self.norm1.weight.device
        nbytes = x.numel() * x.element_size()
        if x.is_cuda and nbytes < streaming.STREAM_MIN_BYTES:
            return False
        free, _ = torch.cuda.mem_get_info(dev)
        live = self._per_seq_bytes(x, False) * x.shape[0]
        return streaming.should_stream(x.is_cuda, nbytes, x.shape[0], live, free)

    def _run_streamed(self, x, valid_token_mask, causal, return_residual):
        dev = self.norm1.weight.device
        pack = self._packed(x.dtype)
        B, S, D = x.shape
        host = not x.is_cuda
        masked = valid_token_mask is not None
        if masked:
            if tuple(valid_token_mask.shape) != (B, S):
                raise ValueError(f"valid_token_mask must be {(B, S)}, got {tuple(valid_token_mask.shape)}")
            if valid_token_mask.dtype not in (torch.bool, torch.uint8):
                raise TypeError(f"valid_token_mask must be bool or uint8, got {valid_token_mask.dtype}")
        free, _ = torch.cuda.mem_get_info(dev)
        step = streaming.plan_chunk(B, self._per_seq_bytes(x, return_residual), free)
        if self.stream_chunk:
            step = max(1, min(step, int(self.stream_chunk)))
        y_all = torch.empty_like(x)
        r_all = torch.empty(x.shape, dtype=torch.float32, device=x.device) if return_residual else None
        ws_cache = {}

        def workspace(n: int) -> torch.Tensor:
            if n not in ws_cache:
                ws_cache.clear()
                ws_cache[n] = torch.empty(ops.layer_workspace_bytes(n, S, D, self.attention.num_heads, masked,
                                                                    x.dtype),
                                          dtype=torch.uint8, device=dev)
            return ws_cache[n]

        def on_oom() -> None:
            ws_cache.clear()
            gc.collect()
            torch.cuda.empty_cache()

        def is_oom(e: BaseException) -> bool:
            return isinstance(e, torch.cuda.OutOfMemoryError)

        if host:
            # Copies in and out overlap the compute of neighbouring chunks.
            def run(xd, md):
                mc = self._mask_bytes(md, xd) if masked else None
                out = self._run_eager(xd, mc, pack, causal, return_residual, ws=workspace(xd.shape[0]))
                return out if return_residual else (out,)

            outs = [r_all, y_all] if return_residual else [y_all]
            streaming.stream_host(x, valid_token_mask, outs, streaming.host_chunk(B, step), run, dev, is_oom,
                                  on_oom)
            return (r_all, y_all) if return_residual else y_all

        def run_chunk(b0: int, b1: int) -> None:
            xc = x[b0:b1].contiguous()
            mc = self._mask_bytes(valid_token_mask[b0:b1], xc) if masked else None
            out = self._run_eager(xc, mc, pack, causal, return_residual, ws=workspace(b1 - b0))
            if return_residual:
                r_all[b0:b1].copy_(out[0])
                y_all[b0:b1].copy_(out[1])
            else:
                y_all[b0:b1].copy_(out)

        def on_oom() -> None:
            ws_cache.clear()
            gc.collect()
            torch.cuda.empty_cache()

        streaming.run_chunked(B, step, run_chunk, on_oom, is_oom)
        return (r_all, y_all) if return_residual else y_all
