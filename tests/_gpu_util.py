"""Shared helpers of the GPU parity tests (not collected: no test_ prefix)."""

from __future__ import annotations

import sys

import torch

from oracle import compare_outputs, make_input, make_sublayer, quantize_like
from oracle.cases import LayerCase, oracle_forward

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def build_pair(d_model: int, heads: int, seed: int = 0, dtype: torch.dtype = torch.float16, graph=None):
    """(fp32 oracle on dtype-rounded weights, HIP module in dtype on the GPU)."""
    from cobra_amd import CobraAttentionSublayer

    ref = make_sublayer(d_model, heads, seed=seed)
    if dtype in (torch.float16, torch.bfloat16):
        quantize_like(ref, dtype)
    mod = CobraAttentionSublayer(d_model, heads, graph=graph)
    mod.load_state_dict(ref.state_dict(), strict=True)
    mod = mod.to(device=DEV, dtype=dtype).eval()
    return ref, mod


def randomise_affine(ref, seed: int) -> None:
    """Non-trivial LayerNorm weights / biases and projection biases, fp16-representable
    (the reference initialises LayerNorms to 1 / 0 and draws the biases with the weights)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for ln in (ref.norm1, ref.norm2):
            ln.weight.copy_((torch.rand(ln.weight.shape, generator=g) + 0.5).half().float())
            ln.bias.copy_(((torch.rand(ln.bias.shape, generator=g) - 0.5) * 0.6).half().float())
        att = ref.attention
        for lin in (att.q_proj, att.k_proj, att.v_proj, att.out_proj):
            lin.bias.copy_(((torch.rand(lin.bias.shape, generator=g) - 0.5) * 0.2).half().float())


def oracle_on(ref, x: torch.Tensor, causal: bool, device, block_q=None, return_residual=False, mask=None):
    """Run the fp32 oracle on ``device`` (CPU for small cases, the GPU for big ones)."""
    layer = ref.to(device)
    try:
        out = oracle_forward(layer, x.to(device), causal=causal, block_q=block_q, return_residual=return_residual,
                             valid_token_mask=mask)
    finally:
        ref.to("cpu")
    if return_residual:
        return out[0].cpu(), out[1].cpu()
    return out.cpu()


def check_case(case: LayerCase, seed: int = 0, input_seed: int = 0, oracle_device="cpu", subset=None):
    """Run the HIP sublayer on the full batch; compare (a subset of) sequences."""
    log(f"[case] {case.name} B{case.batch} S{case.seq_len} D{case.d_model} H{case.heads} causal={case.causal}")
    ref, mod = build_pair(case.d_model, case.heads, seed=seed)
    x = make_input(case.batch, case.seq_len, case.d_model, seed=input_seed).half()
    with torch.inference_mode():
        y = mod(x.to(DEV), causal=case.causal)
        torch.cuda.synchronize()
    y = y.float().cpu()
    log(f"[case] {case.name}: plan={'fused' if mod.plan == 0 else 'staged'}")
    rows = list(range(case.batch)) if subset is None else subset
    want = oracle_on(ref, x[rows].float(), case.causal, oracle_device)
    res = compare_outputs(want, y[rows])
    log(f"[case] {case.name}: max_abs={res.max_abs_error:.3e} max_rel={res.max_relative_error:.3e} "
        f"failed={res.failed_elements}/{res.total_elements}")
    return res
