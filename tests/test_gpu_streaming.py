"""Host-resident inputs: the batch streams through the GPU in chunks, copies in and
out overlapping the compute of neighbouring chunks (TTB:1364-1508 streams the same
way, without the overlap).  Chunking is exact: sequences are independent in every
op (TTB:1446-1450), so the streamed result must pass the gate against the oracle
like a device-resident call, for ragged chunk tails, masks, pinned and pageable
inputs, and the residual output.
"""

import pytest
import torch

from oracle import OracleTransformerConfig, compare_outputs, make_input, make_model, model_forward, quantize_like

from _gpu_util import DEV, build_pair, log, oracle_on

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("pinned", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_sublayer_host_input_streams(pinned, masked):
    ref, mod = build_pair(128, 4)
    mod.stream_chunk = 8  # 37 sequences -> chunks of 8, 8, 8, 8, 5
    B, S = 37, 128
    x = make_input(B, S, 128, seed=12).half()
    m = None
    if masked:
        lengths = torch.randint(1, S + 1, (B,), generator=torch.Generator().manual_seed(3))
        m = torch.arange(S)[None, :] < lengths[:, None]
    if pinned:
        x = x.pin_memory()
    with torch.inference_mode():
        r, y = mod(x, m, return_residual=True)
        torch.cuda.synchronize()
    assert not y.is_cuda and not r.is_cuda and y.dtype == torch.float16 and r.dtype == torch.float32
    want_r, want_y = oracle_on(ref, x.float(), False, "cpu", return_residual=True, mask=m)
    res = compare_outputs(want_y, y.float())
    log(f"[stream sublayer pinned={pinned} masked={masked}] max_abs={res.max_abs_error:.3e} "
        f"failed={res.failed_elements}")
    assert res.passed, res
    assert compare_outputs(want_r, r).passed


def test_host_input_with_mask_just_made_on_the_gpu():
    """Host x, and a device mask whose producing kernels are still queued on the
    compute stream when the call starts: the copy stream must read it only after them."""
    ref, mod = build_pair(128, 4)
    mod.stream_chunk = 4
    B, S = 13, 128
    x = make_input(B, S, 128, seed=21).half()
    lengths = torch.randint(1, S + 1, (B,), generator=torch.Generator().manual_seed(8))
    want_m = torch.arange(S)[None, :] < lengths[:, None]
    with torch.inference_mode():
        # A long queue ahead of the mask's producer, so a copy that did not wait
        # for it would read the buffer before it is written.
        big = torch.randn(4096, 4096, device=DEV)
        for _ in range(20):
            big = big @ big * 1e-3
        m = torch.zeros(B, S, dtype=torch.bool, device=DEV)
        m |= torch.arange(S, device=DEV)[None, :] < lengths.to(DEV)[:, None]
        y = mod(x, m)
        torch.cuda.synchronize()
    want = oracle_on(ref, x.float(), False, "cpu", mask=want_m)
    res = compare_outputs(want, y.float())
    log(f"[stream fresh device mask] max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
    assert res.passed, res


def test_model_host_input_streams():
    from cobra_amd import CobraTransformer, TransformerConfig

    cfg = (10, 128, 128, 4, 256, 2, True)
    ref = quantize_like(make_model(OracleTransformerConfig(*cfg), seed=0), torch.float16)
    mod = CobraTransformer(TransformerConfig(*cfg))
    mod.load_state_dict(ref.state_dict(), strict=True)
    mod = mod.to(device=DEV, dtype=torch.float16).eval()
    mod.stream_chunk = 3
    x = make_input(10, 128, 128, seed=5).half()
    m = torch.rand(10, 128, generator=torch.Generator().manual_seed(1)) < 0.8
    m[:, 0] = True
    with torch.inference_mode():
        y = mod(x, m)
        torch.cuda.synchronize()
    assert not y.is_cuda
    res = compare_outputs(model_forward(ref, x, m), y.float())
    log(f"[stream model] max_abs={res.max_abs_error:.3e} failed={res.failed_elements}")
    assert res.passed, res
