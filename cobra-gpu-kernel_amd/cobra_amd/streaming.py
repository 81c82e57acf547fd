"""Batch-chunk streaming for sublayer passes that do not fit one device pass.

Restates the reference's streaming policy (torch_transformer_benchmark.py:1364-1508)
as pure functions so that the planner and the halve-on-OOM loop can be tested
on the CPU with injected free-memory figures and runners:

* a host-resident input is always streamed (TTB:1427-1428);
* a device input is streamed only when it is at least ``STREAM_MIN_BYTES``
  (TTB:1434-1435), has more than one sequence (TTB:1436-1437) and its live set
  exceeds ``STREAM_SAFETY`` of free memory (TTB:1439);
* the chunk is ``min(batch, free * safety // per_sequence_bytes)``, at least 1
  (TTB:1402-1413);
* a chunk that raises out-of-memory frees the cache, halves the step and is
  retried; at step 1 the error propagates (TTB:1488-1504).

Sequences are independent in every op of the sublayer, so chunking the batch
is exact (TTB:1446-1450).  The live-set model is this build's own: the
library's workspace for one sequence plus the staged input and output.
"""

from __future__ import annotations

from typing import Callable, List, Tuple

STREAM_MIN_BYTES = 1 << 30
STREAM_SAFETY = 0.60


def live_bytes_per_sequence(workspace_per_seq: int, seq_len: int, d_model: int, io_elem: int,
                            resid_out: bool = False) -> int:
    """Device bytes one sequence holds during a pass: workspace + x + y (+ fp32 residual)."""
    b = workspace_per_seq + 2 * seq_len * d_model * io_elem
    if resid_out:
        b += 4 * seq_len * d_model
    return int(b)


def should_stream(x_on_device: bool, x_bytes: int, batch: int, live_bytes_total: int, free_bytes: int,
                  min_bytes: int = STREAM_MIN_BYTES, safety: float = STREAM_SAFETY) -> bool:
    if not x_on_device:
        return True
    if x_bytes < min_bytes:
        return False
    if batch < 2:
        return False
    return live_bytes_total > free_bytes * safety


def plan_chunk(batch: int, per_seq_bytes: int, free_bytes: int, safety: float = STREAM_SAFETY) -> int:
    budget = int(free_bytes * safety)
    return max(1, min(batch, budget // max(1, per_seq_bytes)))


def run_chunked(
    batch: int,
    step: int,
    run_chunk: Callable[[int, int], None],
    on_oom: Callable[[], None],
    is_oom: Callable[[BaseException], bool],
) -> List[Tuple[int, int]]:
    """Walk ``[0, batch)`` in chunks of ``step``; halve ``step`` on OOM.

    Returns the chunks that completed, in order.
    """
    if step < 1:
        raise ValueError("step must be >= 1")
    done: List[Tuple[int, int]] = []
    b0 = 0
    while b0 < batch:
        b1 = min(b0 + step, batch)
        try:
            run_chunk(b0, b1)
        except BaseException as exc:  # noqa: BLE001 - re-raised unless it is an OOM we can absorb
            if not is_oom(exc):
                raise
            on_oom()
            if step == 1:
                raise
            step = max(1, step // 2)
            continue
        done.append((b0, b1))
        b0 = b1
    return done


# ---- host-resident batches: copies overlapped with compute ---------------------------

HOST_MIN_CHUNKS = 4  # a host-resident batch is cut into at least this many chunks when it can be


def host_chunk(batch: int, device_step: int, min_chunks: int = HOST_MIN_CHUNKS) -> int:
    """Chunk size for a host-resident batch: what the device holds, but small enough
    that the copies of one chunk can overlap the compute of its neighbours."""
    return max(1, min(device_step, -(-batch // min_chunks)))


def stream_host(x, mask, outs, step: int, run, dev, is_oom, on_oom) -> None:
    """Run a host-resident batch through the GPU in chunks, filling the host tensors ``outs``.

    ``x``: host [B, ...]; ``mask``: [B, S] (host or device) or None; ``run(xd, md)``
    returns one device tensor per entry of ``outs``.  Two slots of pinned staging and
    device buffers: while chunk i computes on the current stream, a copy stream (default
    priority) brings chunk i+1 in and takes chunk i-1 out, and the host copies between
    pageable and pinned memory run on the CPU in the meantime.  Out of memory: drain,
    halve the chunk, resume at the first chunk whose result was not written.
    """
    import torch

    B = x.shape[0]
    compute = torch.cuda.current_stream(dev)
    copy = torch.cuda.Stream(dev)
    pinned_x = x.is_pinned()
    slots = []

    def new_slot(n):
        s = {"n": n, "pending": None}
        s["pin_in"] = None if pinned_x else torch.empty((n,) + tuple(x.shape[1:]), dtype=x.dtype, pin_memory=True)
        s["dev_in"] = torch.empty((n,) + tuple(x.shape[1:]), dtype=x.dtype, device=dev)
        if mask is not None:
            s["dev_m"] = torch.empty((n,) + tuple(mask.shape[1:]), dtype=mask.dtype, device=dev)
            s["pin_m"] = None if mask.is_cuda else torch.empty((n,) + tuple(mask.shape[1:]), dtype=mask.dtype,
                                                                pin_memory=True)
        s["pin_out"] = [torch.empty((n,) + tuple(o.shape[1:]), dtype=o.dtype, pin_memory=True) for o in outs]
        s["ev_in"] = torch.cuda.Event()
        s["ev_out"] = torch.cuda.Event()
        return s

    def drain(s):
        if s["pending"] is None:
            return
        c0, c1 = s["pending"]
        s["ev_out"].synchronize()
        for o, p in zip(outs, s["pin_out"]):
            o[c0:c1].copy_(p[: c1 - c0])
        s["pending"] = None

    c0 = 0
    while c0 < B:
        if not slots or slots[0]["n"] < step:
            slots = [new_slot(step), new_slot(step)]
            # The slots were allocated on the compute stream (the allocator may hand
            # out blocks that work already queued there still uses), and a device
            # mask may have been produced there just before this call: the copy
            # stream writes the slots and reads the mask only after all of it.
            copy.wait_stream(compute)
        i = 0
        try:
            while c0 < B:
                c1 = min(c0 + step, B)
                n = c1 - c0
                s = slots[i % 2]
                drain(s)  # chunk i-2: its copy-in, compute and copy-out are all done after this
                src = x[c0:c1]
                if not pinned_x:
                    s["pin_in"][:n].copy_(src)
                    src = s["pin_in"][:n]
                with torch.cuda.stream(copy):
                    s["dev_in"][:n].copy_(src, non_blocking=True)
                    if mask is not None:
                        msrc = mask[c0:c1]
                        if s["pin_m"] is not None:
                            s["pin_m"][:n].copy_(msrc)
                            msrc = s["pin_m"][:n]
                        s["dev_m"][:n].copy_(msrc, non_blocking=True)
                    s["ev_in"].record(copy)
                compute.wait_event(s["ev_in"])
                ys = run(s["dev_in"][:n], s["dev_m"][:n] if mask is not None else None)
                done = torch.cuda.Event()
                done.record(compute)
                with torch.cuda.stream(copy):
                    copy.wait_event(done)
                    for y, p in zip(ys, s["pin_out"]):
                        y.record_stream(copy)  # the allocator must not hand y out again before this copy
                        p[:n].copy_(y, non_blocking=True)
                    s["ev_out"].record(copy)
                s["pending"] = (c0, c1)
                i += 1
                c0 = c1
            for k in (i % 2, (i + 1) % 2):  # the older pending chunk first
                drain(slots[k])
        except BaseException as exc:  # noqa: BLE001 - re-raised unless it is an OOM we can absorb
            if not is_oom(exc):
                raise
            # Older chunks still pending are complete once the device is idle: write
            # them out, then retry from the failed chunk (c0), which was not.
            torch.cuda.synchronize(dev)
            for s in slots:
                drain(s)
            slots = []
            on_oom()
            if step == 1:
                raise
            step = max(1, step // 2)
    torch.cuda.current_stream(dev).wait_stream(copy)
