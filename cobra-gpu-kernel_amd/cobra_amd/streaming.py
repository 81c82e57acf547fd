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
