"""CPU restatement of the reference attention sublayer -- TEST INFRASTRUCTURE ONLY.

This package is the checker for the HIP product path, never part of it.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package (``cobra_amd``) must not, and a
test asserts that it does not.

Contents and the reference code each part follows (paths relative to the
reference checkout; ``TTB`` = ``torch_transformer_benchmark.py``):

* ``layer``   -- ``OracleSelfAttention`` / ``OracleAttentionSublayer``: the
  attention half of ``BaselineTransformerBlock`` (TTB:60-123, 129-142), fp32,
  unfused, same op order; plus the query-blocked variant of
  ``tools/reference_chunked.py:73-128`` for sequences whose [S, S] score matrix
  cannot be materialised.
* ``gate``    -- ``compare_outputs`` (TTB:1616-1697): per element
  ``finite and (abs <= atol or abs <= rtol*|ref|)``.
* ``model``   -- ``OracleTransformerConfig`` / ``OracleTransformerBlock`` /
  ``OracleTransformer``: the whole stack (TTB:28-57, 126-173) -- attention
  half, exact-GELU FFN half, block and output row masks, ``final_norm``.
* ``cases``   -- seeded construction (TTB:2024-2031), input generation
  (TTB:1575-1593 semantics on a CPU generator) and the configuration matrix of
  the benchmark (tools/sweep.py:31-47, attention sublayer only).

Parity status: every function here is pinned by CPU tests in
``tests/test_oracle.py`` against closed forms, invariants and an independent
library routine (``torch.nn.functional.multi_head_attention_forward``); see the
docstring of each test for which mistake it would catch.  The reference ships
no golden vectors for this path.
"""

from .cases import (  # noqa: F401
    CONFIGS,
    LayerCase,
    make_input,
    make_sequence,
    make_sublayer,
    quantize_like,
)
from .gate import AccuracyResult, compare_outputs  # noqa: F401
from .layer import OracleAttentionSublayer, OracleSelfAttention  # noqa: F401
from .model import (  # noqa: F401
    OracleTransformer,
    OracleTransformerBlock,
    OracleTransformerConfig,
    make_model,
    model_forward,
)
