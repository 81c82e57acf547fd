"""cobra_amd -- MI355X (gfx950) transformer forward for the COBRA benchmark.

Drop-ins for the benchmark's modules: ``CobraAttentionSublayer`` (the
attention half of a block, one fused kernel for small shapes) and
``CobraTransformer`` (the whole ``BaselineTransformer`` / ``UserOptimizedTransformer``
stack), over ``ops`` (tensor wrappers of the C ABI) over ``libcobra_amd.so``
(hand-written HIP kernels, ``include/cobra_amd.h``).
"""

from . import ops, streaming  # noqa: F401
from ._lib import CobraError, LIB_PATH  # noqa: F401
from .layer import CobraAttentionSublayer, CobraSelfAttention  # noqa: F401
from .model import CobraTransformer, CobraTransformerBlock, TransformerConfig  # noqa: F401

__all__ = ["CobraAttentionSublayer", "CobraSelfAttention", "CobraTransformer", "CobraTransformerBlock",
           "TransformerConfig", "CobraError", "ops", "streaming", "LIB_PATH"]
