"""cobra_amd -- MI355X (gfx950) attention-sublayer forward.

A drop-in for the attention half of the COBRA benchmark's transformer block:
``CobraAttentionSublayer`` (module) over ``ops`` (tensor wrappers of the C ABI)
over ``libcobra_amd.so`` (hand-written HIP kernels, ``include/cobra_amd.h``).
"""

from . import ops, streaming  # noqa: F401
from ._lib import CobraError, LIB_PATH  # noqa: F401
from .layer import CobraAttentionSublayer, CobraSelfAttention  # noqa: F401

__all__ = ["CobraAttentionSublayer", "CobraSelfAttention", "CobraError", "ops", "streaming", "LIB_PATH"]
