"""epure (MI355X build) -- the fused codebook dequant-matmul behind every
packed linear, on hand-written gfx950 HIP kernels.

Public names follow the reference package (epure/__init__.py:31-37) for the
parts this build covers: the packed store, linear and embedding, the fine-tuning
helpers, and the ``epure.kernels`` backend contract.
"""
from . import container
from .finetune import (
    ScaleTuner,
    make_trainable,
    packed_weights,
    snapshot_indices,
    trainable_forward,
    verify_frozen,
)
from .runtime import (
    ExpertHolder,
    PackedEmbedding,
    PackedExperts,
    PackedLinear,
    PackedWeight,
    apply_packed,
    tie_packed_lm_head,
)

__version__ = "0.2.4+mi355x"

__all__ = [
    "PackedWeight", "PackedLinear", "PackedEmbedding", "PackedExperts", "ExpertHolder",
    "apply_packed", "tie_packed_lm_head",
    "make_trainable", "packed_weights", "snapshot_indices", "verify_frozen",
    "trainable_forward", "ScaleTuner", "container",
    "__version__",
]
