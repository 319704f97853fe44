"""Triangle (protein-folding) ops (reference geometric_nn_ops_torch/triangle/__init__.py:6-14)."""

from ._attention_pair_bias import attention_pair_bias
from ._triattn import triangle_attention
from ._trimul import triangle_multiplicative_update

__all__ = [
    "attention_pair_bias",
    "triangle_attention",
    "triangle_multiplicative_update",
]
