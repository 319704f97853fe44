"""Triangle (protein-folding) ops (reference geometric_nn_ops_torch/triangle/__init__.py:6-14).

``attention_pair_bias`` is not provided by this build: it is outside the HIP hot path.
"""

from ._triattn import triangle_attention
from ._trimul import triangle_multiplicative_update

__all__ = [
    "triangle_attention",
    "triangle_multiplicative_update",
]
