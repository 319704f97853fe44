"""The ``cuequivariance_ops_torch`` API served by this build's HIP kernels.

Mirrors the reference's optional shim (hipequivariance_ops_torch/cuequivariance_ops_torch/
__init__.py:1-40): with this package on the path, ``cuequivariance_torch.primitives.triangle``
(which imports ``cuequivariance_ops_torch``) runs on the gfx950 kernels with no source change.
The module-level names cueq deep-imports are provided too:
``triangle_attention.CUEQ_TRIATTN_FALLBACK_THRESHOLD``,
``triangle_multiplicative_update.CUEQ_TRIMUL_FALLBACK_THRESHOLD`` and
``attention_pair_bias_torch.CUEQ_ATTENTION_PAIR_BIAS_FALLBACK_THRESHOLD``.
"""

from . import _guard

_guard.check()

# ruff: noqa: E402  (the imports below run after the installation check)
from ._trimul_precision import TriMulPrecision
from .attention_pair_bias_torch import attention_pair_bias
from .triangle_attention import triangle_attention
from .triangle_multiplicative_update import triangle_multiplicative_update

__all__ = ["attention_pair_bias", "triangle_attention", "triangle_multiplicative_update", "TriMulPrecision"]
