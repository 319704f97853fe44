"""cueq's ``triangle_multiplicative_update`` on the HIP kernels (reference shim
triangle_multiplicative_update.py:1-110).

The kernels take fp32 product precision from ``torch.backends.cuda.matmul.fp32_precision``;
cueq's ``precision`` argument can therefore only be checked against it. Asking for a mode
other than torch's when torch is at ``ieee`` only costs speed (warning); asking for one
other than torch's when torch allows reduced precision could break the caller's accuracy
requirement (ValueError). ``None``, ``"none"`` and ``"default"`` request nothing.
"""

import enum
import warnings

from geometric_nn_ops_torch import _precision
from geometric_nn_ops_torch.triangle import triangle_multiplicative_update as _trimul

from ._trimul_precision import TriMulPrecision

# cueq's documented fallback threshold (advertised, not consulted).
CUEQ_TRIMUL_FALLBACK_THRESHOLD = 16

_NO_PREFERENCE = {"none", "default"}


def _normalise(precision):
    if isinstance(precision, int) and not isinstance(precision, enum.Enum):
        precision = TriMulPrecision(precision)
    if isinstance(precision, enum.Enum):
        precision = precision.name
    return precision.lower() if isinstance(precision, str) else precision


def check_precision(precision) -> None:
    if precision is None:
        return
    wanted = _normalise(precision)
    if wanted in _NO_PREFERENCE:
        return
    current = _precision.torch_precision()
    if wanted == current:
        return
    msg = (f"triangle_multiplicative_update precision={precision!r} requested while "
           f"torch.backends.cuda.matmul.fp32_precision is {current!r}; the kernels follow the torch "
           "setting, so set that instead")
    if current == _precision.IEEE:
        warnings.warn(msg + " (running in full fp32)", stacklevel=3)
    else:
        raise ValueError(msg)


def triangle_multiplicative_update(x, direction="outgoing", mask=None, norm_in_weight=None, norm_in_bias=None,
                                   p_in_weight=None, p_in_bias=None, g_in_weight=None, g_in_bias=None,
                                   norm_out_weight=None, norm_out_bias=None, p_out_weight=None, p_out_bias=None,
                                   g_out_weight=None, g_out_bias=None, eps=1e-5, precision=None):
    check_precision(precision)
    return _trimul(x, direction=direction, mask=mask, norm_in_weight=norm_in_weight, norm_in_bias=norm_in_bias,
                   p_in_weight=p_in_weight, p_in_bias=p_in_bias, g_in_weight=g_in_weight, g_in_bias=g_in_bias,
                   norm_out_weight=norm_out_weight, norm_out_bias=norm_out_bias, p_out_weight=p_out_weight,
                   p_out_bias=p_out_bias, g_out_weight=g_out_weight, g_out_bias=g_out_bias, eps=eps)
