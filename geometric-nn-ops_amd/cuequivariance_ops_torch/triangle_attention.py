"""cueq's ``triangle_attention`` on the HIP kernel (reference shim triangle_attention.py:1-52).

cueq lays q / k / v out as ``(B, N, H, S, D)``; the public op takes ``(B, N, S, H, D)``, so the
head and sequence axes are swapped as strided views (the kernel reads them without copies)
and the output is swapped back. bias ``(B, 1, H, S, S)`` and mask ``(B, N, 1, 1, S)`` are
layout-compatible. The result is always rank 5, as cueq returns it.
"""

import torch

from geometric_nn_ops_torch.triangle import triangle_attention as _triangle_attention

# cueq's documented threshold below which it would use a torch fallback; the HIP kernel
# serves short sequences too, so a low value is advertised (it is not consulted).
CUEQ_TRIATTN_FALLBACK_THRESHOLD = 16


def triangle_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bias: torch.Tensor,
                       mask: torch.Tensor | None = None, scale: float | None = None,
                       return_aux: bool = False):
    if return_aux:
        raise NotImplementedError(
            "cuequivariance_ops_torch shim: triangle_attention(return_aux=True) is not supported")
    swap = lambda t: t.transpose(-2, -3)  # noqa: E731
    out = swap(_triangle_attention(swap(q), swap(k), swap(v), bias,
                                   None if mask is None else mask.bool(), scale))
    if out.dim() < 5:
        out = out.reshape((1,) * (5 - out.dim()) + tuple(out.shape))
    return out
