"""Public ``triangle_multiplicative_update`` (reference geometric_nn_ops_torch/triangle/_trimul.py).

Two backends with the same math:
  * the gfx950 HIP kernels in ``_kernels.trimul``: the forward, and a backward
    (``trimul_bwd_hip``) the reference does not have;
  * the pure-torch, autograd-differentiable path in ``_reference.trimul``.

Dispatch: the reference (_trimul.py:31-36) runs its torch path whenever a backward could
run (grad enabled and x or a weight requires grad). Here such calls run the HIP forward
under ``_TrimulHip``, whose backward is the HIP one, when the inputs are on a HIP device in
a kernel dtype with supported channel counts and the mask does not require grad. The torch
path runs for CPU tensors, other dtypes and channel counts the kernels do not tile (c_z or
c_hidden not a multiple of 32, or above 512). Inference calls run the HIP kernels through
the ``gnn_amd::trimul_fwd`` operator (``geometric_nn_ops_torch._ops``). A missing HIP
library is an error on GPU tensors, never a silent fallback.

``p_in_weight`` / ``g_in_weight`` are the concatenated ``[a; b]`` projections
(``[2 * C_hidden, C_z]``).
"""

import torch

from .. import _ops
from ._kernels import trimul as _hip
from ._reference.trimul import trimul_torch

__all__ = ["triangle_multiplicative_update"]

_KERNEL_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _needs_grad(x: torch.Tensor, weights) -> bool:
    return torch.is_grad_enabled() and (
        x.requires_grad or any(w is not None and w.requires_grad for w in dict(weights).values())
    )


def _needs_torch_path(x: torch.Tensor, weights, mask=None) -> bool:
    weights = dict(weights)
    if not x.is_cuda or x.dtype not in _KERNEL_DTYPES:
        return True
    if weights.get("p_in_weight") is not None and not _hip.supports(x, weights["p_in_weight"]):
        return True
    return _needs_grad(x, weights) and mask is not None and mask.requires_grad


class _TrimulHip(torch.autograd.Function):
    """HIP forward that keeps its workspace (a, b, g, o) for the HIP backward."""

    @staticmethod
    def forward(ctx, x, direction, mask, eps, *ws):
        weights = dict(zip(_hip._WEIGHT_KEYS, ws))
        args, keep, out, workspace, offsets = _hip.build_args(x, direction, mask, eps, weights)
        _hip.run_stage("gnn_trimul_fwd", args, x.device)
        del keep
        ctx.direction, ctx.eps, ctx.offsets = direction, eps, offsets
        ctx.workspace = workspace
        ctx.mask = mask
        ctx.save_for_backward(x, *ws)
        return out.reshape(x.shape)

    @staticmethod
    def backward(ctx, dout):
        x, *ws = ctx.saved_tensors
        weights = dict(zip(_hip._WEIGHT_KEYS, ws))
        dx, dw = _hip.trimul_bwd_hip(x, ctx.direction, ctx.mask, ctx.eps, weights, ctx.workspace,
                                      ctx.offsets, dout)
        ctx.workspace = None
        return (dx, None, None, None, *(dw[k] for k in _hip._WEIGHT_KEYS))


def triangle_multiplicative_update(
    x: torch.Tensor,
    direction: str = "outgoing",
    mask: torch.Tensor | None = None,
    norm_in_weight: torch.Tensor | None = None,
    norm_in_bias: torch.Tensor | None = None,
    p_in_weight: torch.Tensor | None = None,
    p_in_bias: torch.Tensor | None = None,
    g_in_weight: torch.Tensor | None = None,
    g_in_bias: torch.Tensor | None = None,
    norm_out_weight: torch.Tensor | None = None,
    norm_out_bias: torch.Tensor | None = None,
    p_out_weight: torch.Tensor | None = None,
    p_out_bias: torch.Tensor | None = None,
    g_out_weight: torch.Tensor | None = None,
    g_out_bias: torch.Tensor | None = None,
    eps: float = 1e-5,
) -> torch.Tensor:
    """Triangle multiplicative update over a pair representation.

    Args:
        x: ``[*, N, N, C_z]`` pair representation.
        direction: ``"outgoing"`` or ``"incoming"``.
        mask: optional ``[*, N, N]`` pair mask (1 = keep), broadcastable over the leading dims.
        *_weight / *_bias: LayerNorm / projection / gate parameters.
        eps: LayerNorm epsilon.

    Returns:
        ``[*, N, N, C_z]`` updated pair representation.

    fp32 products follow ``torch.backends.cuda.matmul.fp32_precision``.
    """
    weights = dict(
        norm_in_weight=norm_in_weight,
        norm_in_bias=norm_in_bias,
        p_in_weight=p_in_weight,
        p_in_bias=p_in_bias,
        g_in_weight=g_in_weight,
        g_in_bias=g_in_bias,
        norm_out_weight=norm_out_weight,
        norm_out_bias=norm_out_bias,
        p_out_weight=p_out_weight,
        p_out_bias=p_out_bias,
        g_out_weight=g_out_weight,
        g_out_bias=g_out_bias,
    )
    if _needs_torch_path(x, weights.items(), mask):
        return trimul_torch(x, direction, mask, eps=eps, **weights)
    if _needs_grad(x, weights.items()):
        return _TrimulHip.apply(x, direction, mask, eps, *(weights[k] for k in _hip._WEIGHT_KEYS))
    return _ops.trimul_fwd(x, direction, mask, eps=eps, **weights)
