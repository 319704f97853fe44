"""``triangle_multiplicative_update``: the public entry point, with the reference's signature
(geometric_nn_ops_torch/triangle/_trimul.py:39-88 of AMDResearch/geometric-nn-ops).

Where a call goes:
  * a forward that no backward can follow (grad disabled, or nothing requires grad) on a HIP
    tensor of a kernel dtype runs the gfx950 kernels through the ``gnn_amd::trimul_fwd``
    operator;
  * a call that needs gradients, on the same tensors, runs ``_TrimulHip``: the kernels'
    forward, then this library's backward (the reference's own grad calls run autograd
    through its torch code, _trimul.py:31-36);
  * a forward with no backward whose 16-bit widths are above the fused kernels' tiles
    (c_z or c_hidden above 512, both multiples of 32, at most 8192) runs the composed forward
    ``trimul_wide_hip`` (this library's LayerNorm, relayout and contraction kernels with the
    vendor GEMM for the linears);
  * CPU tensors, other dtypes, other channel counts above the kernels' tiles (256 for fp32),
    calls that need gradients with a width above 512 or not a multiple of 32 (the forward
    pads such widths; the backward kernels do not), and a mask that itself requires grad run
    the autograd-differentiable torch restatement in ``_reference.trimul``.
The kernels are never silently replaced: without the HIP library a GPU call raises.

The input projections come stacked: rows ``[0, C_hidden)`` of ``p_in_weight`` and
``g_in_weight`` produce the left operand ``a``, rows ``[C_hidden, 2 C_hidden)`` the right
operand ``b``.
"""

import torch
from torch.autograd.function import once_differentiable

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
    if weights.get("p_in_weight") is not None and not _hip.supports(
            x, weights["p_in_weight"], padded=not _needs_grad(x, weights)):
        # widths above the fused kernels' tiles: the composed HIP forward, without gradients
        return _needs_grad(x, weights) or not _hip.wide_supported(x, weights["p_in_weight"])
    return _needs_grad(x, weights) and mask is not None and mask.requires_grad


class _TrimulHip(torch.autograd.Function):
    """HIP forward whose workspace (the contraction operands a, b and its output o) stays on
    the autograd graph for the HIP backward; the graph owns it, so a backward with
    ``retain_graph=True`` can run again. The output gate gets a buffer of its own, kept for
    the backward where the fused input-side backward covers the widths (its sigmoid
    backward reads the saved gate, as torch's does) and released after the forward
    otherwise (the backward then recomputes it). The backward's kernels
    record no graph of their own, hence ``once_differentiable``: asking for a second
    derivative raises."""

    @staticmethod
    def forward(ctx, x, direction, mask, eps, *ws):
        weights = dict(zip(_hip._WEIGHT_KEYS, ws))
        args, keep, out, workspace, offsets = _hip.build_args(x, direction, mask, eps, weights, separate_gate=True)
        _hip.run_stage("gnn_trimul_fwd", args, x.device)
        gate = keep[-1]  # build_args appends the separate gate buffer last
        del keep
        ctx.direction, ctx.eps, ctx.offsets = direction, eps, offsets
        ctx.workspace = workspace
        # the output gate is kept where the fused input-side backward will read it
        ctx.gate = gate if _hip.proj_bwd_supported(x.dtype, x.shape[-1], weights["p_in_weight"].shape[0] // 2) else None
        ctx.mask = mask
        ctx.save_for_backward(x, *ws)
        return out.reshape(x.shape)

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        x, *ws = ctx.saved_tensors
        weights = dict(zip(_hip._WEIGHT_KEYS, ws))
        dx, dw = _hip.trimul_bwd_hip(x, ctx.direction, ctx.mask, ctx.eps, weights, ctx.workspace,
                                      ctx.offsets, dout, gate=ctx.gate)
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
    """Gated triangle update of a pair tensor: every pixel (i, j) gathers the channel-wise
    products of row i with row j ("outgoing") or of column i with column j ("incoming").

    ``x`` is ``[..., N, N, C_z]`` with any number of leading batch dims; ``mask`` (1 keeps a
    pixel) is ``[..., N, N]`` or broadcasts to it. The LayerNorms take ``norm_in_*`` (size
    C_z) and ``norm_out_*`` (size C_hidden); ``p_in_weight`` / ``g_in_weight`` are the
    stacked ``[2 C_hidden, C_z]`` projections with their optional biases; ``p_out_weight`` is
    ``[C_z, C_hidden]`` and ``g_out_weight`` ``[C_z, C_z]``. ``eps`` goes to both
    LayerNorms. The result has the shape and dtype of ``x``. With fp32 inputs the matrix
    products honour ``torch.backends.cuda.matmul.fp32_precision``.
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
    fwd = _ops.trimul_fwd_impl if _ops.eager_ok(x, mask, *weights.values()) else _ops.trimul_fwd
    return fwd(x, direction, mask, eps=eps, **weights)
