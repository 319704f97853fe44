"""Public ``attention_pair_bias`` with the reference's signature
(geometric_nn_ops_torch/triangle/_attention_pair_bias.py:11-98).

Takes pre-projected q / k / v; does the pair-rep LayerNorm + projection to a per-head bias,
the masked attention, the gate from the single rep and the output projection.

Dispatch: forward-only calls on a HIP device run the gfx950 kernels (the pair-bias
projection and the triangle-attention kernel, through the ``gnn_amd::attention_pair_bias_fwd``
operator) when the queries and keys cover the same tokens (U == V) and the head dim fits
the attention kernel; calls that need a backward, CPU tensors, fp64 and other shapes take
the differentiable torch path. The reference runs the torch math for every call. Masks are
applied as keep where nonzero (the reference's ``(mask - 1) * inf`` for 0 / 1 masks).
"""

import torch

from .. import _ops
from ._kernels import triangle_attention as _hip_attn
from ._reference.attention_pair_bias import attention_pair_bias_torch

_KERNEL_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _needs_torch_path(s, q, k, v, z, weights, z_is_projected) -> bool:
    if not (q.is_cuda and k.is_cuda and v.is_cuda and z.is_cuda and s.is_cuda):
        return True
    if q.dtype not in _KERNEL_DTYPES or q.dtype != k.dtype or q.dtype != v.dtype or z.dtype != q.dtype:
        return True
    if q.shape[2] != k.shape[2] or q.shape[-1] > _hip_attn.max_head_dim(q.dtype):
        return True
    if not z_is_projected and weights[0] is None:
        return True
    return torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (s, q, k, v, z, *weights)
    )


def attention_pair_bias(
    s: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    z: torch.Tensor,
    *,
    proj_g_weight: torch.Tensor,
    proj_o_weight: torch.Tensor,
    proj_z_weight: torch.Tensor | None = None,
    ln_z_weight: torch.Tensor | None = None,
    proj_g_bias: torch.Tensor | None = None,
    proj_o_bias: torch.Tensor | None = None,
    mask: torch.Tensor | None = None,
    scale: float | None = None,
    inf: float | None = None,
    eps: float = 1e-5,
    z_is_projected: bool = False,
    return_z_proj: bool = False,
):
    """Attention with pair bias.

    Args:
        s: ``(BM, S, D)`` single representation; the gate is projected from it and the
            output has its shape.
        q: ``(BM, H, U, DH)`` pre-projected queries; k, v: ``(BM, H, V, DH)``.
        z: pair representation ``(B, U, V, Zc)``, or the projected bias ``(B, H, U, V)``
            when ``z_is_projected``.
        proj_g_weight, proj_o_weight: ``(D, D)`` gate and output projections.
        proj_z_weight: ``(H, Zc)`` pair-bias projection (required unless ``z_is_projected``).
        ln_z_weight: ``(Zc,)`` LayerNorm weight of ``z`` (the LayerNorm has no bias).
        proj_g_bias, proj_o_bias: optional ``(D,)`` biases.
        mask: ``(B, V)`` or ``(BM, V)``, 1 = keep, 0 = mask.
        scale: attention scale, ``None`` -> ``DH ** -0.5``.
        inf: how far masked logits are pushed down; ``None`` -> the logits dtype's sentinel.
        eps: LayerNorm epsilon.
        z_is_projected: ``z`` is a cached ``(B, H, U, V)`` bias.
        return_z_proj: also return the ``(B, H, U, V)`` bias (unmasked) for reuse.

    Returns:
        ``(out, proj_z)``: ``out`` ``(BM, S, D)``; ``proj_z`` the bias when
        ``return_z_proj``, else ``None``.
    """
    BM = q.shape[0]
    B = z.shape[0]
    if BM % B != 0:
        raise ValueError(f"q batch {BM} is not a multiple of z batch {B}")
    if mask is not None and mask.shape[0] not in (B, BM):
        raise ValueError(f"mask batch {mask.shape[0]} must be B={B} or BM={BM}")
    weights = (proj_z_weight, ln_z_weight, proj_g_weight, proj_o_weight, proj_g_bias, proj_o_bias)
    if _needs_torch_path(s, q, k, v, z, weights, z_is_projected):
        return attention_pair_bias_torch(
            s, q, k, v, z, proj_g_weight=proj_g_weight, proj_o_weight=proj_o_weight,
            proj_z_weight=proj_z_weight, ln_z_weight=ln_z_weight, proj_g_bias=proj_g_bias,
            proj_o_bias=proj_o_bias, mask=mask, scale=scale, inf=inf, eps=eps,
            z_is_projected=z_is_projected, return_z_proj=return_z_proj,
        )
    fwd = _ops.attention_pair_bias_fwd_impl if _ops.eager_ok(s, q, k, v, z, mask, *weights) else \
        _ops.attention_pair_bias_fwd
    out, pz = fwd(
        s, q, k, v, z, proj_g_weight, proj_o_weight, proj_z_weight, ln_z_weight, proj_g_bias,
        proj_o_bias, mask, scale, inf, eps, z_is_projected,
    )
    if not return_z_proj:
        return out, None
    return out, (z if z_is_projected else pz)
