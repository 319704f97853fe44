"""The HIP forward kernels registered as torch operators (``torch.ops.gnn_amd.*``).

Each operator calls the C ABI through the host launchers in ``triangle/_kernels`` and has
a shape-only fake implementation, so ``torch.compile`` traces it as one opaque node (no
graph break on the ctypes call) and FakeTensor / meta tracing works without a GPU. The
public ``triangle_attention`` and ``triangle_multiplicative_update`` dispatch their kernel
path through these operators; the differentiable torch path stays outside them (the
operators are forward-only, like the reference's Triton kernels).

Registration follows the boundary the reference's callers bind
(geometric_nn_ops_torch/triangle/_triattn.py:96, _trimul.py:87).

The operator dispatch costs about 10 us of host time per call, so a plain eager call on real
tensors (``eager_ok``) runs the same implementation function directly (``*_impl``); under
torch.compile, FakeTensor or any dispatch mode the callers go through the operator.
"""

from typing import Optional

import torch

__all__ = ["triangle_attention_fwd", "trimul_fwd", "attention_pair_bias_fwd", "eager_ok"]


_PLAIN_TYPES = (torch.Tensor, torch.nn.Parameter)  # Parameter disables __torch_function__


def eager_ok(*tensors) -> bool:
    """True for an eager call whose tensor arguments are plain tensors or module parameters
    (or None) with no tracing or dispatch mode active: the operator's implementation may then
    run directly. Tensor subclasses that override ``__torch_function__`` go through the
    operator."""
    if torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack() > 0:
        return False
    return all(t is None or type(t) in _PLAIN_TYPES for t in tensors)


def triangle_attention_fwd_impl(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    bias: Optional[torch.Tensor],
    mask: Optional[torch.Tensor],
    scale: Optional[float],
) -> torch.Tensor:
    """Canonical 5D ``[B, N_seq, N_res, H, D]`` q / k / v (any strides), bias
    ``[B, 1, H, N, N]``, bool mask ``[B, N_seq, 1, 1, N]``; returns a fresh contiguous
    tensor of q's shape and dtype."""
    from .triangle._kernels.triangle_attention import triangle_attention_hip

    return triangle_attention_hip(q, k, v, bias=bias, mask=mask, scale=scale)


triangle_attention_fwd = torch.library.custom_op("gnn_amd::triangle_attention_fwd", triangle_attention_fwd_impl,
                                                 mutates_args=())


@triangle_attention_fwd.register_fake
def _triangle_attention_fwd_fake(q, k, v, bias, mask, scale):
    return q.new_empty(q.shape)


def trimul_fwd_impl(
    x: torch.Tensor,
    direction: str,
    mask: Optional[torch.Tensor],
    norm_in_weight: Optional[torch.Tensor],
    norm_in_bias: Optional[torch.Tensor],
    p_in_weight: torch.Tensor,
    p_in_bias: Optional[torch.Tensor],
    g_in_weight: torch.Tensor,
    g_in_bias: Optional[torch.Tensor],
    norm_out_weight: Optional[torch.Tensor],
    norm_out_bias: Optional[torch.Tensor],
    p_out_weight: torch.Tensor,
    p_out_bias: Optional[torch.Tensor],
    g_out_weight: torch.Tensor,
    g_out_bias: Optional[torch.Tensor],
    eps: float,
) -> torch.Tensor:
    """``[*, N, N, C_z]`` in, a fresh contiguous tensor of the same shape and dtype out."""
    from .triangle._kernels.trimul import trimul_hip

    return trimul_hip(
        x, direction, mask, eps=eps,
        norm_in_weight=norm_in_weight, norm_in_bias=norm_in_bias,
        p_in_weight=p_in_weight, p_in_bias=p_in_bias,
        g_in_weight=g_in_weight, g_in_bias=g_in_bias,
        norm_out_weight=norm_out_weight, norm_out_bias=norm_out_bias,
        p_out_weight=p_out_weight, p_out_bias=p_out_bias,
        g_out_weight=g_out_weight, g_out_bias=g_out_bias,
    )


trimul_fwd = torch.library.custom_op("gnn_amd::trimul_fwd", trimul_fwd_impl, mutates_args=())


@trimul_fwd.register_fake
def _trimul_fwd_fake(x, direction, mask, *weights_and_eps):
    return x.new_empty(x.shape)


def attention_pair_bias_fwd_impl(
    s: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    z: torch.Tensor,
    proj_g_weight: torch.Tensor,
    proj_o_weight: torch.Tensor,
    proj_z_weight: Optional[torch.Tensor],
    ln_z_weight: Optional[torch.Tensor],
    proj_g_bias: Optional[torch.Tensor],
    proj_o_bias: Optional[torch.Tensor],
    mask: Optional[torch.Tensor],
    scale: Optional[float],
    inf: Optional[float],
    eps: float,
    z_is_projected: bool,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(out [BM, U, D], pz [B, H, U, V])``; with ``z_is_projected`` the second output is an
    empty tensor (the caller already holds the bias)."""
    from .triangle._kernels.attention_pair_bias import attention_pair_bias_hip

    out, pz = attention_pair_bias_hip(
        s, q, k, v, z, proj_g_weight=proj_g_weight, proj_o_weight=proj_o_weight,
        proj_z_weight=proj_z_weight, ln_z_weight=ln_z_weight, proj_g_bias=proj_g_bias,
        proj_o_bias=proj_o_bias, mask=mask, scale=scale, inf=inf, eps=eps,
        z_is_projected=z_is_projected,
    )
    if z_is_projected:
        return out, z.new_empty((0,))
    return out, pz.contiguous()


attention_pair_bias_fwd = torch.library.custom_op("gnn_amd::attention_pair_bias_fwd", attention_pair_bias_fwd_impl,
                                                  mutates_args=())


@attention_pair_bias_fwd.register_fake
def _attention_pair_bias_fwd_fake(s, q, k, v, z, proj_g_weight, proj_o_weight, proj_z_weight, ln_z_weight,
                                  proj_g_bias, proj_o_bias, mask, scale, inf, eps, z_is_projected):
    BM, H, U, _ = q.shape
    out = s.new_empty((BM, U, proj_o_weight.shape[0]))
    if z_is_projected:
        return out, z.new_empty((0,))
    return out, z.new_empty((z.shape[0], H, U, k.shape[2]))
