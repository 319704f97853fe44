"""Differentiable triangle multiplicative update in stock torch.

Same math as the reference's trimul_torch
(geometric_nn_ops_torch/triangle/_reference/trimul.py:57-97): LayerNorm, gated
projection, mask, the outgoing/incoming contraction, output LayerNorm, projection and
gate. The contraction is written as one einsum per direction.
"""

import torch
import torch.nn.functional as F

DIRECTIONS = ("outgoing", "incoming")

# o[..., i, j, c] for a, b of shape [..., N, N, Ch]
_CONTRACTION = {
    True: "...ikc,...jkc->...ijc",   # outgoing: sum over the shared second index
    False: "...kic,...kjc->...ijc",  # incoming: sum over the shared first index
}


def is_outgoing(direction: str) -> bool:
    """Validate ``direction`` (reference _reference/trimul.py:30-34)."""
    if direction not in DIRECTIONS:
        raise ValueError(f"direction must be one of {DIRECTIONS}, got {direction!r}")
    return direction == "outgoing"


def combine_projections(a: torch.Tensor, b: torch.Tensor, outgoing: bool) -> torch.Tensor:
    """The triangle contraction of ``a`` and ``b`` ([..., N, N, Ch]) for one direction."""
    return torch.einsum(_CONTRACTION[outgoing], a, b)


def trimul_torch(
    x,
    direction="outgoing",
    mask=None,
    *,
    eps=1e-5,
    norm_in_weight=None,
    norm_in_bias=None,
    p_in_weight=None,
    p_in_bias=None,
    g_in_weight=None,
    g_in_bias=None,
    norm_out_weight=None,
    norm_out_bias=None,
    p_out_weight=None,
    p_out_bias=None,
    g_out_weight=None,
    g_out_bias=None,
):
    """Triangle multiplicative update on ``x`` ``[*, N, N, C_z]`` with ``mask`` ``[*, N, N]``.

    ``p_in_weight`` / ``g_in_weight`` are the concatenated ``[a; b]`` projections
    (``[2 * C_hidden, C_z]``).
    """
    outgoing = is_outgoing(direction)
    c_hidden = p_in_weight.shape[0] // 2
    z = F.layer_norm(x, (x.shape[-1],), norm_in_weight, norm_in_bias, eps)
    gate_in = torch.sigmoid(F.linear(z, g_in_weight, g_in_bias))
    p = F.linear(z, p_in_weight, p_in_bias) * gate_in
    if mask is not None:
        p = p * mask.unsqueeze(-1)
    o = combine_projections(p[..., :c_hidden], p[..., c_hidden:], outgoing)
    o = F.layer_norm(o, (c_hidden,), norm_out_weight, norm_out_bias, eps)
    gate_out = torch.sigmoid(F.linear(z, g_out_weight, g_out_bias))
    return F.linear(o, p_out_weight, p_out_bias) * gate_out
