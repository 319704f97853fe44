"""Differentiable triangle attention in stock torch, canonical 5D layout.

Same math as the reference's triangle_attention_torch
(geometric_nn_ops_torch/triangle/_reference/triangle_attention.py:11-44): scaled q.k
logits in fp32 (fp64 for fp64 inputs), plus the pair bias and the masked-key bias, a
softmax over keys and the weighted sum of v. It materialises the full
[B, N_seq, H, N_res, N_res] logits, so it is meant for small inputs and for gradients.
"""

import torch

from .._masking import masked_key_bias


def triangle_attention_torch(q, k, v, bias=None, mask=None, scale=None):
    """q, k, v ``[B, N_seq, N_res, H, D]``; bias broadcastable to ``[B, 1, H, N, N]``
    (or ``[B, H, N, N]``); boolean mask broadcastable to ``[B, N_seq, 1, 1, N]``."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    acc = torch.float64 if q.dtype == torch.float64 else torch.float32
    logits = torch.einsum("bsihd,bsjhd->bshij", q.to(acc) * scale, k.to(acc))
    if bias is not None:
        if bias.dim() == 4:
            bias = bias.unsqueeze(-4)
        logits = logits + bias.to(acc)
    if mask is not None:
        logits = logits + masked_key_bias(mask, acc).to(acc)
    probs = torch.softmax(logits, dim=-1)
    o = torch.einsum("bshij,bsjhd->bsihd", probs, v.to(acc))
    return o.to(q.dtype)
