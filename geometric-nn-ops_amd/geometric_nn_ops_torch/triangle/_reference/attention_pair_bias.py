"""Differentiable attention with pair bias in stock torch.

The semantics of the reference's attention_pair_bias_torch
(geometric_nn_ops_torch/triangle/_reference/attention_pair_bias.py:17-89): the pair rep is
LayerNorm-ed (no beta) and projected to one bias per head, the M copies of a batch element
(folded into q/k/v's batch) share that bias, masked keys are pushed down by ``inf`` (by
default the logits dtype's sentinel), and the attention output, gated by
``sigmoid(s W_g^T + b_g)``, goes through the output projection. Used for calls that need
a backward, CPU tensors and shapes outside the HIP kernels.
"""

import torch
import torch.nn.functional as F

from .._masking import mask_val


def project_pair_bias(z, ln_z_weight, proj_z_weight, eps=1e-5):
    """``[B, U, V, Zc]`` -> ``[B, H, U, V]``."""
    zn = F.layer_norm(z, (z.shape[-1],), ln_z_weight, None, eps)
    return F.linear(zn, proj_z_weight).permute(0, 3, 1, 2).contiguous()


def attention_pair_bias_torch(s, q, k, v, z, *, proj_g_weight, proj_o_weight, proj_z_weight=None,
                              ln_z_weight=None, proj_g_bias=None, proj_o_bias=None, mask=None,
                              scale=None, inf=None, eps=1e-5, z_is_projected=False,
                              return_z_proj=False):
    BM, H, U, DH = q.shape
    V = k.shape[2]
    B = z.shape[0]
    if BM % B != 0:
        raise ValueError(f"q batch {BM} is not a multiple of z batch {B}")
    M = BM // B
    scale = DH ** -0.5 if scale is None else scale
    pz = z if z_is_projected else project_pair_bias(z, ln_z_weight, proj_z_weight, eps)

    def split(t, n):  # [B*M, H, n, DH] -> [B, M, H, n, DH]
        return t.reshape(B, M, H, n, DH)

    logits = torch.matmul(split(q, U), split(k, V).transpose(-1, -2)) * scale + pz.unsqueeze(1)
    if mask is not None:
        if mask.shape[0] == B:
            keep = mask.reshape(B, 1, 1, 1, V)
        elif mask.shape[0] == BM:
            keep = mask.reshape(B, M, 1, 1, V)
        else:
            raise ValueError(f"mask batch {mask.shape[0]} must be B={B} or BM={BM}")
        magnitude = mask_val(logits.dtype) if inf is None else inf
        logits = logits + (keep.to(logits.dtype) - 1.0) * magnitude
    o = torch.matmul(torch.softmax(logits, dim=-1), split(v, V))  # [B, M, H, U, DH]
    o = o.reshape(BM, H, U, DH).transpose(1, 2).reshape(BM, U, H * DH).to(s.dtype)
    g = torch.sigmoid(F.linear(s, proj_g_weight, proj_g_bias))
    out = F.linear(o * g, proj_o_weight, proj_o_bias)
    return out, (pz if return_z_proj else None)
