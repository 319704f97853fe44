"""Host side of the HIP attention with pair bias (forward).

Stands in for the reference's attention_pair_bias_torch
(geometric_nn_ops_torch/triangle/_reference/attention_pair_bias.py:25-89), which the
reference runs as stock torch ops. Here:

* the pair rep ``z [B, U, V, Zc]`` goes through ``gnn_pair_bias_proj`` (LayerNorm + head
  projection in one pass, written straight into ``[B, H, U, V]`` with a row pitch the
  attention kernel can read);
* the attention runs on ``gnn_triattn_fwd``: q ``[B*M, H, U, DH]`` is the canonical
  ``[B, N_seq=M, N_res=U, H, DH]`` by a permutation of strides (no copy), the bias is
  shared by the M rows exactly as the reference broadcasts ``pz[:, None]``, the key mask
  ``[B, V]`` / ``[B*M, V]`` becomes a ``[B, M, 1, 1, V]`` view, and the kernel's fresh
  ``[B, M, U, H, DH]`` output already is the merged-heads ``[B*M, U, H*DH]`` layout;
* the gate ``sigmoid(s W_g^T + b_g)`` and the output projection are library GEMMs.
"""

import ctypes

import torch
import torch.nn.functional as F

from ... import _lib
from .._masking import mask_val
from .triangle_attention import triangle_attention_hip

MAX_ZC = 256
MAX_HEADS_X_ZC = 8192


def projection_supported(z: torch.Tensor, heads: int) -> bool:
    zc = z.shape[-1]
    return zc % 8 == 0 and zc <= MAX_ZC and heads * zc <= MAX_HEADS_X_ZC


def pair_bias_projection_hip(z, ln_z_weight, proj_z_weight, eps=1e-5):
    """``z [B, U, V, Zc]`` -> ``[B, H, U, V]`` in z's dtype. The result is a view with a
    row pitch rounded up to 8 elements (what the attention kernel reads without a copy)."""
    lib = _lib.load()
    B, U, V, Zc = z.shape
    H = proj_z_weight.shape[0]
    z = z.contiguous()
    w = proj_z_weight.to(z.dtype).contiguous()
    gamma = None if ln_z_weight is None else ln_z_weight.to(z.dtype).contiguous()
    pitch = (V + 7) // 8 * 8
    buf = (torch.empty if pitch == V else torch.zeros)((B, H, U, pitch), device=z.device, dtype=z.dtype)
    a = _lib.PairBiasArgs()
    a.z, a.proj_w, a.out = z.data_ptr(), w.data_ptr(), buf.data_ptr()
    a.ln_w = None if gamma is None else gamma.data_ptr()
    a.B, a.U, a.V, a.Zc, a.H = B, U, V, Zc, H
    a.out_stride = _lib.I64x3(buf.stride(0), buf.stride(1), buf.stride(2))
    a.eps = float(eps)
    a.dtype = _lib.DTYPE_CODE[z.dtype]
    with torch.cuda.device(z.device):
        rc = lib.gnn_pair_bias_proj(ctypes.byref(a), ctypes.c_void_p(_lib.stream_handle(z.device)))
    _lib.check(rc, "gnn_pair_bias_proj")
    return buf[..., :V]


def attention_pair_bias_hip(s, q, k, v, z, *, proj_g_weight, proj_o_weight, proj_z_weight=None,
                            ln_z_weight=None, proj_g_bias=None, proj_o_bias=None, mask=None,
                            scale=None, inf=None, eps=1e-5, z_is_projected=False):
    """Forward of attention with pair bias on the HIP kernels; returns ``(out, pz)`` with
    ``pz`` the ``[B, H, U, V]`` bias (the input itself when ``z_is_projected``)."""
    BM, H, U, DH = q.shape
    V = k.shape[2]
    B = z.shape[0]
    M = BM // B
    if z_is_projected:
        pz = z
    elif projection_supported(z, H):
        pz = pair_bias_projection_hip(z, ln_z_weight, proj_z_weight, eps)
    else:
        zc = F.layer_norm(z, (z.shape[-1],), ln_z_weight, None, eps)
        pz = F.linear(zc, proj_z_weight, None).permute(0, 3, 1, 2)

    def canon(t, n):  # [B*M, H, n, DH] -> [B, M, n, H, DH] view
        return t.reshape(B, M, H, n, DH).permute(0, 1, 3, 2, 4)

    keep = None
    mask_value = None
    if mask is not None:
        mb = mask.shape[0]
        if mb == B:
            keep = (mask != 0).reshape(B, 1, 1, 1, V).expand(B, M, 1, 1, V)
        else:
            keep = (mask != 0).reshape(B, M, 1, 1, V)
        logits_dtype = torch.promote_types(q.dtype, pz.dtype)
        magnitude = mask_val(logits_dtype) if inf is None else float(inf)
        # the reference adds (keep - 1) * inf in the logits' dtype
        mask_value = float(torch.tensor(-magnitude, dtype=torch.float64).to(logits_dtype).to(torch.float32))
    o = triangle_attention_hip(canon(q, U), canon(k, V), canon(v, V), bias=pz.unsqueeze(1), mask=keep,
                               scale=scale, mask_value=mask_value)
    o = o.reshape(BM, U, H * DH).to(s.dtype)
    g = torch.sigmoid(F.linear(s, proj_g_weight, proj_g_bias))
    out = F.linear(o * g, proj_o_weight, proj_o_bias)
    return out, pz
