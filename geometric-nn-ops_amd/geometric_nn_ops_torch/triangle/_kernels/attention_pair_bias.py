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
* the gate ``sigmoid(s W_g^T + b_g)``, ``o * g`` and the output projection run in one kernel,
  ``gnn_apb_gate_out`` (32 tokens per workgroup, both products on MFMA, the gated tile
  kept in LDS), so neither ``g`` nor ``o * g`` is written to memory; widths it does not
  cover and calls above ``GATE_OUT_MAX_WORK`` take torch's linear layers.
"""

import ctypes

import torch
import torch.nn.functional as F

from ... import _lib, _precision
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
    _lib.call("gnn_pair_bias_proj", a, z.device)
    return buf[..., :V]


GATE_OUT_MAX_16 = 2048  # c_s + attention width (LDS tiles of 32 tokens)
GATE_OUT_MAX_32 = 1024
# tokens x (c_s + width + c_out) up to which the fused kernel runs. Its four waves share one
# 32-token tile, so the LDS feeds every MFMA and it stays latency-bound; above this the
# vendor GEMMs' larger tiles are faster (measured: 24 us against the torch path's ~60 us
# for 384 tokens of c_s = 384, 81 us against ~30 us for 6144 tokens of 768)
GATE_OUT_MAX_WORK = 1 << 21


def gate_out_supported(s, o, proj_g_weight, proj_o_weight) -> bool:
    """Whether the fused kernel covers ``(o * sigmoid(s W_g^T + b_g)) W_o^T + b_o``. It takes
    one token of s per token of o, so s must not broadcast against o (torch's ``o * g`` would
    accept ``[1, U, Cs]`` against ``[BM, U, D]``); such calls keep the F.linear path."""
    if tuple(s.shape[:-1]) != tuple(o.shape[:-1]):
        return False
    o_width = o.shape[-1]
    cs, co = s.shape[-1], proj_o_weight.shape[0]
    cap = GATE_OUT_MAX_32 if s.dtype == torch.float32 else GATE_OUT_MAX_16
    tokens = s.numel() // max(cs, 1)
    return (s.dtype in (torch.bfloat16, torch.float16, torch.float32) and cs % 32 == 0 and o_width % 32 == 0
            and co % 32 == 0 and tuple(proj_g_weight.shape) == (o_width, cs) and cs + o_width <= cap
            and tokens * (cs + o_width + co) <= GATE_OUT_MAX_WORK)


def gate_out_hip(s, o, proj_g_weight, proj_g_bias, proj_o_weight, proj_o_bias):
    """``(o * sigmoid(s W_g^T + b_g)) W_o^T + b_o`` for ``s [..., Cs]``, ``o [..., D]`` in one
    kernel; returns ``[..., Co]`` in s's dtype."""
    dt = s.dtype
    lead = s.shape[:-1]
    cs, d, co = s.shape[-1], o.shape[-1], proj_o_weight.shape[0]
    s2 = s.reshape(-1, cs)
    if s2.stride(-1) != 1 or (s2.stride(0) * s2.element_size()) % 16 or s2.data_ptr() % 16:
        s2 = s2.contiguous()
    o2 = o.reshape(-1, d).to(dt).contiguous()
    m = s2.shape[0]
    gw = proj_g_weight.to(dt).contiguous()
    ow = proj_o_weight.to(dt).contiguous()
    gb = None if proj_g_bias is None else proj_g_bias.to(dt).contiguous()
    ob = None if proj_o_bias is None else proj_o_bias.to(dt).contiguous()
    out = torch.empty((m, co), device=s.device, dtype=dt)
    a = _lib.ApbGateOutArgs()
    a.s, a.o, a.g_w, a.o_w, a.out = s2.data_ptr(), o2.data_ptr(), gw.data_ptr(), ow.data_ptr(), out.data_ptr()
    a.g_b = None if gb is None else gb.data_ptr()
    a.o_b = None if ob is None else ob.data_ptr()
    a.M, a.Cs, a.D, a.Co = m, cs, d, co
    a.s_ld, a.o_ld, a.out_ld = s2.stride(0), o2.stride(0), out.stride(0)
    a.dtype = _lib.DTYPE_CODE[dt]
    a.precision = _lib.PRECISION_CODE[_precision.matmul_precision(fp32_operands=dt == torch.float32)]
    _lib.call("gnn_apb_gate_out", a, s.device)
    return out.reshape(*lead, co)


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
    if gate_out_supported(s, o, proj_g_weight, proj_o_weight):
        return gate_out_hip(s, o, proj_g_weight, proj_g_bias, proj_o_weight, proj_o_bias), pz
    g = torch.sigmoid(F.linear(s, proj_g_weight, proj_g_bias))
    out = F.linear(o * g, proj_o_weight, proj_o_bias)
    return out, pz
