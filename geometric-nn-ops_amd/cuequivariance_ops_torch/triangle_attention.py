"""cueq's ``triangle_attention`` on the HIP kernel (reference shim triangle_attention.py:1-52).

cueq lays q / k / v out as ``(B, N, H, S, D)``; the public op takes ``(B, N, S, H, D)``, so the
head and sequence axes are swapped as strided views (the kernel reads them without copies)
and the output is swapped back. bias ``(B, 1, H, S, S)`` and mask ``(B, N, 1, 1, S)`` are
layout-compatible. The result is always rank 5, as cueq returns it.

``return_aux=True`` also returns cueq's auxiliary tensors, ``(out, lse, max)``: the natural-log
log-sum-exp and the maximum of each query's logits (scaled q.k + bias + masked-key term), fp32,
shaped ``(B, N, H, S, 1)``. The reference's shim refuses them because its Triton kernel does
not expose them (hipequivariance_ops_torch/cuequivariance_ops_torch/triangle_attention.py:34-38);
the HIP forward writes both in the same call that writes the output. Calls that need a
gradient, or that the kernel does not cover, run the public op and compute the two tensors
apart.
"""

import torch

from geometric_nn_ops_torch.triangle import triangle_attention as _triangle_attention

# cueq's documented threshold below which it would use a torch fallback; the HIP kernel
# serves short sequences too, so a low value is advertised (it is not consulted).
CUEQ_TRIATTN_FALLBACK_THRESHOLD = 16


def _rank5(t):
    return t if t is None or t.dim() >= 5 else t.reshape((1,) * (5 - t.dim()) + tuple(t.shape))


def _canonical_bias_mask(q, bias, mask):
    B, Nseq, S, H, _ = q.shape
    if bias is not None:
        if bias.dim() == 4:
            bias = bias.unsqueeze(-4)
        elif bias.dim() > 5:
            bias = bias.reshape(-1, *bias.shape[-4:])
        bias = bias.broadcast_to(B, 1, H, S, S)
    if mask is not None:
        if mask.dim() > 5:
            mask = mask.reshape(-1, *mask.shape[-4:])
        mask = mask.broadcast_to(B, Nseq, 1, 1, S)
    return bias, mask


def _one_call(q, k, v, bias) -> bool:
    """Whether one HIP forward can write o, lse and max: a forward-only rank-5 call on a HIP
    device in a kernel dtype and shape."""
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as hip

    needs_grad = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, k, v, bias))
    return (q.dim() == 5 and q.is_cuda and not needs_grad and q.dtype in (torch.bfloat16, torch.float16, torch.float32)
            and k.dtype == q.dtype and v.dtype == q.dtype and hip.supports(q))


def _aux(q, k, v, bias, mask, scale):
    """(lse, max) ``[B, N, H, S]`` of the logits, for canonical ``[B, N, S, H, D]`` q / k / v."""
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as hip
    from geometric_nn_ops_torch.triangle._masking import masked_key_bias

    B, Nseq, S, H, D = q.shape
    bias, mask = _canonical_bias_mask(q, bias, mask)
    if q.is_cuda and q.dtype in (torch.bfloat16, torch.float16, torch.float32) and hip.supports(q):
        lse = torch.empty((B, Nseq, H, S), device=q.device, dtype=torch.float32)
        mx = torch.empty_like(lse)
        with torch.no_grad():
            hip.triangle_attention_hip(q.detach(), k.detach(), v.detach(), None if bias is None else bias.detach(),
                                       mask, scale, lse=lse, row_max=mx)
        return lse, mx
    # other tensors: the logits in fp32 (fp64 stays fp64), as the torch path computes them
    ct = torch.float64 if q.dtype == torch.float64 else torch.float32
    scale = D ** -0.5 if scale is None else scale
    with torch.no_grad():
        logits = (q.to(ct).transpose(-2, -3) * scale) @ k.to(ct).transpose(-2, -3).transpose(-1, -2)
        if bias is not None:
            logits = logits + bias.to(ct)
        if mask is not None:
            logits = logits + masked_key_bias(mask, q.dtype).to(ct)
        return torch.logsumexp(logits, -1).float(), logits.amax(-1).float()


def triangle_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bias: torch.Tensor,
                       mask: torch.Tensor | None = None, scale: float | None = None,
                       return_aux: bool = False):
    swap = lambda t: t.transpose(-2, -3)  # noqa: E731
    mask = None if mask is None else mask.bool()
    if not return_aux:
        return _rank5(swap(_triangle_attention(swap(q), swap(k), swap(v), bias, mask, scale)))
    q5, k5, v5 = (_rank5(swap(t)) for t in (q, k, v))
    bias5 = None if bias is None else (bias if bias.dim() >= 4 else _rank5(bias))
    mask5 = None if mask is None else _rank5(mask)
    if _one_call(q5, k5, v5, bias5):
        from geometric_nn_ops_torch.triangle._kernels import triangle_attention as hip

        B, Nseq, S, H, _ = q5.shape
        bias5, mask5 = _canonical_bias_mask(q5, bias5, mask5)
        lse = torch.empty((B, Nseq, H, S), device=q.device, dtype=torch.float32)
        mx = torch.empty_like(lse)
        with torch.no_grad():
            out = hip.triangle_attention_hip(q5, k5, v5, bias5, mask5, scale, lse=lse, row_max=mx)
        return swap(out), lse.unsqueeze(-1), mx.unsqueeze(-1)
    out = _rank5(swap(_triangle_attention(swap(q), swap(k), swap(v), bias, mask, scale)))
    lse, mx = _aux(q5, k5, v5, bias5, mask5, scale)
    return out, lse.unsqueeze(-1), mx.unsqueeze(-1)
