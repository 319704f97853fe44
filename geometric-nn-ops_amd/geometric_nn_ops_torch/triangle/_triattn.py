"""Public ``triangle_attention`` with the reference's cueq-compatible signature.

Shape and dtype normalisation follow geometric_nn_ops_torch/triangle/_triattn.py:23-106:
4D inputs gain a batch axis, >5D inputs fold their leading dims, a 4D bias gains the
N_seq axis, bias and mask are broadcast to ``[B, 1, H, N, N]`` / ``[B, N_seq, 1, 1, N]``,
fp64 is computed in fp32, and the output has the input's shape and dtype.

Dispatch: the gfx950 HIP kernel serves every forward-only call on a HIP device, through
the ``gnn_amd::triangle_attention_fwd`` operator (``geometric_nn_ops_torch._ops``).
Calls that need a backward run the HIP forward (saving the log-sum-exp) and the HIP
backward kernels (dq, dk, dv and the N_seq-summed pair-bias gradient) for a head dim that is
a multiple of 8 (at most 128 for bf16 / fp16, 64 for fp32, whose products follow the fp32
precision setting resolved at the forward, 'ieee' or 'bf16x3'), as the reference runs its
Triton forward and backward; other grad-requiring calls, CPU tensors and head dims above the
forward kernel's tile take the differentiable torch path. There is no fallback when the HIP library is
missing: a GPU call then raises.
"""

import torch
from torch.autograd.function import once_differentiable

from .. import _ops, _precision
from ._kernels import triangle_attention as _hip
from ._reference.triangle_attention import triangle_attention_torch

_KERNEL_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _needs_grad(q, k, v, bias) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, k, v, bias))


def _needs_torch_path(q, k, v, bias) -> bool:
    if not q.is_cuda or not _hip.supports(q):
        return True
    return _needs_grad(q, k, v, bias)


class _TriangleAttentionHip(torch.autograd.Function):
    """HIP forward that keeps the log-sum-exp, HIP backward (reference
    EvoformerAttention, triangle_attention.py:1091-1442). The backward kernels record no
    graph, so it is ``once_differentiable``: a second derivative raises instead of coming
    back wrong."""

    @staticmethod
    def forward(ctx, q, k, v, bias, mask, scale):
        B, S, N, H, _ = q.shape
        lse = torch.empty((B, S, H, N), device=q.device, dtype=torch.float32)
        # fp32: the backward runs with the precision the forward resolved
        precision = _precision.matmul_precision(fp32_operands=q.dtype == torch.float32)
        o = _hip.triangle_attention_hip(q, k, v, bias=bias, mask=mask, scale=scale, lse=lse, precision=precision)
        ctx.save_for_backward(q, k, v, bias, mask, o, lse)
        ctx.scale = scale
        ctx.precision = precision
        ctx.bias_grad = bias is not None and bias.requires_grad
        return o

    @staticmethod
    @once_differentiable
    def backward(ctx, do):
        q, k, v, bias, mask, o, lse = ctx.saved_tensors
        dq, dk, dv, dbias = _hip.triangle_attention_bwd_hip(q, k, v, o, do, lse, bias=bias, mask=mask,
                                                            scale=ctx.scale, need_dbias=ctx.bias_grad,
                                                            precision=ctx.precision)
        if dbias is not None:
            dbias = dbias.to(bias.dtype)
        return dq, dk, dv, dbias, None, None


def triangle_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    bias: torch.Tensor | None = None,
    mask: torch.Tensor | None = None,
    scale: float | None = None,
    dynamic: bool = False,
    use_exp2: bool = False,
) -> torch.Tensor:
    """Triangle attention with a cueq-compatible signature.

    Args:
        q, k, v: ``[..., N_seq, N_res, H, D]``; 4D, 5D or 6D (leading dims fold into batch).
        bias: pair bias broadcastable to ``[B, 1, H, N_res, N_res]`` (a ``[B, H, N, N]``
            bias gains the N_seq axis), or ``None``.
        mask: boolean, ``True`` keeps a key; broadcastable to ``[B, N_seq, 1, 1, N_res]``,
            or ``None`` for all-keep.
        scale: softmax scale; ``None`` means ``1/sqrt(D)``.
        dynamic: accepted for API compatibility; the HIP kernel takes every size at run
            time, so both values give bit-identical results.
        use_exp2: accepted for API compatibility; the HIP kernel always evaluates the
            softmax in base 2 with log2(e) folded into its inputs.

    Returns:
        Tensor of the same shape and dtype as ``q``.

    fp32 products follow ``torch.backends.cuda.matmul.fp32_precision``.
    """
    if mask is not None and mask.dtype != torch.bool:
        raise ValueError(f"mask must be bool (keep=True/mask=False), got {mask.dtype}")

    orig_shape = q.shape
    orig_dtype = q.dtype

    if q.dim() < 5:
        lead = (1,) * (5 - q.dim())
        q, k, v = (t.reshape(lead + tuple(t.shape)) for t in (q, k, v))
    elif q.dim() > 5:
        q, k, v = (t.reshape(-1, *t.shape[-4:]) for t in (q, k, v))

    batch, n_seq, n_res, heads, _ = q.shape

    if bias is not None:
        if bias.dim() == 4:
            bias = bias.unsqueeze(-4)
        elif bias.dim() > 5:
            bias = bias.reshape(-1, *bias.shape[-4:])
        bias = bias.broadcast_to(batch, 1, heads, n_res, n_res)
    if mask is not None:
        if mask.dim() > 5:
            mask = mask.reshape(-1, *mask.shape[-4:])
        mask = mask.broadcast_to(batch, n_seq, 1, 1, n_res)

    if q.is_cuda and _needs_grad(q, k, v, bias) and _hip.backward_supported(q) and (
            k.dtype == q.dtype and v.dtype == q.dtype):
        o = _TriangleAttentionHip.apply(q, k, v, bias, mask, scale)
        return o.reshape(orig_shape)
    if _needs_torch_path(q, k, v, bias):
        o = triangle_attention_torch(q, k, v, bias=bias, mask=mask, scale=scale)
        return o.to(orig_dtype).reshape(orig_shape)

    compute_dtype = orig_dtype if orig_dtype in _KERNEL_DTYPES else torch.float32
    fwd = _ops.triangle_attention_fwd_impl if _ops.eager_ok(q, k, v, bias, mask) else _ops.triangle_attention_fwd
    o = fwd(
        q.to(compute_dtype),
        k.to(compute_dtype),
        v.to(compute_dtype),
        None if bias is None else bias.to(compute_dtype),
        mask,
        scale,
    )
    return o.to(orig_dtype).reshape(orig_shape)
