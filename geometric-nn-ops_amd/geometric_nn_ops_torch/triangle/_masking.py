"""Turning a boolean key mask into an additive bias on the softmax logits.

Same sentinel values and spelling as the reference (geometric_nn_ops_torch/triangle/
_masking.py:13-42): kept keys get exactly +0.0 and masked keys -mask_val(dtype).
"""

import functools

import torch


def mask_val(dtype: torch.dtype) -> float:
    """How far a masked key's logit is pushed below zero, for ``dtype``.

    ``1e9`` for fp32 and bf16; half the fp16 maximum for fp16 (``1e9`` overflows to inf
    there); ``1e18`` for fp64, whose ulp at 1e9 would leave a fully masked row's logits
    distinct where fp32's collapse them.
    """
    if dtype == torch.float64:
        return 1e18
    elif dtype == torch.float32 or dtype == torch.bfloat16:
        return 1e9
    elif dtype == torch.float16:
        return torch.finfo(dtype).max / 2
    else:
        raise ValueError(f"Unsupported dtype {dtype}")


def masked_key_bias(mask: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Boolean mask -> additive bias, ``0`` where kept and ``-mask_val`` where not.

    Written as ``mask_val * (mask - 1)`` so kept entries are +0.0 rather than -0.0, which
    is observable after rounding to bf16/fp16.
    """
    return mask_val(dtype) * (mask.to(torch.float32) - 1)


@functools.lru_cache(maxsize=None)
def rounded_mask_value(dtype: torch.dtype) -> float:
    """The masked-key bias after the cast to the compute dtype, as the Triton launcher
    applies it (triangle_attention.py:1470: ``masked_key_bias(mask, q.dtype).to(q.dtype)``).
    One value per dtype, computed once (it is on every call's path)."""
    sentinel = torch.tensor(-mask_val(dtype), dtype=torch.float32)
    return float(sentinel.to(dtype).to(torch.float32))
