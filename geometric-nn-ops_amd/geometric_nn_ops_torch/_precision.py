"""torch's fp32 matmul precision setting, resolved to what the HIP kernels implement.

Mirrors geometric_nn_ops_torch/_precision.py:26-83 of the reference. ``fp32_precision``
selects ``"ieee"`` or ``"tf32"``; gfx950 has no xf32, so ``"tf32"`` resolves along the
chain ``tf32 -> bf16x3 -> ieee`` to the first mode the target allows. The HIP library
implements ``ieee`` (fp32 MFMA) and ``bf16x3`` (three bf16 MFMAs per fp32 product), the
same set Triton reports for gfx950 minus ``bf16x6``, so ``"tf32"`` becomes ``"bf16x3"``.
"""

import torch

IEEE = "ieee"
TF32 = "tf32"

# Modes for each setting, fastest first; every chain ends at "ieee"
# (reference _precision.py:36-39).
_MODES = {
    TF32: ("tf32", "bf16x3", "ieee"),
    IEEE: ("ieee",),
}

# What libgnn_hip.so's kernels implement for fp32 operands on gfx950.
HIP_ALLOWED = ("ieee", "bf16x3")


def torch_precision() -> str:
    """torch's current fp32 matmul precision (reference _precision.py:44-54)."""
    if hasattr(torch.backends.cuda.matmul, "fp32_precision"):
        return TF32 if torch.backends.cuda.matmul.fp32_precision == TF32 else IEEE
    return TF32 if torch.backends.cuda.matmul.allow_tf32 else IEEE


def resolve(precision: str, allowed: tuple[str, ...]) -> str:
    """Dot mode for ``precision`` on a target supporting ``allowed``
    (reference _precision.py:57-70)."""
    if precision not in _MODES:
        raise ValueError(f"unknown precision {precision!r}, expected one of {tuple(_MODES)}")
    for mode in _MODES[precision]:
        if mode in allowed:
            return mode
    raise RuntimeError(f"target supports none of {_MODES[precision]}; it allows only {allowed}")


def _allowed_dot_precisions() -> tuple[str, ...]:
    """fp32 dot modes of the HIP kernels (fixed for gfx950; the reference asks Triton,
    _precision.py:73-81)."""
    return HIP_ALLOWED


def matmul_precision(*, fp32_operands: bool) -> str:
    """Mode for the kernels' fp32 products; non-fp32 operands are pinned to ieee, since
    bf16/fp16 always use their native MFMA (reference _precision.py:84-93)."""
    if not fp32_operands:
        return IEEE
    return resolve(torch_precision(), _allowed_dot_precisions())
