"""Host side of the HIP triangle multiplicative update forward.

``trimul_hip`` takes the same arguments as the reference's ``trimul_triton``
(geometric_nn_ops_torch/triangle/_kernels/trimul.py:404-448) and runs the whole op as
three HIP kernels through ``gnn_trimul_fwd``: LN-in + gated projections, the per-channel
N x N x N contraction, and LN-out + p_out + gate. Forward only. The intermediates live in
one workspace tensor allocated here through torch's caching allocator.
"""

import ctypes
import math

import torch

from ... import _lib, _precision
from .._reference.trimul import is_outgoing

_WEIGHT_KEYS = (
    "norm_in_weight", "norm_in_bias", "p_in_weight", "p_in_bias", "g_in_weight", "g_in_bias",
    "norm_out_weight", "norm_out_bias", "p_out_weight", "p_out_bias", "g_out_weight", "g_out_bias",
)
_ARG_FIELD = {
    "norm_in_weight": "ln_in_w", "norm_in_bias": "ln_in_b",
    "p_in_weight": "p_in_w", "p_in_bias": "p_in_b",
    "g_in_weight": "g_in_w", "g_in_bias": "g_in_b",
    "norm_out_weight": "ln_out_w", "norm_out_bias": "ln_out_b",
    "p_out_weight": "p_out_w", "p_out_bias": "p_out_b",
    "g_out_weight": "g_out_w", "g_out_bias": "g_out_b",
}
MAX_CHANNELS = 512


def supports(x: torch.Tensor, p_in_weight: torch.Tensor) -> bool:
    """Whether the HIP kernels cover these channel counts (multiples of 32, at most 512)."""
    c_z, c_hidden = x.shape[-1], p_in_weight.shape[0] // 2
    return (c_z % 32 == 0 and c_hidden % 32 == 0 and c_z <= MAX_CHANNELS
            and c_hidden <= MAX_CHANNELS and x.dim() >= 3)


def _expect(name, t, shape):
    if t is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def _aligned(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def build_args(x, direction, mask, eps, weights):
    """Validated, kernel-ready tensors and the filled ``gnn_trimul_args``.

    Returns (args, keepalive, out, workspace, offsets)."""
    outgoing = is_outgoing(direction)
    if x.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"trimul_hip: unsupported dtype {x.dtype}")
    N, N2, C = x.shape[-3], x.shape[-2], x.shape[-1]
    if N != N2:
        raise ValueError(f"x must be [*, N, N, C_z], got {tuple(x.shape)}")
    for key in ("p_in_weight", "g_in_weight", "p_out_weight", "g_out_weight"):
        if weights.get(key) is None:
            raise ValueError(f"{key} is required")
    Ch = weights["p_in_weight"].shape[0] // 2
    expected = {
        "p_in_weight": (2 * Ch, C), "g_in_weight": (2 * Ch, C), "p_out_weight": (C, Ch),
        "g_out_weight": (C, C), "norm_in_weight": (C,), "norm_in_bias": (C,),
        "norm_out_weight": (Ch,), "norm_out_bias": (Ch,), "p_in_bias": (2 * Ch,),
        "g_in_bias": (2 * Ch,), "p_out_bias": (C,), "g_out_bias": (C,),
    }
    for key, shape in expected.items():
        _expect(key, weights.get(key), shape)
    lead = x.shape[:-3]
    B = math.prod(lead)

    xk = _aligned(x.reshape(B, N, N, C))
    out = torch.empty((B, N, N, C), device=x.device, dtype=x.dtype)
    keep = [xk]

    args = _lib.TrimulArgs()
    args.x, args.out = xk.data_ptr(), out.data_ptr()
    if mask is not None:
        m = mask.to(device=x.device, dtype=x.dtype).expand(*x.shape[:-1]).reshape(B, N, N)
        keep.append(m)
        args.mask = m.data_ptr()
        args.mask_stride = _lib.I64x3(*m.stride())
    for key in _WEIGHT_KEYS:
        w = weights.get(key)
        if w is None:
            continue
        w = _aligned(w.to(device=x.device, dtype=x.dtype))
        keep.append(w)
        setattr(args, _ARG_FIELD[key], w.data_ptr())
    dtype = _lib.DTYPE_CODE[x.dtype]
    offsets = (ctypes.c_size_t * 4)()
    lib = _lib.load()
    nbytes = lib.gnn_trimul_workspace_bytes(B, N, C, Ch, dtype, offsets)
    workspace = torch.empty(nbytes, device=x.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = workspace.data_ptr(), nbytes
    args.B, args.N, args.C, args.Ch = B, N, C, Ch
    args.eps = float(eps)
    args.outgoing = 1 if outgoing else 0
    args.dtype = dtype
    precision = _precision.matmul_precision(fp32_operands=x.dtype == torch.float32)
    args.precision = _lib.PRECISION_CODE[precision]
    return args, keep, out, workspace, tuple(offsets)


def run_stage(fn_name: str, args, device) -> None:
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = getattr(lib, fn_name)(ctypes.byref(args), ctypes.c_void_p(_lib.stream_handle(device)))
    _lib.check(rc, fn_name)


def trimul_hip(
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
    """Triangle multiplicative update on the HIP kernels. Forward only.

    ``x`` ``[*, N, N, C_z]`` (bf16, fp16 or fp32 on a HIP device), ``mask`` ``[*, N, N]``
    (broadcastable; 1 = keep) or ``None``; weights as in the torch path.
    """
    weights = dict(
        norm_in_weight=norm_in_weight, norm_in_bias=norm_in_bias,
        p_in_weight=p_in_weight, p_in_bias=p_in_bias,
        g_in_weight=g_in_weight, g_in_bias=g_in_bias,
        norm_out_weight=norm_out_weight, norm_out_bias=norm_out_bias,
        p_out_weight=p_out_weight, p_out_bias=p_out_bias,
        g_out_weight=g_out_weight, g_out_bias=g_out_bias,
    )
    args, keep, out, workspace, _ = build_args(x, direction, mask, eps, weights)
    run_stage("gnn_trimul_fwd", args, x.device)
    del keep, workspace
    return out.reshape(x.shape)
