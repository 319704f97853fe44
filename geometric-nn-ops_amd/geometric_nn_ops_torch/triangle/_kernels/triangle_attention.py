"""Host side of the HIP triangle-attention forward.

``triangle_attention_hip`` takes the canonical 5D layout with a boolean mask and stands
in for the reference's ``triangle_attention_triton`` + ``EvoformerAttention.forward``
(geometric_nn_ops_torch/triangle/_kernels/triangle_attention.py:1447-1484, :1091-1276):
same argument meaning, same shape assertions, ``scale=None`` meaning ``D**-0.5``, and the
masked-key bias rounded to the input dtype. It is forward-only. q/k/v/bias views are
passed to the kernel through their strides (no copies unless a stride or alignment is
unusable), and the output is a fresh contiguous ``[B, N_seq, N_res, H, D]`` tensor.
"""

import ctypes

import torch

from ... import _lib, _precision
from .._masking import rounded_mask_value

MAX_HEAD_DIM = 256  # the kernel's largest head-dim tile (16-bit inputs)
MAX_HEAD_DIM_FP32 = 128  # fp32 tiles take twice the LDS
MAX_N_RES = 32768


def max_head_dim(dtype: torch.dtype) -> int:
    return MAX_HEAD_DIM_FP32 if dtype == torch.float32 else MAX_HEAD_DIM


def supports(q: torch.Tensor) -> bool:
    """Whether the HIP kernel covers this input (dtype handled by the caller)."""
    return q.shape[-1] <= max_head_dim(q.dtype) and q.shape[-3] <= MAX_N_RES


def _vectorizable(t: torch.Tensor) -> bool:
    """Unit stride on the last dim, the other strides multiples of 8 elements, 16-byte base."""
    st = t.stride()
    return t.data_ptr() % 16 == 0 and st[-1] == 1 and all(x % 8 == 0 for x in st[:-1])


def _prepare(t: torch.Tensor) -> torch.Tensor:
    """q/k/v in a form the kernel can address: unit stride on D, other strides multiples
    of 8 elements and a 16-byte aligned base; D padded to a multiple of 8."""
    d = t.shape[-1]
    if d % 8:
        t = torch.nn.functional.pad(t, (0, 8 - d % 8))
    if not _vectorizable(t):
        t = t.contiguous()
        if not _vectorizable(t):
            t = t.clone()
    return t


def _prepare_bias(bias: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``[B, 1, H, N, N]`` bias in ``dtype``. The 16-bit row kernel reads any strides (its
    pre-pass rewrites the bias in fragment order); the tiled kernel needs unit key stride, a
    query pitch that is a multiple of 8 elements and a 16-byte aligned base, so such views
    are copied with the pitch padded (zeros past N)."""
    bias = bias.to(dtype)
    if bias.stride(-1) == 1 and bias.stride(-2) % 8 == 0 and bias.data_ptr() % 16 == 0:
        return bias
    B, _, H, N, _ = bias.shape
    pitch = (N + 7) // 8 * 8
    padded = torch.zeros((B, 1, H, N, pitch), device=bias.device, dtype=bias.dtype)
    padded[..., :N] = bias
    return padded[..., :N]


def _set_bias(args, bias: torch.Tensor) -> None:
    args.bias = bias.data_ptr()
    args.bias_stride = _lib.I64x4(bias.stride(0), bias.stride(2), bias.stride(3), bias.stride(4))


def bias_for_kernel(args, bias: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Points ``args`` (shapes and dtype already set) at the ``[B, 1, H, N, N]`` pair bias in
    ``dtype`` and returns the tensor the kernel will read (the caller keeps it alive). The
    library asks for fragment-order scratch exactly when its row-resident kernel runs, and
    that kernel's pre-pass reads any strides; otherwise the bias is given the unit key stride
    and aligned pitch the tiled kernel needs. Asking the library keeps this decision in one
    place (``triattn_row_applicable`` in the C sources)."""
    bias = bias.to(dtype)
    _set_bias(args, bias)
    if _lib.load().gnn_triattn_workspace_bytes(ctypes.byref(args)) == 0:
        bias = _prepare_bias(bias, dtype)
        _set_bias(args, bias)
    return bias


def workspace_for(args, device) -> torch.Tensor | None:
    """Sets ``args.workspace`` to a fresh scratch tensor of the size the library asks for
    (``None`` when the call needs none); the caller keeps the tensor alive over the launch."""
    nbytes = _lib.load().gnn_triattn_workspace_bytes(ctypes.byref(args))
    if nbytes == 0:
        return None
    ws = torch.empty(nbytes, device=device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
    return ws


def triangle_attention_hip(q, k, v, bias=None, mask=None, scale=None, dynamic=False, use_exp2=False,
                           lse=None, mask_value=None, row_max=None, precision=None):
    """Triangle attention forward on the canonical 5D layout.

    q/k/v ``[B, N_seq, N_res, H, D]`` (bf16, fp16 or fp32, on a HIP device); bias
    ``[B, 1, H, N_res, N_res]`` or ``None``; mask ``[B, N_seq, 1, 1, N_res]`` bool or
    ``None``. ``dynamic`` is accepted for API parity and has no effect (N is always a
    runtime argument); ``use_exp2`` likewise (the kernel always evaluates the softmax in
    base 2). ``lse``, if given, is a float32 ``[B, N_seq, H, N_res]`` tensor that receives
    the natural-log log-sum-exp of each query's logits; ``row_max``, likewise shaped, receives
    each query's largest logit (scaled q.k + bias + mask term). ``mask_value`` overrides the logit
    offset of masked keys (default: the dtype's sentinel rounded to the dtype, as the
    reference launcher applies it).
    """
    del dynamic, use_exp2
    if q.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"triangle_attention_hip: unsupported dtype {q.dtype}")
    dim_q, dim_k, dim_v = q.shape[-1], k.shape[-1], v.shape[-1]
    assert dim_q == dim_k and dim_k == dim_v
    B, S, N, H, D = q.shape
    assert k.shape == q.shape and v.shape == q.shape, f"{tuple(k.shape)} / {tuple(v.shape)} != {tuple(q.shape)}"
    if mask is not None:
        assert mask.shape == (B, S, 1, 1, N), f"{tuple(mask.shape)} != {(B, S, 1, 1, N)}"
    if bias is not None:
        assert bias.shape == (B, 1, H, N, N), f"{tuple(bias.shape)} != {(B, 1, H, N, N)}"
    if scale is None:
        scale = D**-0.5

    qk, kk, vk = _prepare(q), _prepare(k), _prepare(v)
    Dp = qk.shape[-1]
    o = torch.empty((B, S, N, H, Dp), device=q.device, dtype=q.dtype)

    args = _lib.TriAttnArgs()
    args.q, args.k, args.v, args.o = qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), o.data_ptr()
    args.B, args.S, args.N, args.H, args.D = B, S, N, H, Dp
    args.q_stride = _lib.I64x4(*qk.stride()[:4])
    args.k_stride = _lib.I64x4(*kk.stride()[:4])
    args.v_stride = _lib.I64x4(*vk.stride()[:4])
    args.o_stride = _lib.I64x4(*o.stride()[:4])
    args.dtype = _lib.DTYPE_CODE[q.dtype]
    if bias is not None:
        bias = bias_for_kernel(args, bias, q.dtype)
    if mask is not None:
        if mask.dtype != torch.bool:
            raise ValueError(f"mask must be bool (keep=True/mask=False), got {mask.dtype}")
        args.mask = mask.data_ptr()
        args.mask_stride = _lib.I64x3(mask.stride(0), mask.stride(1), mask.stride(4))
    if lse is not None:
        assert lse.shape == (B, S, H, N) and lse.dtype == torch.float32 and lse.is_contiguous()
        args.lse = lse.data_ptr()
    if row_max is not None:
        assert row_max.shape == (B, S, H, N) and row_max.dtype == torch.float32 and row_max.is_contiguous()
        args.row_max = row_max.data_ptr()
    args.scale = float(scale)
    args.mask_value = rounded_mask_value(q.dtype) if mask_value is None else float(mask_value)
    if precision is None:
        precision = _precision.matmul_precision(fp32_operands=q.dtype == torch.float32)
    args.precision = _lib.PRECISION_CODE[precision]

    ws = workspace_for(args, q.device)
    _lib.call("gnn_triattn_fwd", args, q.device)
    del ws
    if Dp != D:
        o = o[..., :D].contiguous()
    return o


def backward_supported(q: torch.Tensor) -> bool:
    """Whether the HIP backward covers these inputs: a head dim that is a multiple of 8, at
    most 128 for bf16 / fp16 and at most 64 for fp32 (whose tiles take twice the LDS)."""
    d = q.shape[-1]
    if d % 8 != 0:
        return False
    if q.dtype in (torch.bfloat16, torch.float16):
        return d <= 128
    return q.dtype == torch.float32 and d <= 64


_CUS = 256  # MI355X compute units; the pair-bias kernel's LDS ring holds one workgroup each
_ROW_S = 1.5e-6  # one N_seq row of a 128 x 128 tile (measured at D = 32)
_PLANE_BPS = 5.0e12  # a partial plane is written once and read once by the ordered reduction


def dbias_splits(B: int, S: int, N: int, H: int) -> int:
    """N_seq ranges for the pair-bias gradient (at most N_seq and 64), minimising a cost
    model: the rounds of (128 x 128 tile, range) workgroups over the compute units times the
    rows per range, plus the fp32 partial plane that each range writes and the ordered
    reduction reads back."""
    tiles = B * H * ((N + 127) // 128) ** 2
    plane = B * H * N * N * 4
    best, best_cost = 1, None
    for s in range(1, min(S, 64) + 1):
        rounds = -(-tiles * s // _CUS)
        cost = rounds * -(-S // s) * _ROW_S + (2 * s * plane / _PLANE_BPS if s > 1 else 0.0)
        if best_cost is None or cost < best_cost:
            best, best_cost = s, cost
    return best


def triangle_attention_bwd_hip(q, k, v, o, dout, lse, bias=None, mask=None, scale=None, mask_value=None,
                               need_dbias=True, precision=None):
    """Gradients of the HIP forward: ``(dq, dk, dv, dbias)`` with dq/dk/dv like q and dbias
    ``[B, 1, H, N, N]`` fp32 (``None`` without a bias or when ``need_dbias`` is false).
    Replaces EvoformerAttention.backward (triangle_attention.py:1278-1442); ``lse`` is the
    forward's ``[B, N_seq, H, N]`` natural-log log-sum-exp. fp32 products run as the
    forward's did: ``precision`` is the resolved ``'ieee'`` or ``'bf16x3'`` (``None``:
    resolved now from ``torch.backends.cuda.matmul.fp32_precision``)."""
    B, S, N, H, D = q.shape
    if scale is None:
        scale = D**-0.5
    qk, kk, vk, ok, dk_ = (_prepare(t) for t in (q, k, v, o, dout.to(q.dtype)))
    assert qk.shape[-1] == D, "the HIP backward needs a head dim that is a multiple of 8"
    dq = torch.empty((B, S, N, H, D), device=q.device, dtype=q.dtype)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    delta = torch.empty((B, S, H, N), device=q.device, dtype=torch.float32)
    a = _lib.TriAttnBwdArgs()
    a.q, a.k, a.v, a.o, a.dout = qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), ok.data_ptr(), dk_.data_ptr()
    a.lse = lse.contiguous().data_ptr()
    a.dq, a.dk, a.dv, a.delta = dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr()
    a.B, a.S, a.N, a.H, a.D = B, S, N, H, D
    a.q_stride = _lib.I64x4(*qk.stride()[:4])
    a.k_stride = _lib.I64x4(*kk.stride()[:4])
    a.v_stride = _lib.I64x4(*vk.stride()[:4])
    a.o_stride = _lib.I64x4(*ok.stride()[:4])
    a.do_stride = _lib.I64x4(*dk_.stride()[:4])
    a.dq_stride = _lib.I64x4(*dq.stride()[:4])
    a.dk_stride = _lib.I64x4(*dk.stride()[:4])
    a.dv_stride = _lib.I64x4(*dv.stride()[:4])
    dbias = None
    if bias is not None:
        bias = _prepare_bias(bias, q.dtype)
        a.bias = bias.data_ptr()
        a.bias_stride = _lib.I64x4(bias.stride(0), bias.stride(2), bias.stride(3), bias.stride(4))
        if need_dbias:
            dbias = torch.empty((B, 1, H, N, N), device=q.device, dtype=torch.float32)
            a.dbias = dbias.data_ptr()
            splits = dbias_splits(B, S, N, H)
            a.dbias_splits = splits
            if splits > 1:
                ws = torch.empty((splits, B, H, N, N), device=q.device, dtype=torch.float32)
                a.dbias_ws = ws.data_ptr()
    if mask is not None:
        a.mask = mask.data_ptr()
        a.mask_stride = _lib.I64x3(mask.stride(0), mask.stride(1), mask.stride(4))
    a.scale = float(scale)
    a.mask_value = rounded_mask_value(q.dtype) if mask_value is None else float(mask_value)
    a.dtype = _lib.DTYPE_CODE[q.dtype]
    if precision is None:
        precision = _precision.matmul_precision(fp32_operands=q.dtype == torch.float32)
    a.precision = _lib.PRECISION_CODE[precision]
    _lib.call("gnn_triattn_bwd", a, q.device)
    return dq, dk, dv, dbias
