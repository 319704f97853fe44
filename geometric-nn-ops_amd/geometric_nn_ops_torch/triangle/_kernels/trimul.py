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
WIDE_MAX_CHANNELS = 8192  # the wide-row LayerNorm's limit (gnn_layernorm_rows forward)


def _pad32(n: int) -> int:
    return (n + 31) // 32 * 32


def supports(x: torch.Tensor, p_in_weight: torch.Tensor, *, padded: bool = True) -> bool:
    """Whether the HIP kernels cover these channel counts: at most 512 once rounded up to a
    multiple of 32 (256 for fp32). Widths that are not multiples of 32 run the forward on
    zero-padded copies (``padded``); the HIP backward takes multiples of 32 only."""
    c_z, c_hidden = x.shape[-1], p_in_weight.shape[0] // 2
    if c_z < 1 or c_hidden < 1 or x.dim() < 3:
        return False
    if not padded and (c_z % 32 or c_hidden % 32):
        return False
    limit = 256 if x.dtype == torch.float32 else MAX_CHANNELS
    return _pad32(c_z) <= limit and _pad32(c_hidden) <= limit


def wide_supported(x: torch.Tensor, p_in_weight: torch.Tensor) -> bool:
    """Whether ``trimul_wide_hip`` covers these widths: 16-bit inputs whose c_z or c_hidden
    is above the fused kernels' 512, both multiples of 32 and at most 8192."""
    C, Ch = x.shape[-1], p_in_weight.shape[0] // 2
    return (x.dtype in (torch.bfloat16, torch.float16) and x.dim() >= 3 and C % 32 == 0 and Ch % 32 == 0
            and max(C, Ch) > MAX_CHANNELS and max(C, Ch) <= WIDE_MAX_CHANNELS)


def _pad_channels(x, weights):
    """x and the weights zero-padded to channel counts that are multiples of 32, for the
    forward kernels, with the real widths the LayerNorms average over. The a / b halves of
    the stacked input projections are padded separately (rows [0, Ch) and [Ch', Ch' + Ch)),
    so padded hidden channels give a = b = 0, o = 0, and padded input channels meet zero
    weight columns; the padded output channels are sliced off by the caller.

    Returns (x', weights', C', Ch')."""
    C = x.shape[-1]
    Ch = weights["p_in_weight"].shape[0] // 2
    Cp, Chp = _pad32(C), _pad32(Ch)

    def pad(t, shape, blocks):
        """t copied into zeros of ``shape``; blocks: per dim, the offsets of its parts."""
        out = t.new_zeros(shape)
        if t.dim() == 1:
            for o, (lo, hi) in zip(blocks[0], _parts(t.shape[0], len(blocks[0]))):
                out[o:o + hi - lo] = t[lo:hi]
        else:
            for o, (lo, hi) in zip(blocks[0], _parts(t.shape[0], len(blocks[0]))):
                out[o:o + hi - lo, :t.shape[1]] = t[lo:hi]
        return out

    xp = torch.nn.functional.pad(x, (0, Cp - C))
    w = dict(weights)
    stacked = {"p_in_weight": (2 * Chp, Cp), "g_in_weight": (2 * Chp, Cp), "p_in_bias": (2 * Chp,),
               "g_in_bias": (2 * Chp,)}
    plain = {"p_out_weight": (Cp, Chp), "g_out_weight": (Cp, Cp), "p_out_bias": (Cp,), "g_out_bias": (Cp,),
             "norm_in_weight": (Cp,), "norm_in_bias": (Cp,), "norm_out_weight": (Chp,), "norm_out_bias": (Chp,)}
    for key, shape in stacked.items():
        if w.get(key) is not None:
            w[key] = pad(w[key], shape, [(0, Chp)])
    for key, shape in plain.items():
        if w.get(key) is not None:
            w[key] = pad(w[key], shape, [(0,)])
    return xp, w, Cp, Chp


def _parts(n, k):
    """k equal consecutive parts of range(n)."""
    step = n // k
    return [(i * step, (i + 1) * step) for i in range(k)]


def _expect(name, t, shape):
    if t is not None and t.shape != shape:
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def _aligned(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _kernel_ready(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """``t`` on ``like``'s device and dtype, contiguous and 16-byte aligned (as is, when it
    already is: the usual case for parameters, and the checks are cheaper than the copies)."""
    if t.dtype == like.dtype and t.device == like.device and t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t
    return _aligned(t.to(device=like.device, dtype=like.dtype))


def build_args(x, direction, mask, eps, weights, separate_gate=False):
    """Validated, kernel-ready tensors and the filled ``gnn_trimul_args``. With
    ``separate_gate`` the output gate gets a buffer of its own (in the keepalive list) and the
    workspace holds only a, b and o, which is what a backward needs.

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
        w = _kernel_ready(w, x)
        keep.append(w)
        setattr(args, _ARG_FIELD[key], w.data_ptr())
    dtype = _lib.DTYPE_CODE[x.dtype]
    offsets = (ctypes.c_size_t * 4)()
    lib = _lib.load()
    nbytes = lib.gnn_trimul_workspace_bytes(B, N, C, Ch, dtype, offsets)
    if separate_gate:  # the gate region is the workspace's last: stop before it
        nbytes = offsets[2]
        gate = torch.empty((B, N, N, C), device=x.device, dtype=x.dtype)
        keep.append(gate)
        args.gate = gate.data_ptr()
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
    _lib.call(fn_name, args, device)


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
    C, Ch = x.shape[-1], p_in_weight.shape[0] // 2
    if wide_supported(x, p_in_weight):  # widths above the fused kernels' tiles
        return trimul_wide_hip(x, direction, mask, eps, weights)
    if C % 32 or Ch % 32:  # zero-padded copies; the LayerNorms average over the real widths
        xp, wp, _, _ = _pad_channels(x, weights)
        args, keep, out, workspace, _ = build_args(xp, direction, mask, eps, wp)
        args.ln_in_channels, args.ln_out_channels = C, Ch
        run_stage("gnn_trimul_fwd", args, x.device)
        del keep, workspace
        return out[..., :C].reshape(x.shape)
    args, keep, out, workspace, _ = build_args(x, direction, mask, eps, weights)
    run_stage("gnn_trimul_fwd", args, x.device)
    del keep, workspace
    return out.reshape(x.shape)


def trimul_wide_hip(x, direction, mask, eps, weights):
    """The forward for 16-bit widths above the fused kernels' 512 (``wide_supported``), on
    this library's kernels where the math is not a plain matrix product: LN_in and LN_out on
    ``gnn_layernorm_rows`` (its wide-row kernel), the contraction on ``gnn_trimul_contract``
    (stage 2 takes any width), a / b moved into the contraction's per-channel planes and o out
    of them by ``gnn_trimul_relayout``; the three input projections as one ``[4 Ch + C, C]``
    linear and p_out on the vendor GEMM; the sigmoid gates and the mask in torch, in the
    reference's order and roundings (``_reference/trimul.py:57-97``). The pair grid is taken
    to NP = round_up(N, 32) with the pixels past N masked out (a = b = 0 there), so that the
    relayout's row blocks are the contraction's; the output is cut back to N."""
    outgoing = is_outgoing(direction)
    lead, N, C = x.shape[:-3], x.shape[-3], x.shape[-1]
    Ch = weights["p_in_weight"].shape[0] // 2
    B, NP = math.prod(lead), _pad32(N)
    dev, dt = x.device, x.dtype
    w = {k: (None if v is None else _kernel_ready(v, x)) for k, v in weights.items()}
    xb = x.reshape(B, N, N, C)
    m = (torch.ones((B, N, N), device=dev, dtype=dt) if mask is None
         else mask.to(device=dev, dtype=dt).expand(*x.shape[:-1]).reshape(B, N, N))
    if NP != N:
        xb = torch.nn.functional.pad(xb, (0, 0, 0, NP - N, 0, NP - N))
        m = torch.nn.functional.pad(m, (0, NP - N, 0, NP - N))
    M = B * NP * NP
    z = layernorm_rows_hip(_aligned(xb.reshape(M, C)), w.get("norm_in_weight"), w.get("norm_in_bias"), eps)

    def bias(key, n):
        return torch.zeros(n, device=dev, dtype=dt) if w.get(key) is None else w[key]

    lin = torch.nn.functional.linear(
        z, torch.cat([w["p_in_weight"], w["g_in_weight"], w["g_out_weight"]], 0),
        torch.cat([bias("p_in_bias", 2 * Ch), bias("g_in_bias", 2 * Ch), bias("g_out_bias", C)]))
    del z
    p = lin[:, :2 * Ch] * torch.sigmoid(lin[:, 2 * Ch:4 * Ch])
    p = _aligned(p * m.reshape(M, 1))
    gate_out = torch.sigmoid(lin[:, 4 * Ch:])
    del lin
    # a and b into the contraction's k-blocked planes (outgoing: plane row i, column k;
    # incoming: transposed per channel), then the contraction at NP. The stage-2 call reads
    # only the workspace's a / b and writes its o (x, out, the weights and the gate buffer it
    # is given are checked, not read), so the workspace stops before the gate region.
    dtc = _lib.DTYPE_CODE[dt]
    off = (ctypes.c_size_t * 4)()
    _lib.load().gnn_trimul_workspace_bytes(B, NP, C, Ch, dtc, off)
    workspace = torch.empty(off[2], device=dev, dtype=torch.uint8)
    args = _lib.TrimulArgs()
    any_ptr = w["p_in_weight"].data_ptr()
    args.x = args.out = args.gate = any_ptr
    args.p_in_w, args.g_in_w = w["p_in_weight"].data_ptr(), w["g_in_weight"].data_ptr()
    args.p_out_w, args.g_out_w = w["p_out_weight"].data_ptr(), w["g_out_weight"].data_ptr()
    args.workspace, args.workspace_bytes = workspace.data_ptr(), off[2]
    args.B, args.N, args.C, args.Ch = B, NP, C, Ch
    args.eps, args.outgoing, args.dtype = float(eps), int(outgoing), dtc
    args.precision = _lib.PRECISION_CODE["ieee"]
    for i, c0 in ((0, 0), (1, Ch)):
        relayout_hip(p, workspace[off[i]:], _lib.RELAYOUT_PIXELS_TO_BLOCKED, B, NP, Ch, src_ld=2 * Ch,
                     dst_ld=32, src_c0=c0, transposed=outgoing)
    del p
    run_stage("gnn_trimul_contract", args, dev)
    o = torch.empty((M, Ch), device=dev, dtype=dt)
    o_planes = workspace[off[3]:off[3] + B * Ch * NP * NP * o.element_size()].view(dt)
    relayout_hip(o_planes, o, _lib.RELAYOUT_PLANES_TO_PIXELS, B, NP, Ch, src_ld=NP, dst_ld=Ch)
    del workspace
    on = layernorm_rows_hip(o, w.get("norm_out_weight"), w.get("norm_out_bias"), eps)
    del o
    out = torch.nn.functional.linear(on, w["p_out_weight"], w.get("p_out_bias")) * gate_out
    out = out.view(B, NP, NP, C)
    if NP != N:
        out = out[:, :N, :N]
    return out.reshape(*lead, N, N, C)


# ------------------------------------------------------------------------------ backward
# The reference has no native trimul backward: with gradients it runs trimul_torch under
# autograd (geometric_nn_ops_torch/triangle/_trimul.py:31-36; math in
# triangle/_reference/trimul.py:57-97). trimul_bwd_hip differentiates the same math. The
# LayerNorms (forward recompute and backward, with deterministic per-workgroup weight-gradient
# partials) and the two sigmoid gates run on this library's kernels (gnn_layernorm_rows,
# gnn_trimul_gate_bwd), and for 16-bit types so do the contraction's two N^3 products per
# channel (gnn_trimul_contract_bwd, reading a and b in place in the forward's workspace) and
# the moves between pixel-major tensors and per-channel planes (gnn_trimul_relayout). The
# other matrix products (the three input projections as one [4 Ch + C, C] linear, p_out, the
# weight gradients, and fp32's contraction products) go to the vendor GEMM through torch.
# a, b and o come from the forward's workspace.

def layernorm_rows_hip(x2d, weight=None, bias=None, eps=1e-5, *, dy=None, partials=False):
    """Row LayerNorm of ``x2d`` ``[R, K]`` (columns contiguous): ``LN(x)`` when ``dy`` is
    None, else ``dx`` and, with ``partials``, ``(dweight, dbias)`` in fp32 summed over the
    kernel's per-workgroup partial rows."""
    lib = _lib.load()
    R, K = x2d.shape
    out = torch.empty((R, K), device=x2d.device, dtype=x2d.dtype)
    a = _lib.LayerNormArgs()
    a.x, a.out = x2d.data_ptr(), out.data_ptr()
    a.weight = None if weight is None else weight.data_ptr()
    a.rows, a.K = R, K
    a.x_stride, a.out_stride = x2d.stride(0), out.stride(0)
    a.eps, a.dtype = float(eps), _lib.DTYPE_CODE[x2d.dtype]
    part = None
    if dy is None:
        a.bias = None if bias is None else bias.data_ptr()
    else:
        a.dy, a.dy_stride = dy.data_ptr(), dy.stride(0)
        if partials:
            part = torch.empty((lib.gnn_layernorm_partials(R, K), 2, K), device=x2d.device,
                               dtype=torch.float32)
            a.partial = part.data_ptr()
    _lib.call("gnn_layernorm_rows", a, x2d.device)
    if part is None:
        return out
    sums = part.sum(0)
    return out, sums[0], sums[1]


def gate_bwd_hip(grad, value, gate_pre, mask_rows=None, *, d_value=None, d_gate_pre=None, sums=False,
                 gate_is_sigmoid=False):
    """Backward of ``value * sigmoid(gate_pre) * mask_rows[:, None]`` for ``[R, K]`` row
    views (columns contiguous); writes into ``d_value`` / ``d_gate_pre`` (allocated when
    None) and returns them, followed with ``sums`` by their fp32 column sums (the bias
    gradients of the layers behind value and gate_pre), from the kernel's per-workgroup
    partial rows where K allows it. With ``gate_is_sigmoid`` the third operand is the saved
    ``sigmoid(gate_pre)`` itself."""
    lib = _lib.load()
    R, K = grad.shape
    if d_value is None:
        d_value = torch.empty((R, K), device=grad.device, dtype=grad.dtype)
    if d_gate_pre is None:
        d_gate_pre = torch.empty((R, K), device=grad.device, dtype=grad.dtype)
    nparts = lib.gnn_gate_bwd_partials(R, K) if sums else 0
    part = torch.empty((nparts, 2, K), device=grad.device, dtype=torch.float32) if nparts else None
    a = _lib.GateBwdArgs()
    a.partial = None if part is None else part.data_ptr()
    a.grad, a.value, a.gate_pre = grad.data_ptr(), value.data_ptr(), gate_pre.data_ptr()
    a.d_value, a.d_gate_pre = d_value.data_ptr(), d_gate_pre.data_ptr()
    if mask_rows is not None:
        a.mask, a.mask_stride = mask_rows.data_ptr(), mask_rows.stride(0)
    a.rows, a.K = R, K
    a.grad_stride, a.value_stride, a.gate_stride = grad.stride(0), value.stride(0), gate_pre.stride(0)
    a.dv_stride, a.dg_stride = d_value.stride(0), d_gate_pre.stride(0)
    a.dtype = _lib.DTYPE_CODE[grad.dtype]
    a.gate_is_sigmoid = int(gate_is_sigmoid)
    _lib.call("gnn_trimul_gate_bwd", a, grad.device)
    if not sums:
        return d_value, d_gate_pre
    if part is not None:
        colsum = part.sum(0)
        return d_value, d_gate_pre, colsum[0], colsum[1]
    return (d_value, d_gate_pre, d_value.sum(0, dtype=torch.float32), d_gate_pre.sum(0, dtype=torch.float32))


def proj_bwd_supported(dtype, C, Ch):
    """Whether gnn_trimul_proj_bwd covers these widths (16-bit, C in {64, 128}, 2 Ch <= 256)."""
    return dtype in (torch.bfloat16, torch.float16) and C in (64, 128) and 16 <= Ch <= 128 and (2 * Ch) % 32 == 0


def proj_bwd_hip(xk, w, mask_rows, dab, d_p, d_g, eps):
    """gnn_trimul_proj_bwd: z = LN_in(x) and the backward of a|b = p * sigmoid(g) * mask
    with p / g recomputed on the fly; writes ``d_p`` / ``d_g`` (row views) and returns
    ``(z, p_in bias gradient, g_in bias gradient)``, the latter two fp32."""
    lib = _lib.load()
    M, C = xk.shape
    Ch = w["p_in_weight"].shape[0] // 2
    z = torch.empty((M, C), device=xk.device, dtype=xk.dtype)
    part = torch.empty((lib.gnn_trimul_proj_bwd_partials(M), 2, 2 * Ch), device=xk.device, dtype=torch.float32)
    w = {k: (None if v is None else _kernel_ready(v, xk)) for k, v in w.items()}
    a = _lib.TrimulProjBwdArgs()
    a.x, a.z, a.partial = xk.data_ptr(), z.data_ptr(), part.data_ptr()
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    a.ln_w, a.ln_b = ptr(w.get("norm_in_weight")), ptr(w.get("norm_in_bias"))
    a.p_in_w, a.p_in_b = w["p_in_weight"].data_ptr(), ptr(w.get("p_in_bias"))
    a.g_in_w, a.g_in_b = w["g_in_weight"].data_ptr(), ptr(w.get("g_in_bias"))
    if mask_rows is not None:
        a.mask, a.mask_stride = mask_rows.data_ptr(), mask_rows.stride(0)
    a.d_ab, a.d_p, a.d_g = dab.data_ptr(), d_p.data_ptr(), d_g.data_ptr()
    a.rows, a.C, a.Ch = M, C, Ch
    a.x_ld, a.dab_ld, a.dl_ld = xk.stride(0), dab.stride(0), d_p.stride(0)
    a.eps, a.dtype = float(eps), _lib.DTYPE_CODE[xk.dtype]
    _lib.call("gnn_trimul_proj_bwd", a, xk.device)
    sums = part.sum(0)
    return z, sums[0], sums[1]


def out_bwd_supported(dtype, C, Ch):
    """Whether gnn_trimul_out_bwd covers these widths (16-bit, C in {64, 128}, c_hidden in {32, 64, 128})."""
    return dtype in (torch.bfloat16, torch.float16) and C in (64, 128) and Ch in (32, 64, 128)


def out_bwd_hip(o_cm, w, gate_pm, dout2, d_go, B, N, eps):
    """gnn_trimul_out_bwd: from the channel-major ``o_cm`` [B, Ch, N, NP], the saved gate and
    the output gradient (pixel-major rows), ``(on, dy, d_o, sums)`` with on = LN_out(o), dy the
    gradient of p_out's output, d_o that of o (pixel-major) and ``sums`` [4, 128] fp32 (the
    p_out / g_out bias and the LN_out weight / bias gradients, each from column 0); d(g_out
    pre-activation) goes into ``d_go`` (a row view)."""
    lib = _lib.load()
    M, C = dout2.shape
    Ch = o_cm.shape[1]
    dev, dt = dout2.device, dout2.dtype
    on = torch.empty((M, Ch), device=dev, dtype=dt)
    dy = torch.empty((M, C), device=dev, dtype=dt)
    d_o = torch.empty((M, Ch), device=dev, dtype=dt)
    part = torch.empty((lib.gnn_trimul_out_bwd_partials(B, N), 4, 128), device=dev, dtype=torch.float32)
    w = {k: (None if v is None else _kernel_ready(v, dout2)) for k, v in w.items()}
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    a = _lib.TrimulOutBwdArgs()
    a.o, a.gate, a.dout = o_cm.data_ptr(), gate_pm.data_ptr(), dout2.data_ptr()
    a.ln_w, a.ln_b = ptr(w.get("norm_out_weight")), ptr(w.get("norm_out_bias"))
    a.p_out_w, a.p_out_b = w["p_out_weight"].data_ptr(), ptr(w.get("p_out_bias"))
    a.on, a.dy, a.d_go, a.d_o, a.partial = on.data_ptr(), dy.data_ptr(), d_go.data_ptr(), d_o.data_ptr(), part.data_ptr()
    a.B, a.N, a.C, a.Ch = B, N, C, Ch
    a.dgo_ld = d_go.stride(0)
    a.eps, a.dtype = float(eps), _lib.DTYPE_CODE[dt]
    _lib.call("gnn_trimul_out_bwd", a, dev)
    return on, dy, d_o, part.sum(0)


def _wgrad(d, t, slices=64):
    """``d^T t`` for ``[M, O]`` / ``[M, I]`` with M in the hundreds of thousands: the sum
    over M split into batched slices (one GEMM each, summed in fp32 in slice order), since a
    single product with an O x I output leaves most of the GPU idle."""
    M = d.shape[0]
    while slices > 1 and M % slices:
        slices //= 2
    ds = d.reshape(slices, M // slices, d.shape[1])
    ts = t.reshape(slices, M // slices, t.shape[1])
    return torch.bmm(ds.transpose(1, 2), ts).sum(0, dtype=torch.float32)  # [O, I], contiguous


def _operand(ws, off, B, Ch, N, NP, dtype):
    """The contraction operand of the workspace as ``[B * Ch, N, N]`` (row = output index,
    column = contraction index), contiguous."""
    el = torch.empty((), dtype=dtype).element_size()
    n = B * Ch * N * NP
    flat = ws[off:off + n * el].view(dtype)
    if el == 2:  # k-blocked [B, Ch, NP / 32, N, 32]
        t = flat.view(B * Ch, NP // 32, N, 32).permute(0, 2, 1, 3).reshape(B * Ch, N, NP)
    else:  # row-major [B, Ch, N, NP]
        t = flat.view(B * Ch, N, NP)
    return t[..., :N].contiguous()


def relayout_hip(src, dst, mode, B, N, Ch, *, src_ld, dst_ld, src_c0=0, dst_c0=0, transposed=False):
    """gnn_trimul_relayout (16-bit) between pixel-major rows and per-channel planes."""
    a = _lib.TrimulRelayoutArgs()
    a.src, a.dst = src.data_ptr(), dst.data_ptr()
    a.B, a.N, a.Ch = B, N, Ch
    a.src_ld, a.dst_ld, a.src_c0, a.dst_c0 = src_ld, dst_ld, src_c0, dst_c0
    a.mode, a.transposed, a.dtype = mode, int(transposed), _lib.DTYPE_CODE[src.dtype]
    _lib.call("gnn_trimul_relayout", a, src.device)
    return dst


def contract_bwd_hip(workspace, offsets, do_pm, B, Ch, N):
    """``(dA, dB)`` ``[B, Ch, N, NP]`` of the contraction o_c = A_c B_c^T for 16-bit types:
    ``dA_c = dO_c B_c`` and ``dB_c = dO_c^T A_c``, with A and B read in place from the
    forward's ``workspace`` and dO given pixel-major, ``do_pm`` ``[B N N, Ch]`` (plane c of
    batch b: dO_c[i, j] = do_pm[(b, i, j), c])."""
    dt, dev = do_pm.dtype, do_pm.device
    NP = (N + 31) // 32 * 32
    do_i = torch.empty((B, Ch, NP // 32, NP, 32), device=dev, dtype=dt)  # [i / 32][j][i % 32]
    do_j = torch.empty_like(do_i)                                       # [j / 32][i][j % 32]
    for t, transposed in ((do_i, False), (do_j, True)):
        relayout_hip(do_pm, t, _lib.RELAYOUT_PIXELS_TO_BLOCKED, B, N, Ch, src_ld=do_pm.stride(0), dst_ld=32,
                     transposed=transposed)
    da = torch.empty((B, Ch, N, NP), device=dev, dtype=dt)
    db = torch.empty_like(da)
    a = _lib.TrimulContractBwdArgs()
    a.a = workspace.data_ptr() + offsets[0]
    a.b = workspace.data_ptr() + offsets[1]
    a.do_i, a.do_j, a.da, a.db = do_i.data_ptr(), do_j.data_ptr(), da.data_ptr(), db.data_ptr()
    a.planes, a.N, a.dtype = B * Ch, N, _lib.DTYPE_CODE[dt]
    _lib.call("gnn_trimul_contract_bwd", a, dev)
    return da, db


def trimul_bwd_hip(x, direction, mask, eps, weights, workspace, offsets, dout, gate=None, fused=None):
    """Gradients ``(dx, {weight name: grad or None})`` of the triangle multiplicative update
    given the forward's ``workspace`` / ``offsets`` (a, b, o), its output gate ``gate``
    (sigmoid(g_out(z)), or None) and the output gradient. With the saved gate, 16-bit inputs
    and widths gnn_trimul_proj_bwd covers (``fused`` None or True), the input side runs as
    that one kernel: the output gate's backward uses the saved gate, and z, the recomputed
    input projections and their gate backward never pass through a [M, 4 Ch + C] tensor;
    otherwise LN_in(x) and the three input projections are recomputed as one linear."""
    outgoing = is_outgoing(direction)
    N, C = x.shape[-2], x.shape[-1]
    lead = x.shape[:-3]
    B = math.prod(lead)
    M = B * N * N
    dt = x.dtype
    dev = x.device
    w = {k: (None if v is None else v.to(device=dev, dtype=dt)) for k, v in weights.items()}
    Ch = w["p_in_weight"].shape[0] // 2
    NP = (N + 31) // 32 * 32

    def zeros_or(t, n):
        return t if t is not None else torch.zeros(n, device=dev, dtype=dt)

    use_fused = gate is not None and proj_bwd_supported(dt, C, Ch) and fused is not False
    if fused and not use_fused:
        raise ValueError("trimul_bwd_hip: the fused input-side backward does not cover this call")
    xk = _aligned(x.reshape(M, C))
    dout2 = _aligned(dout.reshape(M, C).to(dt))
    # the three projections of z as one linear: [p_in (2 Ch); g_in (2 Ch); g_out (C)]
    wcat = torch.cat([w["p_in_weight"], w["g_in_weight"], w["g_out_weight"]], 0)
    if use_fused:
        gate_pm = _aligned(gate.reshape(M, C))
    else:
        z = layernorm_rows_hip(xk, w["norm_in_weight"], w["norm_in_bias"], eps)
        bcat = torch.cat([zeros_or(w["p_in_bias"], 2 * Ch), zeros_or(w["g_in_bias"], 2 * Ch),
                          zeros_or(w["g_out_bias"], C)])
        lin = torch.nn.functional.linear(z, wcat, bcat)  # [M, 4 Ch + C]
        p, gpre, gopre = lin[:, :2 * Ch], lin[:, 2 * Ch:4 * Ch], lin[:, 4 * Ch:]
    # output stage: out = p_out(LN_out(o)) * sigmoid(gopre)
    o_cm = workspace[offsets[3]:offsets[3] + B * Ch * N * NP * x.element_size()].view(dt).view(B, Ch, N, NP)
    dlin = torch.empty((M, 4 * Ch + C), device=dev, dtype=dt)
    grads = {}
    if use_fused and out_bwd_supported(dt, C, Ch):
        # the output side in one kernel, from the channel-major o and the saved gate
        on, dy, do_pm, sums = out_bwd_hip(o_cm, w, gate_pm, dout2, dlin[:, 4 * Ch:], B, N, eps)
        db_pout, db_gout = sums[0, :C], sums[1, :C]
        grads["norm_out_weight"], grads["norm_out_bias"] = sums[2, :Ch], sums[3, :Ch]
    else:
        if x.element_size() == 2:
            o_pm = relayout_hip(o_cm, torch.empty((M, Ch), device=dev, dtype=dt), _lib.RELAYOUT_PLANES_TO_PIXELS,
                                B, N, Ch, src_ld=NP, dst_ld=Ch)
        else:
            o_pm = o_cm[..., :N].permute(0, 2, 3, 1).reshape(M, Ch).contiguous()
        on = layernorm_rows_hip(o_pm, w["norm_out_weight"], w["norm_out_bias"], eps)
        y = torch.nn.functional.linear(on, w["p_out_weight"], w["p_out_bias"])
        if use_fused:  # torch's sigmoid backward reads the saved output as well
            dy, _, db_pout, db_gout = gate_bwd_hip(dout2, y, gate_pm, d_gate_pre=dlin[:, 4 * Ch:], sums=True,
                                                   gate_is_sigmoid=True)
        else:
            dy, _, db_pout, db_gout = gate_bwd_hip(dout2, y, gopre, d_gate_pre=dlin[:, 4 * Ch:], sums=True)
        don = dy @ w["p_out_weight"]
        do_pm, dlnw, dlnb = layernorm_rows_hip(o_pm, w["norm_out_weight"], eps=eps, dy=don, partials=True)
        grads["norm_out_weight"], grads["norm_out_bias"] = dlnw, dlnb
    grads["p_out_weight"] = _wgrad(dy, on)
    grads["p_out_bias"] = db_pout
    # contraction: o_c = A_c B_c^T per (batch, channel) plane; dO_c[i, j] is pixel (i, j).
    # dA / dB planes go back to the pixel layout of a / b (plane [i, k] is pixel (i, k)
    # outgoing, (k, i) incoming), into the two halves of dab.
    dab = torch.empty((M, 2 * Ch), device=dev, dtype=dt)
    if x.element_size() == 2:  # this library's kernels, reading A and B in the workspace
        dA, dB = contract_bwd_hip(workspace, offsets, do_pm, B, Ch, N)
        for t, c0 in ((dA, 0), (dB, Ch)):
            relayout_hip(t, dab, _lib.RELAYOUT_PLANES_TO_PIXELS, B, N, Ch, src_ld=NP, dst_ld=2 * Ch, dst_c0=c0,
                         transposed=not outgoing)
    else:  # fp32: the vendor GEMM
        A = _operand(workspace, offsets[0], B, Ch, N, NP, dt)
        Bm = _operand(workspace, offsets[1], B, Ch, N, NP, dt)
        do_cm = do_pm.view(B, N, N, Ch).permute(0, 3, 1, 2).reshape(B * Ch, N, N).contiguous()
        dA4 = torch.bmm(do_cm, Bm).view(B, Ch, N, N)                                   # dO B
        dB4 = torch.bmm(A.transpose(1, 2), do_cm).view(B, Ch, N, N).transpose(-1, -2)  # dO^T A
        perm = (0, 2, 3, 1) if outgoing else (0, 3, 2, 1)
        dab4 = dab.view(B, N, N, 2 * Ch)
        dab4[..., :Ch] = dA4.permute(*perm)
        dab4[..., Ch:] = dB4.permute(*perm)
    m_rows = None
    if mask is not None:
        m_rows = mask.to(device=dev, dtype=dt).expand(*x.shape[:-1]).reshape(M).contiguous()
    if use_fused:
        z, db_pin, db_gin = proj_bwd_hip(xk, w, m_rows, dab, dlin[:, :2 * Ch], dlin[:, 2 * Ch:4 * Ch], eps)
    else:
        _, _, db_pin, db_gin = gate_bwd_hip(dab, p, gpre, m_rows, d_value=dlin[:, :2 * Ch],
                                            d_gate_pre=dlin[:, 2 * Ch:4 * Ch], sums=True)
    dwcat = _wgrad(dlin, z)
    dbcat = torch.cat([db_pin, db_gin, db_gout])
    grads["p_in_weight"], grads["g_in_weight"], grads["g_out_weight"] = (
        dwcat[:2 * Ch], dwcat[2 * Ch:4 * Ch], dwcat[4 * Ch:])
    grads["p_in_bias"], grads["g_in_bias"], grads["g_out_bias"] = (
        dbcat[:2 * Ch], dbcat[2 * Ch:4 * Ch], dbcat[4 * Ch:])
    dz = dlin @ wcat
    dx, dlnw, dlnb = layernorm_rows_hip(xk, w["norm_in_weight"], eps=eps, dy=dz, partials=True)
    grads["norm_in_weight"], grads["norm_in_bias"] = dlnw, dlnb
    # every parameter gradient is fp32 here: one concatenation and one conversion per
    # parameter dtype instead of a small conversion launch per parameter
    out = dict.fromkeys(_WEIGHT_KEYS)
    by_dtype = {}
    for key in _WEIGHT_KEYS:
        if weights.get(key) is not None:
            by_dtype.setdefault(weights[key].dtype, []).append(key)
    for pdt, keys in by_dtype.items():
        flat = torch.cat([grads[k].reshape(-1) for k in keys]).to(pdt)
        off = 0
        for k in keys:
            n = weights[k].numel()
            out[k] = flat[off:off + n].view(weights[k].shape)
            off += n
    return dx.reshape(x.shape), out
