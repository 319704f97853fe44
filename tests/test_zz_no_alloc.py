"""gnn_triattn_fwd_noalloc (scratch in the library's static device array) against
gnn_triattn_fwd (caller workspace) through the C ABI: identical bits, on two calls in a row,
the second with a smaller input, so a stale array from the first call would show."""

import ctypes

import pytest
import torch

from helpers import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(q, k, v, o, bias, mask):
    from geometric_nn_ops_torch import _lib
    from geometric_nn_ops_torch.triangle._masking import rounded_mask_value

    B, S, N, H, D = q.shape
    a = _lib.TriAttnArgs()
    a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    a.B, a.S, a.N, a.H, a.D = B, S, N, H, D
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", o)):
        setattr(a, name, _lib.I64x4(*t.stride()[:4]))
    if bias is not None:
        a.bias = bias.data_ptr()
        a.bias_stride = _lib.I64x4(bias.stride(0), bias.stride(2), bias.stride(3), bias.stride(4))
    if mask is not None:
        a.mask = mask.data_ptr()
        a.mask_stride = _lib.I64x3(mask.stride(0), mask.stride(1), mask.stride(4))
    a.scale, a.mask_value = D**-0.5, rounded_mask_value(q.dtype)
    a.dtype, a.precision = _lib.DTYPE_CODE[q.dtype], _lib.GNN_PREC_IEEE
    return a


def _both(B, S, N, H, D, dtype, seed, with_bias=True, transposed_bias=False):
    from geometric_nn_ops_torch import _lib
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as TA

    lib = _lib.load()
    g = gen(seed)
    q, k, v = (torch.randn(B, S, N, H, D, generator=g).to(DEV, dtype) for _ in range(3))
    bias = None
    if with_bias:
        bias = torch.randn(B, 1, H, N, N, generator=g).to(DEV, dtype)
        if transposed_bias:
            bias = bias.transpose(-1, -2)
    mask = (torch.rand(B, S, 1, 1, N, generator=g) < 0.8).to(DEV)
    mask[..., 0] = True
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    o_ref, o_na = torch.full_like(q, float("nan")), torch.full_like(q, float("nan"))
    a = _args(q, k, v, o_ref, bias, mask)
    ws = TA.workspace_for(a, q.device)
    _lib.check(lib.gnn_triattn_fwd(ctypes.byref(a), st), "gnn_triattn_fwd")
    b = _args(q, k, v, o_na, bias, mask)
    _lib.check(lib.gnn_triattn_fwd_noalloc(ctypes.byref(b), st), "gnn_triattn_fwd_noalloc")
    torch.cuda.synchronize()
    del ws
    return o_ref, o_na


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_noalloc_matches_the_workspace_entry_point(dtype):
    # the first call fills more of the static array than the second reads
    for shape, seed, tb in (((2, 6, 200, 4, 32), 1, False), ((1, 3, 70, 2, 32), 2, True)):
        o_ref, o_na = _both(*shape, dtype, seed, transposed_bias=tb)
        assert torch.isfinite(o_ref).all()
        assert torch.equal(o_na, o_ref), shape


def test_noalloc_without_scratch_use():
    """Calls that need no scratch (no pair bias; fp32 on the tiled kernel) give the same
    result through both entry points."""
    o_ref, o_na = _both(1, 2, 64, 4, 32, torch.bfloat16, 3, with_bias=False)
    assert torch.equal(o_na, o_ref)
    o_ref, o_na = _both(1, 2, 48, 2, 32, torch.float32, 4, with_bias=False)
    assert torch.equal(o_na, o_ref)
