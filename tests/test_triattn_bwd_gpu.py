"""HIP triangle-attention backward (gnn_triattn_bwd through the public op's autograd)
against the fp64 oracle gradients (oracle.triangle_attention_grad, pinned by finite
differences), with the reference's tolerance table (testutil/metrics.py:103-108, which its
tests apply to the gradients as well) and the structural zero gradients of masked keys."""

import pytest
import torch

from helpers import TRIANGLE_ATTENTION_TOL, assert_close_to_oracle, attention_inputs, gen, key_mask, to_np
from oracle import triangle_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])


def run(q, k, v, bias, mask, scale, dout):
    from geometric_nn_ops_torch.triangle import triangle_attention

    leaves = [t.detach().requires_grad_(True) for t in (q, k, v)]
    b = None if bias is None else bias.detach().requires_grad_(True)
    o = triangle_attention(*leaves, b, mask, scale)
    o.backward(dout)
    return o, [t.grad for t in leaves], None if b is None else b.grad


class matmul_precision:
    """Sets torch.backends.cuda.matmul.fp32_precision for a block (not thread safe)."""

    def __init__(self, value):
        self.value = value

    def __enter__(self):
        self.old = torch.backends.cuda.matmul.fp32_precision
        torch.backends.cuda.matmul.fp32_precision = self.value

    def __exit__(self, *exc):
        torch.backends.cuda.matmul.fp32_precision = self.old


def check_against_oracle(shape, dtype, *, with_bias=True, with_mask=True, seed=0, scale=None, dead_rows=(),
                         precision="ieee"):
    B, S, N, H, D = shape
    t = attention_inputs(B, S, N, H, D, dtype, seed=seed, with_bias=with_bias, bias_scale=0.5, device=DEV)
    mask = key_mask(B, S, N, seed=seed + 1, frac_keep=0.75, device=DEV) if with_mask else None
    for s in dead_rows:  # every key of N_seq row s masked
        mask[:, s] = False
    dout = (torch.randn(B, S, N, H, D, generator=gen(seed + 2))).to(DEV, dtype)
    with matmul_precision(precision if dtype == torch.float32 else "ieee"):
        o, (dq, dk, dv), db = run(t["q"], t["k"], t["v"], t.get("bias"), mask, scale, dout)
    want = O.triangle_attention_grad(to_np(t["q"]), to_np(t["k"]), to_np(t["v"]),
                                     None if not with_bias else to_np(t["bias"]),
                                     None if mask is None else mask.cpu().numpy(), scale, to_np(dout))
    tol = TRIANGLE_ATTENTION_TOL[dtype, precision if dtype == torch.float32 else "ieee"]
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), want[:3]):
        assert_close_to_oracle(name, got, ref, tol)
    if with_bias:
        assert_close_to_oracle("dbias", db, want[3], tol)
    return mask, (dk, dv)


def test_uses_the_hip_backward(monkeypatch):
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as K

    calls = []
    real = K.triangle_attention_bwd_hip
    monkeypatch.setattr(K, "triangle_attention_bwd_hip", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    check_against_oracle((1, 2, 32, 2, 32), torch.bfloat16, seed=3)
    assert calls == [1]


@DTYPES
@pytest.mark.parametrize("shape", [(1, 1, 32, 4, 32), (1, 4, 48, 2, 16), (2, 2, 100, 2, 32), (1, 3, 130, 4, 8),
                                   (1, 2, 200, 2, 24), (1, 2, 257, 1, 32)],
                         ids=["n32", "d16", "n100_batched", "n130_d8", "n200_d24", "n257"])
def test_matches_oracle(shape, dtype):
    check_against_oracle(shape, dtype, seed=11)


@DTYPES
@pytest.mark.parametrize(("with_bias", "with_mask"), [(False, False), (False, True), (True, False)],
                         ids=["plain", "mask_only", "bias_only"])
def test_optional_inputs(dtype, with_bias, with_mask):
    check_against_oracle((1, 3, 72, 2, 32), dtype, with_bias=with_bias, with_mask=with_mask, seed=5, scale=0.3)


@DTYPES
def test_masked_keys_get_no_key_or_value_gradient(dtype):
    mask, (dk, dv) = check_against_oracle((1, 3, 96, 2, 32), dtype, seed=21)
    dropped = ~mask[:, :, 0, 0, :]  # [B, S, N]
    assert dropped.any()
    assert torch.all(dk[dropped] == 0) and torch.all(dv[dropped] == 0)


def test_ending_node_views():
    """Ending-node callers pass transposed views (storage [B, N, S, H, D], canonical
    [B, S, N, H, D] by strides): the backward reads them by strides."""
    B, S, N, H, D = 1, 3, 64, 2, 32
    dtype = torch.bfloat16
    store = attention_inputs(B, N, S, H, D, dtype, seed=31, with_bias=False, device=DEV)
    q, k, v = (store[x].transpose(1, 2) for x in "qkv")
    assert not q.is_contiguous()
    bias = (0.5 * torch.randn(B, 1, H, N, N, generator=gen(32))).to(DEV, dtype)
    mask = key_mask(B, S, N, seed=33, device=DEV)
    dout = torch.randn(B, S, N, H, D, generator=gen(34)).to(DEV, dtype)
    _, (dq, dk, dv), db = run(q, k, v, bias, mask, None, dout)
    want = O.triangle_attention_grad(to_np(q), to_np(k), to_np(v), to_np(bias), mask.cpu().numpy(), None,
                                     to_np(dout))
    tol = TRIANGLE_ATTENTION_TOL[dtype, "ieee"]
    for name, got, ref in zip(("dq", "dk", "dv", "dbias"), (dq, dk, dv, db), want):
        assert_close_to_oracle(name, got, ref, tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16,
                                   pytest.param(torch.float16, marks=pytest.mark.xfail(
                                       strict=True, reason="fp16 mask_val too small to swamp the logits"))],
                         ids=["bf16", "fp16"])
@pytest.mark.parametrize("n", [64, 96], ids=["n64", "n96"])
def test_fully_masked_rows(dtype, n):
    """N_seq rows whose keys are all masked next to ordinary rows, as the reference's
    test_fully_masked_row (tests/test_triangle_attention.py:535-562, fp16 a strict xfail
    there too): the forward's lse of such a row is the bare sentinel, and P of a masked key
    is divided by N_res (the reference's correction) to give softmax's uniform 1 / N_res.
    n = 64 is one whole key tile, n = 96 a ragged one."""
    check_against_oracle((1, 4, n, 2, 32), dtype, seed=61, dead_rows=(1, 3))


@pytest.mark.parametrize("n", [1024, 1025], ids=["n1024_row_max", "n1025_tiled"])
def test_row_kernel_limit(n):
    """D = 32 at the row-resident backward's largest N_res (1024: K / V or Q' / dO of a row
    fill 128 KB of LDS) and one past it (the tiled dq / dk-dv kernels take over)."""
    check_against_oracle((1, 1, n, 2, 32), torch.bfloat16, seed=71)


@pytest.mark.parametrize("splits", [1, 3], ids=["one_range", "three_ranges"])
def test_dbias_long_row_ranges(splits, monkeypatch):
    """The pair-bias gradient with N_seq ranges longer than 64 rows (the D = 32 kernel stages
    the key-mask bytes 64 rows at a time) and ranges of uneven length, fully masked rows on
    both sides of the 64-row boundary, ragged keys (N = 72)."""
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as K

    monkeypatch.setattr(K, "dbias_splits", lambda *a: splits)
    check_against_oracle((1, 131, 72, 2, 32), torch.bfloat16, seed=83, dead_rows=(5, 64, 70))


def test_headline_rows_bf16():
    """N_res = 512 (the headline width), 8 N_seq rows, pair bias and ragged masks."""
    check_against_oracle((1, 8, 512, 4, 32), torch.bfloat16, seed=41)


@pytest.mark.parametrize("precision", ["ieee", "tf32"])
@pytest.mark.parametrize("shape", [(1, 1, 32, 4, 32), (1, 4, 32, 8, 8), (1, 1, 64, 16, 48), (2, 2, 48, 4, 32),
                                   (1, 3, 130, 2, 64)],
                         ids=["pairformer_32", "msa_d8", "atom_d48", "batched", "n130_d64"])
def test_fp32_hip_backward(shape, precision, monkeypatch):
    """fp32 gradients through the HIP backward under both fp32_precision settings ('tf32'
    resolves to the bf16x3 split on gfx950), at the reference's SHAPES
    (tests/test_triangle_attention.py:46-51, its fp32 ieee / tf32 accuracy cases :493-512)
    and a ragged N = 130 at the largest fp32 head dim, against the fp64 oracle with the
    reference's fp32 tolerances."""
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as K

    calls = []
    real = K.triangle_attention_bwd_hip
    monkeypatch.setattr(K, "triangle_attention_bwd_hip", lambda *a, **kw: calls.append(kw.get("precision")) or real(*a, **kw))
    check_against_oracle(shape, torch.float32, seed=51, precision=precision)
    assert calls == ["ieee" if precision == "ieee" else "bf16x3"]


def test_fp32_fully_masked_rows():
    """fp32 rows whose keys are all masked beside ordinary ones, through the HIP backward."""
    check_against_oracle((1, 4, 96, 2, 32), torch.float32, seed=63, dead_rows=(0, 2))


def test_fp32_tf32_changes_the_gradients():
    """The split products differ from the full fp32 ones (the reference's
    test_tf32_changes_the_result, tests/test_triangle_attention.py:460-490)."""
    from geometric_nn_ops_torch.triangle import triangle_attention

    B, S, N, H, D = 1, 1, 32, 4, 32
    t = attention_inputs(B, S, N, H, D, torch.float32, seed=3, with_bias=True, device=DEV)
    mask = key_mask(B, S, N, seed=5, device=DEV)
    dout = torch.randn(B, S, N, H, D, generator=gen(31)).to(DEV)
    grads = {}
    for precision in ("ieee", "tf32"):
        with matmul_precision(precision):
            leaves = [t[n].detach().requires_grad_(True) for n in ("q", "k", "v", "bias")]
            triangle_attention(*leaves[:3], leaves[3], mask).backward(dout)
            grads[precision] = [x.grad for x in leaves]
    for full, reduced in zip(grads["ieee"], grads["tf32"]):
        assert not torch.equal(full, reduced)


def test_fp32_wide_head_keeps_the_torch_gradient(monkeypatch):
    """fp32 head dims above 64 are differentiated by the torch path (no HIP backward call)."""
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as K

    calls = []
    real = K.triangle_attention_bwd_hip
    monkeypatch.setattr(K, "triangle_attention_bwd_hip", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    check_against_oracle((1, 2, 40, 2, 96), torch.float32, seed=51)
    assert calls == []


@DTYPES
@pytest.mark.parametrize("shape", [(1, 2, 40, 2, 64), (1, 3, 100, 2, 48), (1, 2, 130, 2, 128), (2, 2, 72, 1, 96)],
                         ids=["n40_d64", "n100_d48", "n130_d128", "b2_n72_d96"])
def test_wide_heads(shape, dtype, monkeypatch):
    """Head dims above 32 (the reference's atom_d48 case, tests/test_triangle_attention.py:
    46-51, among them) take the HIP backward: the tiled kernels in 32-column chunks of the
    head dim (D = 48 and 64 in two, 96 and 128 in four, the columns past D zero), against
    the oracle's gradients with bias and mask."""
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as K

    calls = []
    real = K.triangle_attention_bwd_hip
    monkeypatch.setattr(K, "triangle_attention_bwd_hip", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    check_against_oracle(shape, dtype, seed=53)
    assert calls == [1]


def test_backward_twice_with_retained_graph_and_no_second_derivative():
    """A retained graph runs the HIP backward again with the same result; a second derivative
    is refused (the backward kernels record no graph)."""
    from geometric_nn_ops_torch.triangle import triangle_attention

    B, S, N, H, D = 1, 2, 40, 2, 32
    t = attention_inputs(B, S, N, H, D, torch.bfloat16, seed=21, with_bias=True, device=DEV)
    q, k, v, bias = (t[n].detach().requires_grad_() for n in ("q", "k", "v", "bias"))
    mask = key_mask(B, S, N, seed=22, device=DEV)
    o = triangle_attention(q, k, v, bias, mask)
    fn = o.grad_fn  # the public op reshapes the Function's output: walk past the view node
    while fn is not None and "TriangleAttentionHip" not in type(fn).__name__:
        fn = fn.next_functions[0][0] if fn.next_functions else None
    assert fn is not None
    dout = torch.randn(B, S, N, H, D, generator=gen(23)).to(DEV, torch.bfloat16)
    first = torch.autograd.grad(o, [q, bias], dout, retain_graph=True)
    o.backward(dout)
    assert torch.equal(q.grad, first[0]) and torch.equal(bias.grad, first[1])

    o2 = triangle_attention(q, k, v, bias, mask)
    (gq,) = torch.autograd.grad(o2.float().square().sum(), q, create_graph=True)
    with pytest.raises(RuntimeError):
        gq.float().sum().backward()
