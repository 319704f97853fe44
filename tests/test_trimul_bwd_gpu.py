"""Triangle multiplicative update backward on the GPU: gnn_layernorm_rows and
gnn_trimul_gate_bwd against the oracle's closed forms, and every gradient of the public op
(through _TrimulHip: HIP forward + HIP backward) against oracle/trimul_grad, which
tests/test_oracle.py pins to finite differences of the forward oracle.

The reference has no native trimul backward (its gradients come from autograd through
trimul_torch, triangle/_trimul.py:31-36), so there is no reference tolerance for gradients;
they are held to the reference's forward tolerance table for the same dtype
(testutil/metrics.py:96-102: bf16 cos >= 1 - 1e-4 and rel-fro <= 1.5e-2, fp32 ieee
cos >= 1 - 1e-6 and rel-fro <= 1.5e-3), each gradient tensor on its own.
"""

import numpy as np
import pytest
import torch
from unittest import mock

from helpers import TRIMUL_TOL, Tolerance, assert_close_to_oracle, gen, np_weights, pair_input, randn, to_np, \
    trimul_weights
from oracle import triangle_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _k():
    from geometric_nn_ops_torch.triangle._kernels import trimul as K
    return K


# ------------------------------------------------------------------ LayerNorm rows kernel
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("K", [32, 96, 128, 512])
def test_layernorm_rows_forward_and_backward(dtype, K):
    R = 301
    g = gen(K)
    # rows are views into a wider buffer: the row stride is not K
    xb = randn((R, K + 32), g=g, scale=2.0) + 0.5
    x = xb.to(DEV, dtype)[:, 16:16 + K]
    dyb = randn((R, K + 64), g=g)
    dy = dyb.to(DEV, dtype)[:, :K]
    w = (1 + 0.3 * randn((K,), g=g)).to(DEV, dtype)
    b = (0.3 * randn((K,), g=g)).to(DEV, dtype)
    tol = TRIMUL_TOL[dtype, "ieee"]
    y = _k().layernorm_rows_hip(x, w, b, 1e-5)
    assert_close_to_oracle("ln", y, O.layer_norm(to_np(x), to_np(w), to_np(b)), tol)
    dx, dw, db = _k().layernorm_rows_hip(x, w, eps=1e-5, dy=dy, partials=True)
    want = O.layer_norm_grad(to_np(x), to_np(dy), to_np(w))
    assert_close_to_oracle("dx", dx, want[0], tol)
    assert_close_to_oracle("dw", dw, want[1], Tolerance(1 - 1e-6, 1e-4))  # fp32 sums of fp32 products
    assert_close_to_oracle("db", db, want[2], Tolerance(1 - 1e-6, 1e-4))


def test_layernorm_rows_partials_are_deterministic():
    x = randn((5000, 128), seed=3).to(DEV, torch.bfloat16)
    dy = randn((5000, 128), seed=4).to(DEV, torch.bfloat16)
    first = _k().layernorm_rows_hip(x, None, eps=1e-5, dy=dy, partials=True)
    for _ in range(3):
        again = _k().layernorm_rows_hip(x, None, eps=1e-5, dy=dy, partials=True)
        for a, b in zip(first, again):
            assert torch.equal(a, b)


# ------------------------------------------------------------------ gate backward kernel
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
@pytest.mark.parametrize("K", [96, 128])
def test_gate_bwd(dtype, masked, K):
    """Values against the oracle's formula, and the column sums (bias gradients): from the
    kernel's per-workgroup partials at K = 128, from torch at K = 96 (12 chunks per row do
    not divide the workgroup); both equal the sums of the stored outputs."""
    R = 333 if K == 96 else 70000
    g = gen(7)
    buf = randn((R, 3 * K + 32), g=g, scale=3.0).to(DEV, dtype)
    grad, value, gate = buf[:, :K], buf[:, K + 8:2 * K + 8], buf[:, 2 * K + 16:3 * K + 16]
    mask = (torch.rand(R, generator=g) < 0.7).to(DEV, dtype) if masked else None
    out = torch.zeros((R, 2 * K + 16), device=DEV, dtype=dtype)
    dv, dg, sdv, sdg = _k().gate_bwd_hip(grad, value, gate, mask, d_value=out[:, :K], d_gate_pre=out[:, K + 16:],
                                         sums=True)
    for got, t in ((sdv, dv), (sdg, dg)):
        want = t.double().sum(0)
        assert got.dtype == torch.float32
        torch.testing.assert_close(got.double(), want, rtol=1e-5, atol=1e-3)
    gr, v, gp = (to_np(t) for t in (grad, value, gate))
    s = 1 / (1 + np.exp(-gp))
    m = to_np(mask)[:, None] if masked else 1.0
    tol = TRIMUL_TOL[dtype, "ieee"]
    assert_close_to_oracle("d_value", dv, gr * s * m, tol)
    assert_close_to_oracle("d_gate_pre", dg, gr * v * m * s * (1 - s), tol)
    assert torch.count_nonzero(out[:, K:K + 16]) == 0  # the gap between the two outputs is untouched


# ------------------------------------------------------- contraction backward kernel
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("N", [1, 37, 64, 100, 300, 512, 700])
def test_contract_bwd_kernel(dtype, N):
    """gnn_trimul_contract_bwd against fp32 matmuls of the same 16-bit operands: dA = dO B and
    dB = dO^T A per plane, A and B given k-blocked in a workspace as the forward leaves them
    (128-row tiles below N = 512, 256-row tiles from 512 on; N not a multiple of 32 exercises
    the zero-padded dO rows against the clamped operand rows)."""
    from oracle.triangle_oracle import rel_fro

    B, Ch = 1, 8
    NP = (N + 31) // 32 * 32
    g = gen(N)
    A, Bm, dO = (randn((B, Ch, N, N), g=g).to(DEV, dtype) for _ in range(3))

    def kblocked(t):  # [B, Ch, N, N] -> [B, Ch, NP / 32, N, 32], zero columns past N
        z = torch.zeros((B, Ch, N, NP), device=DEV, dtype=dtype)
        z[..., :N] = t
        return z.view(B, Ch, N, NP // 32, 32).permute(0, 1, 3, 2, 4).contiguous()

    nbytes = B * Ch * N * NP * 2
    cm = (nbytes + 255) // 256 * 256
    ws = torch.zeros(2 * cm, device=DEV, dtype=torch.uint8)
    ws[:nbytes].view(dtype).copy_(kblocked(A).flatten())
    ws[cm:cm + nbytes].view(dtype).copy_(kblocked(Bm).flatten())
    do_pm = dO.permute(0, 2, 3, 1).reshape(B * N * N, Ch).contiguous()
    da, db = _k().contract_bwd_hip(ws, (0, cm), do_pm, B, Ch, N)
    want_a = dO.float() @ Bm.float()
    want_b = dO.float().transpose(-1, -2) @ A.float()
    bound = 4e-3 if dtype == torch.bfloat16 else 1e-3  # one rounding of the outputs
    for got, want in ((da[..., :N], want_a), (db[..., :N], want_b)):
        assert torch.isfinite(got).all()
        assert rel_fro(got.double().cpu().numpy(), want.double().cpu().numpy()) < bound


@pytest.mark.parametrize("N", [5, 40, 96, 130])
def test_relayout_kernels(N):
    """gnn_trimul_relayout against torch permutes, bit-exact: pixel rows -> i- and j-blocked
    planes (zero outside N x N), and planes -> pixel rows (plain and transposed) into a
    channel window of wider rows (the halves of dab)."""
    from geometric_nn_ops_torch import _lib

    K = _k()
    B, Ch, dtype = 2, 24, torch.bfloat16
    NP = (N + 31) // 32 * 32
    pm = randn((B, N, N, Ch + 8), seed=N).to(DEV, dtype)  # 8 extra channels: src_c0 = 8
    blocked = torch.full((B, Ch, NP // 32, NP, 32), float("nan"), device=DEV, dtype=dtype)
    sq = torch.zeros((B, Ch, NP, NP), device=DEV, dtype=dtype)
    sq[:, :, :N, :N] = pm[..., 8:].permute(0, 3, 1, 2)
    for transposed, want in ((False, sq.view(B, Ch, NP // 32, 32, NP).transpose(-1, -2)),
                             (True, sq.view(B, Ch, NP, NP // 32, 32).permute(0, 1, 3, 2, 4))):
        K.relayout_hip(pm.view(-1, Ch + 8), blocked, _lib.RELAYOUT_PIXELS_TO_BLOCKED, B, N, Ch, src_ld=Ch + 8,
                       dst_ld=32, src_c0=8, transposed=transposed)
        assert torch.equal(blocked, want.contiguous())
    planes = randn((B, Ch, N, NP), seed=N + 1).to(DEV, dtype)
    for transposed in (False, True):
        out = torch.full((B, N, N, 2 * Ch), float("nan"), device=DEV, dtype=dtype)
        K.relayout_hip(planes, out, _lib.RELAYOUT_PLANES_TO_PIXELS, B, N, Ch, src_ld=NP, dst_ld=2 * Ch,
                       dst_c0=Ch, transposed=transposed)
        want = planes[..., :N].permute(0, 3, 2, 1) if transposed else planes[..., :N].permute(0, 2, 3, 1)
        assert torch.equal(out[..., Ch:], want)
        assert torch.isnan(out[..., :Ch]).all()  # the other channel window is untouched


# ------------------------------------------------------------------ the op's gradients
def _run(x, direction, mask, w, dout):
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    x = x.to(DEV).requires_grad_()
    wd = {k: v.to(DEV).requires_grad_() for k, v in w.items()}
    out = triangle_multiplicative_update(x, direction, None if mask is None else mask.to(DEV), **wd)
    out.backward(dout.to(DEV, out.dtype))
    return out, x.grad, {k: v.grad for k, v in wd.items()}


def _check_grads(x, direction, mask, w, dout, dtype):
    _, gx, gw = _run(x, direction, mask, w, dout)
    want = O.trimul_grad(to_np(x), direction, None if mask is None else to_np(mask), to_np(dout),
                         **np_weights(w))
    tol = TRIMUL_TOL[dtype, "ieee"]
    assert_close_to_oracle("dx", gx, want["x"], tol)
    for key, grad in gw.items():
        assert grad is not None, key
        assert grad.dtype == dtype
        assert_close_to_oracle(key, grad, want[key], tol)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_trimul_grads_match_oracle(direction, dtype):
    w = trimul_weights(64, 32, dtype, seed=41, biases=True, ln_random=True)
    x, mask = pair_input(2, 24, 64, dtype, seed=42)
    dout = randn((2, 24, 24, 64), seed=43).to(dtype)
    _check_grads(x, direction, mask, w, dout, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize(("C", "Ch", "N", "direction"),
                         [(128, 128, 40, "outgoing"), (64, 32, 70, "incoming"), (128, 64, 24, "incoming"),
                          (128, 96, 40, "outgoing")],
                         ids=["c128_h128_n40", "c64_h32_n70", "c128_h64_n24", "c128_h96_n40"])
def test_fused_backward_matches_unfused(dtype, C, Ch, N, direction):
    """The fused backward kernels -- gnn_trimul_proj_bwd (z, the input projections recomputed
    tile by tile, their gate backward) and gnn_trimul_out_bwd (LN_out, p_out recomputed, the
    output gate's backward from the saved gate, d(on) and the LN_out backward; not for
    c_hidden = 96, which keeps the unfused output side) -- against the unfused path (LayerNorms,
    linears and gates as separate launches from recomputed pre-activations), on the same
    forward: every gradient, with projection biases, random LayerNorm parameters and a mask;
    N = 70 leaves a partial last pixel tile (and, for the output side, a partial row tile)."""
    K = _k()
    w = {k: v.to(DEV) for k, v in trimul_weights(C, Ch, dtype, seed=91, biases=True, ln_random=True).items()}
    x, mask = pair_input(1, N, C, dtype, seed=92)
    x, mask = x.to(DEV), mask.to(DEV)
    dout = randn((1, N, N, C), seed=93).to(DEV, dtype)
    with torch.no_grad():
        args, keep, out, ws, off = K.build_args(x, direction, mask, 1e-5, w, separate_gate=True)
        K.run_stage("gnn_trimul_fwd", args, x.device)
        gate = keep[-1]
        got = K.trimul_bwd_hip(x, direction, mask, 1e-5, w, ws, off, dout, gate=gate, fused=True)
        want = K.trimul_bwd_hip(x, direction, mask, 1e-5, w, ws, off, dout, gate=gate, fused=False)
    # the two paths round differently (the saved bf16 / fp16 gate against a sigmoid of the
    # recomputed pre-activation; z from two LayerNorm kernels): each against the other at the
    # 16-bit bar, and the fused one against the fp64 oracle
    tol = Tolerance(1 - 1e-4, 1e-2)
    oracle = O.trimul_grad(to_np(x), direction, to_np(mask), to_np(dout), **np_weights(w))
    assert_close_to_oracle("dx", got[0], to_np(want[0]).astype(np.float64), tol)
    assert_close_to_oracle("dx", got[0], oracle["x"], TRIMUL_TOL[torch.bfloat16, "ieee"])
    for key, grad in got[1].items():
        if grad is None:
            assert want[1][key] is None, key
            continue
        assert_close_to_oracle(key, grad, to_np(want[1][key]).astype(np.float64), tol)
        assert_close_to_oracle(key, grad, oracle[key], TRIMUL_TOL[torch.bfloat16, "ieee"])


def test_fused_backward_refusals():
    """gnn_trimul_proj_bwd covers 16-bit inputs with C in {64, 128} and 2 c_hidden <= 256,
    gnn_trimul_out_bwd 16-bit inputs with C in {64, 128} and c_hidden in {32, 64, 128};
    trimul_bwd_hip takes the unfused path by itself outside them."""
    K = _k()
    assert K.proj_bwd_supported(torch.bfloat16, 128, 128) and K.proj_bwd_supported(torch.float16, 64, 32)
    assert not K.proj_bwd_supported(torch.float32, 128, 128)
    assert not K.proj_bwd_supported(torch.bfloat16, 96, 32)
    assert not K.proj_bwd_supported(torch.bfloat16, 128, 160)
    assert K.out_bwd_supported(torch.bfloat16, 128, 128) and K.out_bwd_supported(torch.float16, 64, 32)
    assert not K.out_bwd_supported(torch.bfloat16, 128, 96) and not K.out_bwd_supported(torch.float32, 128, 128)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_grads_c128_ragged_n(direction):
    """c_z = c_hidden = 128 (the fixed-width projection kernel) at an N that is not a multiple
    of 32 (row padding of the a / b operands)."""
    dtype = torch.bfloat16
    w = trimul_weights(128, 128, dtype, seed=51, biases=True, ln_random=True)
    x, mask = pair_input(1, 40, 128, dtype, seed=52)
    dout = randn((1, 40, 40, 128), seed=53).to(dtype)
    _check_grads(x, direction, mask, w, dout, dtype)


def test_trimul_grads_batched_no_mask_no_biases():
    dtype = torch.bfloat16
    w = trimul_weights(64, 64, dtype, seed=61)  # LN affine present, projection biases absent
    x, _ = pair_input((2, 2), 16, 64, dtype, seed=62)
    dout = randn((2, 2, 16, 16, 64), seed=63).to(dtype)
    _check_grads(x, "incoming", None, w, dout, dtype)


def test_grad_calls_take_the_hip_backward():
    from geometric_nn_ops_torch.triangle import _trimul

    w = trimul_weights(32, 32, torch.bfloat16, seed=1)
    x, mask = pair_input(1, 12, 32, torch.bfloat16, seed=3)
    with mock.patch.object(_trimul, "trimul_torch", wraps=_trimul.trimul_torch) as ref:
        out, gx, _ = _run(x, "outgoing", mask, w, torch.ones(1, 12, 12, 32))
    assert not ref.called
    assert out.grad_fn is not None and "TrimulHip" in type(out.grad_fn).__name__
    assert gx is not None and torch.isfinite(gx).all()


def test_mask_requiring_grad_takes_the_torch_path():
    from geometric_nn_ops_torch.triangle import _trimul, triangle_multiplicative_update

    w = {k: v.to(DEV) for k, v in trimul_weights(32, 32, torch.float32, seed=1).items()}
    x, mask = pair_input(1, 12, 32, torch.float32, seed=3)
    mask = mask.to(DEV).requires_grad_()
    with mock.patch.object(_trimul, "trimul_torch", wraps=_trimul.trimul_torch) as ref:
        out = triangle_multiplicative_update(x.to(DEV).requires_grad_(), "outgoing", mask, **w)
        out.sum().backward()
    assert ref.called and mask.grad is not None


def test_backward_twice_with_retained_graph():
    """The forward's workspace belongs to the graph: a second backward over a graph kept with
    ``retain_graph=True`` gives the same gradients as the first."""
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    dtype = torch.bfloat16
    w = {k: v.to(DEV).requires_grad_() for k, v in trimul_weights(64, 64, dtype, seed=71, biases=True).items()}
    x, mask = pair_input(1, 20, 64, dtype, seed=72)
    x = x.to(DEV).requires_grad_()
    out = triangle_multiplicative_update(x, "incoming", mask.to(DEV), **w)
    assert "TrimulHip" in type(out.grad_fn).__name__
    dout = randn((1, 20, 20, 64), seed=73).to(DEV, dtype)
    first = torch.autograd.grad(out, [x, w["p_in_weight"], w["norm_out_weight"]], dout, retain_graph=True)
    out.backward(dout)
    assert torch.equal(x.grad, first[0])
    assert torch.equal(w["p_in_weight"].grad, first[1])
    assert torch.equal(w["norm_out_weight"].grad, first[2])


def test_second_derivative_raises():
    """The HIP backward records no graph of its own, so a double backward is refused rather
    than returning partial second-order gradients."""
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    dtype = torch.bfloat16
    w = {k: v.to(DEV) for k, v in trimul_weights(32, 32, dtype, seed=74).items()}
    x, _ = pair_input(1, 12, 32, dtype, seed=75)
    x = x.to(DEV).requires_grad_()
    out = triangle_multiplicative_update(x, "outgoing", None, **w)
    (gx,) = torch.autograd.grad(out.float().square().sum(), x, create_graph=True)
    with pytest.raises(RuntimeError):
        gx.float().sum().backward()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_separate_gate_buffer(dtype):
    """gnn_trimul_args.gate: the output gate in a buffer of its own gives the same output bit
    for bit, and the workspace then stops at the gate offset (a, b and o only); the autograd
    forward keeps that workspace (and the gate buffer where the fused input-side backward
    reads it)."""
    from geometric_nn_ops_torch.triangle import _trimul

    K = _k()
    w = {k: v.to(DEV) for k, v in trimul_weights(64, 64, dtype, seed=81, biases=True).items()}
    x, mask = pair_input(1, 40, 64, dtype, seed=82)
    x, mask = x.to(DEV), mask.to(DEV)
    with torch.no_grad():
        outs, wss = [], []
        for sep in (False, True):
            args, keep, out, ws, off = K.build_args(x, "incoming", mask, 1e-5, w, separate_gate=sep)
            K.run_stage("gnn_trimul_fwd", args, x.device)
            torch.cuda.synchronize()
            outs.append(out)
            wss.append((ws, off, keep))
    assert torch.equal(outs[0], outs[1])
    (ws0, off0, _), (ws1, off1, keep1) = wss
    assert ws1.numel() == off1[2] < ws0.numel()
    el = x.element_size()
    N, Ch, NP = 40, 64, 64
    assert torch.equal(ws0[:off0[3]], ws1[:off1[3]])  # a and b (zero-padded to NP, fully written)

    def o_valid(ws, off):  # o is [B, Ch, N, NP]; columns >= N are not written
        return ws[off[3]:off[3] + Ch * N * NP * el].view(dtype).view(Ch, N, NP)[..., :N]

    assert torch.equal(o_valid(ws0, off0), o_valid(ws1, off1))
    gate = keep1[-1]
    assert torch.equal(ws0[off0[2]:off0[2] + gate.numel() * el].view(dtype).view(gate.shape), gate)
    # the autograd forward keeps the a / b / o workspace only
    captured = {}
    real = _trimul._TrimulHip.forward

    def spy(ctx, *args):
        o = real(ctx, *args)
        captured["ws"], captured["off"] = ctx.workspace, ctx.offsets
        return o

    xg = x.clone().requires_grad_()
    with mock.patch.object(_trimul._TrimulHip, "forward", staticmethod(spy)):
        out = _trimul.triangle_multiplicative_update(xg, "incoming", mask, **w)
    assert torch.equal(out.detach(), outs[0])
    assert captured["ws"].numel() == captured["off"][2]
