"""HIP attention with pair bias (pair-bias projection kernel + triangle-attention kernel)
against the fp64 CPU oracle, and the reference's structural tests.

Structural cases restate AMDResearch/geometric-nn-ops tests/test_attention_pair_bias.py:27-230
(masked keys ignored, masked logits suppressed, cached bias, unmasked returned bias, per-copy
masks, the inf argument, fully masked rows, mask layouts, bias shared over the multiplicity
axis); accuracy uses its tolerance table (testutil/metrics.py:110-115) against the fp64
oracle, plus an AF3-pairformer-sized case (H=16, DH=24, c_z=128, 384 tokens).
"""

import numpy as np
import pytest
import torch

from helpers import (ATTENTION_PAIR_BIAS_TOL, apb_inputs, apb_key_mask, assert_close_to_oracle, gen, to_np)
from oracle import triangle_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


class matmul_precision:
    """Sets torch.backends.cuda.matmul.fp32_precision for a block (not thread safe)."""

    def __init__(self, value):
        self.value = value

    def __enter__(self):
        self.old = torch.backends.cuda.matmul.fp32_precision
        torch.backends.cuda.matmul.fp32_precision = self.value

    def __exit__(self, *exc):
        torch.backends.cuda.matmul.fp32_precision = self.old


def apb(**kw):
    from geometric_nn_ops_torch.triangle import attention_pair_bias

    with torch.no_grad():
        return attention_pair_bias(**kw)


def on_gpu(t, dtype):
    return {k: v.to(DEV, dtype) for k, v in t.items()}


def oracle(t, **kw):
    return O.attention_pair_bias(**{k: to_np(v) for k, v in t.items()},
                                 **{k: (to_np(v) if torch.is_tensor(v) else v) for k, v in kw.items()})


def test_uses_the_hip_kernels(monkeypatch):
    """A forward-only GPU call goes through the pair-bias projection, attention and fused
    gate / output projection kernels."""
    from geometric_nn_ops_torch.triangle._kernels import attention_pair_bias as K

    calls = []
    for name in ("pair_bias_projection_hip", "gate_out_hip"):
        real = getattr(K, name)
        monkeypatch.setattr(K, name, lambda *a, _r=real, _n=name, **k: calls.append(_n) or _r(*a, **k))
    t = on_gpu(apb_inputs(1, 1, 4, 32, 32, 16, 16, seed=1), torch.bfloat16)
    out, _ = apb(**t)
    assert calls == ["pair_bias_projection_hip", "gate_out_hip"] and out.is_cuda and out.dtype == torch.bfloat16


@pytest.mark.parametrize(("dtype", "precision"),
                         [(torch.float32, "ieee"), (torch.float32, "tf32"), (torch.bfloat16, "ieee"),
                          (torch.float16, "ieee")], ids=["fp32_ieee", "fp32_tf32", "bf16", "fp16"])
@pytest.mark.parametrize("biases", [True, False], ids=["biases", "no_biases"])
def test_gate_out_kernel_matches_oracle(dtype, precision, biases):
    """gnn_apb_gate_out on its own: c_s, attention width and c_out all different, a token
    count that is not a multiple of the 32-token tile, s read through a padded row pitch
    (the last 32 columns of a wider tensor), against the fp64 oracle of
    (o * sigmoid(s Wg^T + bg)) Wo^T + bo (attention_pair_bias.py:86-89)."""
    from geometric_nn_ops_torch.triangle._kernels import attention_pair_bias as K

    M, Cs, D, Co = 77, 96, 64, 160
    g = gen(31)
    s_wide = torch.randn(M, Cs + 32, generator=g)
    s = s_wide[:, 32:]
    o = torch.randn(M, D, generator=g)
    gw = torch.randn(D, Cs, generator=g) * Cs ** -0.5
    ow = torch.randn(Co, D, generator=g) * D ** -0.5
    gb = torch.randn(D, generator=g) * 0.3 if biases else None
    ob = torch.randn(Co, generator=g) * 0.3 if biases else None
    dev = lambda t: None if t is None else t.to(DEV, dtype)  # noqa: E731
    with matmul_precision(precision):
        got = K.gate_out_hip(dev(s_wide)[:, 32:], dev(o), dev(gw), dev(gb), dev(ow), dev(ob))
    q = lambda t: None if t is None else to_np(t.to(dtype).double())  # noqa: E731
    gate = O.sigmoid(O.linear(q(s), q(gw), q(gb)))
    want = O.linear(q(o) * gate, q(ow), q(ob))
    assert got.shape == (M, Co) and got.dtype == dtype
    tol = {torch.bfloat16: 1e-2, torch.float16: 2e-3}.get(dtype, 2e-3 if precision == "tf32" else 1e-5)
    assert O.rel_fro(to_np(got), want) <= tol


@pytest.mark.parametrize(("dtype", "precision"),
                         [(torch.float32, "ieee"), (torch.float32, "tf32"), (torch.bfloat16, "ieee"),
                          (torch.float16, "ieee")], ids=["fp32_ieee", "fp32_tf32", "bf16", "fp16"])
@pytest.mark.parametrize("shape", [(1, 1, 4, 32, 16, 16), (2, 3, 4, 48, 8, 16), (1, 2, 8, 100, 32, 64),
                                   (2, 1, 2, 70, 24, 40)], ids=["base", "multiplicity", "n100_d32", "ragged"])
def test_matches_oracle(shape, dtype, precision):
    B, M, H, U, DH, Zc = shape
    t = apb_inputs(B, M, H, U, U, DH, Zc, seed=3, biases=True)
    mask = apb_key_mask(B, U, seed=9, frac_keep=0.8)
    with matmul_precision(precision):
        out, pz = apb(**on_gpu(t, dtype), mask=mask.to(DEV), return_z_proj=True)
    q = {k: v.to(dtype).float() for k, v in t.items()}  # the oracle sees the rounded inputs
    want, want_pz = oracle(q, mask=mask, return_z_proj=True)
    tol = ATTENTION_PAIR_BIAS_TOL[dtype, precision]
    assert_close_to_oracle("pz", pz, want_pz, tol)
    assert_close_to_oracle("out", out, want, tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
def test_projection_kernel_matches_oracle(dtype):
    from geometric_nn_ops_torch.triangle._kernels.attention_pair_bias import pair_bias_projection_hip

    g = gen(5)
    z = torch.randn(2, 37, 45, 128, generator=g)
    w = torch.randn(16, 128, generator=g) * 128 ** -0.5
    lw = 1.0 + 0.1 * torch.randn(128, generator=g)
    with torch.no_grad():
        got = pair_bias_projection_hip(z.to(DEV, dtype), lw.to(DEV, dtype), w.to(DEV, dtype), 1e-5)
    assert got.shape == (2, 16, 37, 45) and got.stride(-1) == 1 and got.stride(-2) % 8 == 0
    want = O.pair_bias_projection(to_np(z.to(dtype)), to_np(lw.to(dtype)), to_np(w.to(dtype)), 1e-5)
    tol = {torch.bfloat16: 1e-2, torch.float16: 2e-3, torch.float32: 1e-5}[dtype]
    assert O.rel_fro(to_np(got), want) <= tol


def test_af3_pairformer_size_bf16():
    """384 tokens, 16 heads of 24, c_s = 384, c_z = 128, a ragged key mask."""
    B, M, H, U, DH, Zc = 1, 1, 16, 384, 24, 128
    t = apb_inputs(B, M, H, U, U, DH, Zc, seed=21, biases=True)
    mask = apb_key_mask(B, U, seed=23, frac_keep=0.85)
    out, pz = apb(**on_gpu(t, torch.bfloat16), mask=mask.to(DEV), return_z_proj=True)
    q = {k: v.to(torch.bfloat16).float() for k, v in t.items()}
    want, want_pz = oracle(q, mask=mask, return_z_proj=True)
    tol = ATTENTION_PAIR_BIAS_TOL[torch.bfloat16, "ieee"]
    assert_close_to_oracle("pz", pz, want_pz, tol, rel_fro_max=1e-2)
    assert_close_to_oracle("out", out, want, tol, rel_fro_max=1e-2)


# ---- structural (exact) cases -------------------------------------------------------------
DTYPES = pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                                 ids=["fp32", "bf16", "fp16"])


@DTYPES
def test_masked_keys_are_ignored(dtype):
    B, M, H, U, DH, Zc = 1, 1, 4, 32, 16, 16
    t = on_gpu(apb_inputs(B, M, H, U, U, DH, Zc, seed=3), dtype)
    mask = apb_key_mask(B, U, seed=5, frac_keep=0.7, device=DEV)
    dropped = (mask == 0).reshape(B, 1, U, 1)
    assert dropped.any()
    noise = torch.randn(t["v"].shape, generator=gen(7)).to(DEV, dtype) * 1e3
    perturbed = {**t, "v": torch.where(dropped, t["v"] + noise, t["v"])}
    out, _ = apb(**t, mask=mask)
    out_p, _ = apb(**perturbed, mask=mask)
    torch.testing.assert_close(out, out_p, rtol=0, atol=0)
    assert not torch.allclose(apb(**t)[0], apb(**perturbed)[0])


@DTYPES
def test_masked_logits_are_suppressed(dtype):
    B, M, H, U, DH, Zc = 1, 1, 4, 32, 16, 16
    t = on_gpu(apb_inputs(B, M, H, U, U, DH, Zc, seed=3), dtype)
    mask = apb_key_mask(B, U, seed=5, frac_keep=0.7, device=DEV)
    keyd = (mask == 0).reshape(B, 1, U, 1)
    zd = (mask == 0).reshape(B, 1, U, 1)
    g = gen(11)
    perturbed = {**t, "k": torch.where(keyd, t["k"] + torch.randn(t["k"].shape, generator=g).to(DEV, dtype), t["k"]),
                 "z": torch.where(zd, t["z"] + torch.randn(t["z"].shape, generator=g).to(DEV, dtype), t["z"])}
    torch.testing.assert_close(apb(**t, mask=mask)[0], apb(**perturbed, mask=mask)[0], rtol=0, atol=0)


@DTYPES
@pytest.mark.parametrize("multiplicity", [1, 3], ids=["m1", "m3"])
def test_cached_pair_bias(dtype, multiplicity):
    B, M, H, U, DH, Zc = 2, multiplicity, 4, 32, 16, 16
    t = on_gpu(apb_inputs(B, M, H, U, U, DH, Zc, seed=31), dtype)
    mask = apb_key_mask(B, U, seed=55, frac_keep=0.6, device=DEV)
    full, projected = apb(**t, mask=mask, return_z_proj=True)
    cached, again = apb(**{**t, "z": projected}, mask=mask, z_is_projected=True, return_z_proj=True)
    assert projected.shape == (B, H, U, U) and again is not None
    torch.testing.assert_close(full, cached, rtol=0, atol=0)
    _, unmasked = apb(**t, return_z_proj=True)
    torch.testing.assert_close(projected, unmasked, rtol=0, atol=0)


@pytest.mark.parametrize("multiplicity", [1, 3], ids=["m1", "m3"])
def test_per_copy_mask(multiplicity):
    B, M, H, U, DH, Zc = 2, multiplicity, 4, 32, 16, 16
    t = on_gpu(apb_inputs(B, M, H, U, U, DH, Zc, seed=41), torch.float32)
    per_copy = apb_key_mask(B * M, U, seed=43, frac_keep=0.6)
    out, _ = apb(**t, mask=per_copy.to(DEV))
    want, _ = oracle({k: v.cpu() for k, v in t.items()}, mask=per_copy)
    assert_close_to_oracle("out", out, want, ATTENTION_PAIR_BIAS_TOL[torch.float32, "ieee"])


def test_inf_argument_is_honoured():
    B, M, H, U, DH, Zc = 1, 1, 4, 32, 16, 16
    t = on_gpu(apb_inputs(B, M, H, U, U, DH, Zc, seed=57), torch.float32)
    mask = apb_key_mask(B, U, seed=59, frac_keep=0.5)
    suppressed, _ = apb(**t, mask=mask.to(DEV), inf=1e6)
    barely, _ = apb(**t, mask=mask.to(DEV), inf=1.0)
    assert not torch.allclose(suppressed, barely, rtol=1e-2, atol=1e-2)
    want, _ = oracle({k: v.cpu() for k, v in t.items()}, mask=mask, inf=1.0)
    assert_close_to_oracle("inf=1", barely, want, ATTENTION_PAIR_BIAS_TOL[torch.float32, "ieee"])


@DTYPES
def test_fully_masked_rows(dtype):
    B, M, H, U, DH, Zc = 1, 1, 4, 32, 16, 16
    t = on_gpu(apb_inputs(B, M, H, U, U, DH, Zc, seed=61), dtype)
    mask = torch.zeros(B, U, device=DEV, dtype=dtype)
    out, projected = apb(**t, mask=mask, return_z_proj=True)
    assert torch.isfinite(out).all() and torch.isfinite(projected).all()


def test_mask_layouts_agree():
    B, M, H, U, DH, Zc = 2, 3, 4, 16, 8, 16
    t = on_gpu(apb_inputs(B, M, H, U, U, DH, Zc, seed=3), torch.float32)
    per_batch = apb_key_mask(B, U, seed=5, frac_keep=0.6, device=DEV)
    per_copy = per_batch.repeat_interleave(M, dim=0)
    torch.testing.assert_close(apb(**t, mask=per_batch)[0], apb(**t, mask=per_copy)[0], rtol=0, atol=0)


def test_pair_bias_is_shared_across_the_multiplicity_axis():
    B, M, H, U, DH, Zc = 2, 3, 4, 16, 8, 16
    t = on_gpu(apb_inputs(B, M, H, U, U, DH, Zc, seed=7), torch.float32)
    for key in ("s", "q", "k", "v"):
        grouped = t[key].reshape(B, M, *t[key].shape[1:])
        t[key] = grouped[:, :1].expand_as(grouped).reshape(t[key].shape).contiguous()
    out = apb(**t)[0].reshape(B, M, U, H * DH)
    for copy in range(1, M):
        torch.testing.assert_close(out[:, copy], out[:, 0], rtol=0, atol=0)
    assert not torch.equal(out[0, 0], out[1, 0])


def test_unequal_query_and_key_counts_take_the_torch_path():
    """U != V has no square-attention kernel: the differentiable torch path answers."""
    B, M, H, U, V, DH, Zc = 1, 2, 2, 12, 20, 8, 8
    t = apb_inputs(B, M, H, U, V, DH, Zc, seed=71)
    out, _ = apb(**on_gpu(t, torch.float32))
    want, _ = oracle(t)
    assert_close_to_oracle("out", out, want, ATTENTION_PAIR_BIAS_TOL[torch.float32, "ieee"])


def test_grad_calls_take_the_torch_path():
    from geometric_nn_ops_torch.triangle import attention_pair_bias

    t = on_gpu(apb_inputs(1, 1, 2, 16, 16, 8, 8, seed=73), torch.float32)
    t["q"].requires_grad_(True)
    out, _ = attention_pair_bias(**t)
    out.sum().backward()
    assert t["q"].grad is not None and torch.isfinite(t["q"].grad).all()
