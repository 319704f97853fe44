"""The cuequivariance_ops_torch shim (geometric-nn-ops_amd/cuequivariance_ops_torch), after
the reference's hipequivariance_ops_torch/tests: import surface and deep-imported constants
(test_import_compat.py), the installation guard, cueq's triangle-attention layout and rank,
the trimul precision policy (test_precision_check.py) and the attention_pair_bias argument
mapping. cuequivariance_torch itself is not installed here, so the shim's functions are
called directly; the GPU cases check they give exactly what the public ops give."""

import importlib
import warnings
from unittest import mock

import pytest
import torch

import cuequivariance_ops_torch as cueq
from cuequivariance_ops_torch import _guard
from geometric_nn_ops_torch.triangle import attention_pair_bias, triangle_attention, triangle_multiplicative_update
from helpers import apb_inputs, apb_key_mask, pair_input, trimul_weights

# the package rebinds the submodule names to the functions, as cueq's callers expect
tmu_module = importlib.import_module("cuequivariance_ops_torch.triangle_multiplicative_update")


class fp32_precision:
    def __init__(self, value):
        self.value = value

    def __enter__(self):
        self.old = torch.backends.cuda.matmul.fp32_precision
        torch.backends.cuda.matmul.fp32_precision = self.value

    def __exit__(self, *exc):
        torch.backends.cuda.matmul.fp32_precision = self.old


def test_import_surface():
    assert set(cueq.__all__) == {"attention_pair_bias", "triangle_attention", "triangle_multiplicative_update",
                                 "TriMulPrecision"}
    from cuequivariance_ops_torch.attention_pair_bias_torch import CUEQ_ATTENTION_PAIR_BIAS_FALLBACK_THRESHOLD
    from cuequivariance_ops_torch.triangle_attention import CUEQ_TRIATTN_FALLBACK_THRESHOLD
    from cuequivariance_ops_torch.triangle_multiplicative_update import CUEQ_TRIMUL_FALLBACK_THRESHOLD

    assert CUEQ_TRIATTN_FALLBACK_THRESHOLD > 0 and CUEQ_TRIMUL_FALLBACK_THRESHOLD > 0
    assert CUEQ_ATTENTION_PAIR_BIAS_FALLBACK_THRESHOLD > 1 << 30
    assert [m.value for m in cueq.TriMulPrecision] == [-1, 0, 1, 2, 3]


def test_guard_rejects_the_real_wheel_and_warns_on_version():
    with mock.patch.object(_guard, "installed", return_value={"cuequivariance-ops-torch-cu12", "torch"}):
        with pytest.raises(RuntimeError, match="cuequivariance-ops-torch-cu12"):
            _guard.check()
    with mock.patch.object(_guard, "installed", return_value={"torch"}), \
            mock.patch.object(_guard.metadata, "version", return_value="0.8.0"):
        with pytest.warns(RuntimeWarning, match="0.9.1"):
            _guard.check()
    with mock.patch.object(_guard, "installed", return_value={"torch"}), \
            mock.patch.object(_guard.metadata, "version", return_value="0.9.1"), warnings.catch_warnings():
        warnings.simplefilter("error")
        _guard.check()


def _cueq_attention_inputs(device="cpu", dtype=torch.float32, batch=True):
    g = torch.Generator().manual_seed(0)
    B, N, H, S, D = 1, 3, 4, 24, 16
    shape = (B, N, H, S, D) if batch else (N, H, S, D)
    q, k, v = (torch.randn(*shape, generator=g).to(device, dtype) for _ in range(3))
    bias = (0.3 * torch.randn(1, 1, H, S, S, generator=g)).to(device, dtype)
    mask = torch.rand(*((B,) if batch else ()), N, 1, 1, S, generator=g) < 0.8
    mask[..., 0] = True
    return q, k, v, bias, mask.to(device)


def test_triangle_attention_layout_and_rank():
    q, k, v, bias, mask = _cueq_attention_inputs()
    out = cueq.triangle_attention(q, k, v, bias, mask=mask.float(), scale=0.3)
    swap = lambda t: t.transpose(-2, -3)  # noqa: E731
    want = swap(triangle_attention(swap(q), swap(k), swap(v), bias, mask, 0.3))
    assert out.shape == q.shape and torch.equal(out, want)
    qb, kb, vb, bb, mb = _cueq_attention_inputs(batch=False)
    out4 = cueq.triangle_attention(qb, kb, vb, bb[0], mask=mb)
    assert out4.dim() == 5 and out4.shape[0] == 1


def _aux_oracle(q, k, bias, mask, scale):
    """cueq-layout (lse, max) from oracle.triangle_attention_lse_max (canonical layout)."""
    import numpy as np

    from oracle import triangle_oracle as O

    sw = lambda t: np.swapaxes(t.double().cpu().numpy(), -2, -3)  # noqa: E731
    lse, mx = O.triangle_attention_lse_max(sw(q), sw(k), bias.double().cpu().numpy(),
                                           None if mask is None else mask.cpu().numpy(), scale)
    return lse[..., None], mx[..., None]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["fp32", "fp64"])
def test_triangle_attention_return_aux_cpu(dtype):
    """(out, lse, max) with lse / max the log-sum-exp and maximum of each query's logits,
    (B, N, H, S, 1) fp32, against the oracle; out is the plain call's output."""
    import numpy as np

    q, k, v, bias, mask = (t if t.dtype == torch.bool else t.to(dtype) for t in _cueq_attention_inputs())
    out, lse, mx = cueq.triangle_attention(q, k, v, bias, mask=mask, scale=0.3, return_aux=True)
    assert torch.equal(out, cueq.triangle_attention(q, k, v, bias, mask=mask, scale=0.3))
    B, N, H, S, _ = q.shape
    assert lse.shape == mx.shape == (B, N, H, S, 1) and lse.dtype == mx.dtype == torch.float32
    want_lse, want_mx = _aux_oracle(q, k, bias, mask, 0.3)
    np.testing.assert_allclose(lse.numpy(), want_lse, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(mx.numpy(), want_mx, rtol=1e-5, atol=1e-5)
    assert (lse >= mx).all()


def test_trimul_precision_policy():
    check = tmu_module.check_precision
    with fp32_precision("ieee"), warnings.catch_warnings():
        warnings.simplefilter("error")
        for ok in (None, "none", "DEFAULT", cueq.TriMulPrecision.NONE, 0, "ieee", cueq.TriMulPrecision.IEEE, 3):
            check(ok)
    with fp32_precision("ieee"), pytest.warns(UserWarning, match="full fp32"):
        check("tf32")
    with fp32_precision("tf32"):
        check("tf32")
        check(cueq.TriMulPrecision.TF32)
        with pytest.raises(ValueError, match="fp32_precision"):
            check("ieee")
        with pytest.raises(ValueError):
            check(cueq.TriMulPrecision.TF32x3)


def test_trimul_matches_the_public_op_on_cpu():
    x, mask = pair_input(1, 12, 32, torch.float32, seed=2)
    w = trimul_weights(32, 32, torch.float32, seed=3, biases=True)
    out = cueq.triangle_multiplicative_update(x, "incoming", mask, precision="default", **w)
    assert torch.equal(out, triangle_multiplicative_update(x, "incoming", mask, **w))


def test_attention_pair_bias_argument_mapping():
    t = apb_inputs(2, 2, 4, 12, 12, 8, 16, seed=5, biases=True)
    mask = apb_key_mask(2, 12, seed=6, frac_keep=0.6)
    kw = dict(mask=mask, num_heads=4, w_proj_z=t["proj_z_weight"], w_proj_g=t["proj_g_weight"],
              w_proj_o=t["proj_o_weight"], w_ln_z=t["ln_z_weight"], b_proj_g=t["proj_g_bias"],
              b_proj_o=t["proj_o_bias"])
    out, pz = cueq.attention_pair_bias(t["s"], t["q"], t["k"], t["v"], t["z"], **kw)
    want, want_pz = attention_pair_bias(t["s"], t["q"], t["k"], t["v"], t["z"], proj_g_weight=t["proj_g_weight"],
                                        proj_o_weight=t["proj_o_weight"], proj_z_weight=t["proj_z_weight"],
                                        ln_z_weight=t["ln_z_weight"], proj_g_bias=t["proj_g_bias"],
                                        proj_o_bias=t["proj_o_bias"], mask=mask, inf=1e6, return_z_proj=True)
    assert torch.equal(out, want) and torch.equal(pz, want_pz)
    with pytest.warns(UserWarning, match="b_ln_z is ignored"):
        cueq.attention_pair_bias(t["s"], t["q"], t["k"], t["v"], t["z"], **kw, b_ln_z=torch.ones(16))
    with pytest.raises(ValueError, match="num_heads=3"):
        cueq.attention_pair_bias(t["s"], t["q"], t["k"], t["v"], t["z"], **{**kw, "num_heads": 3})
    cached, _ = cueq.attention_pair_bias(t["s"], t["q"], t["k"], t["v"], pz, **kw, is_cached_z_proj=True)
    assert torch.equal(cached, out)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
def test_triangle_attention_return_aux_gpu(dtype):
    """The HIP forward's lse and exact row maximum (row kernel for 16-bit, tiled kernel for
    fp32) against the fp64 oracle; the output equals the plain call's, also under autograd."""
    from helpers import assert_close_to_oracle, Tolerance

    q, k, v, bias, mask = _cueq_attention_inputs("cuda", dtype)
    with torch.no_grad():
        out, lse, mx = cueq.triangle_attention(q, k, v, bias, mask=mask, scale=0.3, return_aux=True)
        assert torch.equal(out, cueq.triangle_attention(q, k, v, bias, mask=mask, scale=0.3))
    want_lse, want_mx = _aux_oracle(q, k, bias, mask, 0.3)
    tol = Tolerance(1 - 1e-5, 5e-3 if dtype != torch.float32 else 1e-5)
    assert_close_to_oracle("lse", lse, want_lse, tol)
    assert_close_to_oracle("max", mx, want_mx, tol)
    if dtype != torch.float32:
        qg = q.detach().requires_grad_()
        out2, lse2, _ = cueq.triangle_attention(qg, k, v, bias, mask=mask, scale=0.3, return_aux=True)
        assert torch.equal(out2.detach(), out) and torch.equal(lse2, lse)
        out2.float().sum().backward()
        assert qg.grad is not None and torch.isfinite(qg.grad).all()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("jump", [0.0, 25.0], ids=["plain", "hot_later_keys"])
def test_return_aux_is_one_forward(dtype, jump):
    """return_aux=True on the HIP path is a single forward that writes o, lse and the exact
    row maximum; o is bit-identical to the plain call. With keys in later 64-key tiles whose
    logits lie `jump` above the first tile's (the row kernel measures its probabilities
    against the first tile's maximum), lse and max still match the oracle."""
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as hip
    from helpers import Tolerance, assert_close_to_oracle

    g = torch.Generator().manual_seed(5)
    B, N, H, S, D = 1, 2, 4, 200, 32
    q, k, v = (torch.randn(B, N, H, S, D, generator=g) for _ in range(3))
    bias = 0.5 * torch.randn(1, 1, H, S, S, generator=g)
    bias[..., [140, 190]] += jump
    mask = torch.rand(B, N, 1, 1, S, generator=g) < 0.8
    mask[..., 0] = True
    q, k, v, bias, mask = (t.to("cuda", dtype) if t.is_floating_point() else t.to("cuda")
                           for t in (q, k, v, bias, mask))
    with torch.no_grad():
        plain = cueq.triangle_attention(q, k, v, bias, mask=mask)
        with mock.patch.object(hip, "triangle_attention_hip", wraps=hip.triangle_attention_hip) as spy:
            out, lse, mx = cueq.triangle_attention(q, k, v, bias, mask=mask, return_aux=True)
    assert spy.call_count == 1
    assert torch.equal(out, plain) and torch.isfinite(out).all()
    want_lse, want_mx = _aux_oracle(q, k, bias, mask, D**-0.5)
    tol = Tolerance(1 - 1e-5, 5e-3)
    assert_close_to_oracle("lse", lse, want_lse, tol)
    assert_close_to_oracle("max", mx, want_mx, tol)


@pytest.mark.gpu
def test_shim_runs_the_hip_kernels_exactly():
    q, k, v, bias, mask = _cueq_attention_inputs("cuda", torch.bfloat16)
    swap = lambda t: t.transpose(-2, -3)  # noqa: E731
    with torch.no_grad():
        out = cueq.triangle_attention(q, k, v, bias, mask=mask)
        want = swap(triangle_attention(swap(q), swap(k), swap(v), bias, mask))
    assert torch.equal(out, want)
    x, m = pair_input(1, 40, 64, torch.bfloat16, seed=2, device="cuda")
    w = trimul_weights(64, 64, torch.bfloat16, seed=3, device="cuda")
    with torch.no_grad():
        assert torch.equal(cueq.triangle_multiplicative_update(x, "outgoing", m, **w),
                           triangle_multiplicative_update(x, "outgoing", m, **w))
    t = {k_: v_.to("cuda", torch.bfloat16) for k_, v_ in apb_inputs(1, 2, 4, 32, 32, 16, 16, seed=9).items()}
    with torch.no_grad():
        out, pz = cueq.attention_pair_bias(t["s"], t["q"], t["k"], t["v"], t["z"], None, 4, t["proj_z_weight"],
                                           t["proj_g_weight"], t["proj_o_weight"], t["ln_z_weight"])
        want, want_pz = attention_pair_bias(t["s"], t["q"], t["k"], t["v"], t["z"],
                                            proj_g_weight=t["proj_g_weight"], proj_o_weight=t["proj_o_weight"],
                                            proj_z_weight=t["proj_z_weight"], ln_z_weight=t["ln_z_weight"],
                                            inf=1e6, return_z_proj=True)
    assert torch.equal(out, want) and torch.equal(pz, want_pz)
