"""Public API on a CPU-only host: signatures, normalisation, dispatch and the differentiable
torch path (reference tests/test_trimul.py:442-525, tests/test_triangle_attention.py:303-426,
tests/test_precision.py:43-103)."""

import inspect
from unittest import mock

import numpy as np
import pytest
import torch

from geometric_nn_ops_torch import _precision
from geometric_nn_ops_torch.triangle import triangle_attention, triangle_multiplicative_update
from geometric_nn_ops_torch.triangle import _trimul, _triattn
from geometric_nn_ops_torch.triangle._kernels import trimul as _kt
from geometric_nn_ops_torch.triangle._masking import mask_val, masked_key_bias, rounded_mask_value
from helpers import attention_inputs, key_mask, np_weights, pair_input, to_np, trimul_weights
from oracle import triangle_oracle as O


def test_signatures_match_the_reference():
    """Parameter names, order and defaults of the reference's public ops
    (_triattn.py:23-32, _trimul.py:39-56)."""
    sa = inspect.signature(triangle_attention)
    assert list(sa.parameters) == ["q", "k", "v", "bias", "mask", "scale", "dynamic", "use_exp2"]
    assert [sa.parameters[n].default for n in ("bias", "mask", "scale", "dynamic", "use_exp2")] == [
        None, None, None, False, False]
    st = inspect.signature(triangle_multiplicative_update)
    assert list(st.parameters) == [
        "x", "direction", "mask", "norm_in_weight", "norm_in_bias", "p_in_weight", "p_in_bias",
        "g_in_weight", "g_in_bias", "norm_out_weight", "norm_out_bias", "p_out_weight", "p_out_bias",
        "g_out_weight", "g_out_bias", "eps"]
    assert st.parameters["direction"].default == "outgoing" and st.parameters["eps"].default == 1e-5


# --------------------------------------------------------------------------------- masking
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_mask_val_is_representable(dtype):
    assert torch.tensor(-mask_val(dtype), dtype=dtype).isfinite()


def test_rounded_mask_value():
    assert rounded_mask_value(torch.float32) == -1e9
    assert rounded_mask_value(torch.float16) == -32752.0
    bf = rounded_mask_value(torch.bfloat16)
    assert bf == float(torch.tensor(-1e9).bfloat16().float()) and bf != -1e9
    b = masked_key_bias(torch.tensor([True, False]), torch.float32)
    assert b[0].item() == 0 and not torch.signbit(b[0]) and b[1].item() == -1e9


# ------------------------------------------------------------------------------- precision
@pytest.mark.parametrize(("allowed", "expected"), [
    (("tf32", "tf32x3", "ieee", "bf16x3", "bf16x6"), "tf32"),
    (("ieee", "bf16x3", "bf16x6"), "bf16x3"),
    (("ieee",), "ieee"),
])
def test_tf32_resolution(allowed, expected):
    assert _precision.resolve("tf32", allowed) == expected
    assert _precision.resolve("ieee", allowed) == "ieee"


def test_precision_errors_and_torch_setting():
    with pytest.raises(ValueError, match="unknown precision"):
        _precision.resolve("bf16", ("ieee",))
    with pytest.raises(RuntimeError, match="supports none of"):
        _precision.resolve("tf32", ("bf16x6",))
    prev = torch.backends.cuda.matmul.fp32_precision
    try:
        torch.backends.cuda.matmul.fp32_precision = "tf32"
        assert _precision.matmul_precision(fp32_operands=True) == "bf16x3"
        assert _precision.matmul_precision(fp32_operands=False) == "ieee"
        torch.backends.cuda.matmul.fp32_precision = "ieee"
        assert _precision.matmul_precision(fp32_operands=True) == "ieee"
    finally:
        torch.backends.cuda.matmul.fp32_precision = prev


# ------------------------------------------------------------------------ attention on CPU
def _attn_oracle(t, mask=None, scale=None):
    return O.triangle_attention(to_np(t["q"]), to_np(t["k"]), to_np(t["v"]), to_np(t["bias"]),
                                None if mask is None else mask.numpy(), scale)


def test_attention_cpu_matches_oracle_and_shapes():
    t = attention_inputs(1, 2, 16, 2, 8, torch.float64, seed=3)
    mask = key_mask(1, 2, 16, seed=1)
    want = _attn_oracle(t, mask)
    np.testing.assert_allclose(to_np(triangle_attention(**t, mask=mask)), want, rtol=1e-12, atol=1e-12)
    # 4D input, 4D bias, lower-rank masks, 6D input
    un = {k: v[0] for k, v in t.items()}
    out4 = triangle_attention(un["q"], un["k"], un["v"], t["bias"][:, 0], mask)
    assert out4.shape == un["q"].shape
    np.testing.assert_allclose(to_np(out4), want[0], rtol=1e-12, atol=1e-12)
    for rank in (4, 3):
        lower = mask[(0,) * (5 - rank)]
        explicit = lower.expand_as(mask).contiguous()
        np.testing.assert_allclose(to_np(triangle_attention(**t, mask=lower)), _attn_oracle(t, explicit),
                                   rtol=1e-12, atol=1e-12)
    six = {k: v.expand(2, *v.shape).reshape(2, 1, *v.shape[1:]) for k, v in t.items()}
    out6 = triangle_attention(six["q"], six["k"], six["v"], six["bias"])
    assert out6.shape == six["q"].shape


def test_attention_rejects_non_bool_mask():
    t = attention_inputs(1, 1, 8, 2, 8, torch.float32)
    with pytest.raises(ValueError, match="mask must be bool"):
        triangle_attention(**t, mask=key_mask(1, 1, 8).float())


def test_attention_cpu_is_differentiable():
    t = attention_inputs(1, 2, 8, 2, 8, torch.float32, seed=2)
    t = {k: v.requires_grad_() for k, v in t.items()}
    triangle_attention(**t, mask=key_mask(1, 2, 8)).sum().backward()
    assert all(v.grad is not None and torch.isfinite(v.grad).all() for v in t.values())


def test_attention_dispatch_on_cpu():
    t = attention_inputs(1, 1, 8, 2, 8, torch.float32)
    assert _triattn._needs_torch_path(t["q"], t["k"], t["v"], t["bias"])


# --------------------------------------------------------------------------- trimul on CPU
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_cpu_matches_oracle(direction):
    w = trimul_weights(16, 12, torch.float64, seed=2, biases=True, ln_random=True)
    x, mask = pair_input((2, 1), 7, 16, torch.float64, seed=5)
    got = triangle_multiplicative_update(x, direction, mask[0, 0], **w)
    want = O.trimul(to_np(x), direction, to_np(mask[0, 0]), **np_weights(w))
    np.testing.assert_allclose(to_np(got), want, rtol=1e-11, atol=1e-11)


def test_trimul_rejects_bad_direction():
    w = trimul_weights(16, 16, torch.float32)
    x, mask = pair_input(1, 6, 16, torch.float32)
    with pytest.raises(ValueError, match="direction must be one of"):
        triangle_multiplicative_update(x, "outgoin", mask, **w)


def test_trimul_cpu_is_differentiable():
    """Reference test_trimul.py:507-525: gradients reach x and every parameter."""
    w = trimul_weights(16, 12, torch.float32, seed=2, biases=True)
    w = {k: v.requires_grad_() for k, v in w.items()}
    x, _ = pair_input((), 8, 16, torch.float32, seed=49)
    x.requires_grad_()
    triangle_multiplicative_update(x, "outgoing", torch.ones(8, 8), **w).sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    for key, weight in w.items():
        assert weight.grad is not None, f"{key} received no gradient"


@pytest.mark.parametrize("config", ["cpu", "float64", "input_requires_grad", "weights_require_grad"])
def test_unsupported_configs_use_the_torch_path(config):
    dtype = torch.float64 if config == "float64" else torch.float32
    w = trimul_weights(32, 32, dtype, seed=1)
    x, mask = pair_input(1, 12, 32, dtype, seed=3)
    if config == "input_requires_grad":
        x.requires_grad_()
    if config == "weights_require_grad":
        w = {k: v.requires_grad_() for k, v in w.items()}
    with mock.patch.object(_trimul, "trimul_torch", wraps=_trimul.trimul_torch) as ref, \
            mock.patch.object(_kt, "trimul_hip", wraps=_kt.trimul_hip) as kern:
        triangle_multiplicative_update(x, "outgoing", mask, **w)
    assert ref.called and not kern.called


def test_kernel_dispatch_rule_for_gpu_tensors():
    """The GPU rule, evaluated on a stand-in tensor that reports is_cuda: kernels (forward,
    and the HIP backward when gradients are needed) unless the mask requires grad or the
    channel counts are outside the kernels' tiling."""
    class FakeCuda:
        is_cuda = True
        dtype = torch.bfloat16
        requires_grad = False
        shape = (1, 8, 8, 128)

        def dim(self):
            return 4

    w = {"p_in_weight": torch.zeros(256, 128)}
    assert not _trimul._needs_torch_path(FakeCuda(), w.items())
    assert not _trimul._needs_grad(FakeCuda(), w.items())
    # gradients go to the HIP forward + backward, unless the mask itself requires grad
    w_req = {"p_in_weight": torch.zeros(256, 128, requires_grad=True)}
    assert not _trimul._needs_torch_path(FakeCuda(), w_req.items())
    assert _trimul._needs_grad(FakeCuda(), w_req.items())
    assert _trimul._needs_torch_path(FakeCuda(), w_req.items(), torch.ones(8, 8, requires_grad=True))
    with torch.no_grad():
        assert not _trimul._needs_grad(FakeCuda(), w_req.items())
        assert not _trimul._needs_torch_path(FakeCuda(), w_req.items(), torch.ones(8, 8, requires_grad=True))
    # c_hidden = 48 (not a multiple of 32): the forward pads it, the backward does not
    assert not _trimul._needs_torch_path(FakeCuda(), {"p_in_weight": torch.zeros(96, 128)}.items())
    assert _trimul._needs_torch_path(FakeCuda(), {"p_in_weight": torch.zeros(96, 128, requires_grad=True)}.items())
    # widths above the fused tiles: c_hidden = 544 (a multiple of 32) takes the composed wide
    # forward without gradients and the torch path with them; c_hidden = 520 the torch path
    assert not _trimul._needs_torch_path(FakeCuda(), {"p_in_weight": torch.zeros(1088, 128)}.items())
    assert _trimul._needs_torch_path(FakeCuda(), {"p_in_weight": torch.zeros(1088, 128, requires_grad=True)}.items())
    assert _trimul._needs_torch_path(FakeCuda(), {"p_in_weight": torch.zeros(1040, 128)}.items())


def test_operators_have_fake_implementations():
    """The gnn_amd operators trace under FakeTensorMode without a GPU or the HIP library
    (what torch.compile relies on): shapes and dtypes of the results."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    import geometric_nn_ops_torch._ops  # noqa: F401  (registers the operators)

    with FakeTensorMode():
        q = torch.empty(1, 3, 16, 4, 32, dtype=torch.bfloat16)
        o = torch.ops.gnn_amd.triangle_attention_fwd(q, q, q, None, None, None)
        assert o.shape == q.shape and o.dtype == q.dtype
        x = torch.empty(2, 16, 16, 64, dtype=torch.float16)
        pw, ow, gw = torch.empty(64, 64, dtype=x.dtype), torch.empty(64, 32, dtype=x.dtype), torch.empty(64, 64, dtype=x.dtype)
        out = torch.ops.gnn_amd.trimul_fwd(x, "outgoing", None, None, None, pw, None, pw, None, None, None, ow, None,
                                           gw, None, 1e-5)
        assert out.shape == x.shape and out.dtype == x.dtype


def test_fused_gate_needs_one_s_token_per_o_token():
    """The fused gate / output projection takes its token count from s; an s that would only
    broadcast against o (torch's o * g accepts it) keeps the F.linear path."""
    from geometric_nn_ops_torch.triangle._kernels import attention_pair_bias as K

    o, gw, ow = torch.empty(3, 40, 64), torch.empty(64, 96), torch.empty(32, 64)
    assert K.gate_out_supported(torch.empty(3, 40, 96), o, gw, ow)
    assert not K.gate_out_supported(torch.empty(1, 40, 96), o, gw, ow)
    assert not K.gate_out_supported(torch.empty(40, 96), o, gw, ow)


def test_eager_fast_path_accepts_module_parameters():
    """Module weights are nn.Parameter: a plain eager call with them still runs the operator's
    implementation directly; tensor subclasses and dispatch modes go through the operator."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from geometric_nn_ops_torch import _ops

    t = torch.ones(3)
    lin = torch.nn.Linear(4, 4)
    assert _ops.eager_ok(t, None, lin.weight, lin.bias)

    class Sub(torch.Tensor):
        pass

    assert not _ops.eager_ok(t, t.as_subclass(Sub))
    with FakeTensorMode():
        assert not _ops.eager_ok(torch.empty(3))



# ---------------------------------------------------------------- attention with pair bias
def test_attention_pair_bias_signature_matches_the_reference():
    """_attention_pair_bias.py:11-30: positional s, q, k, v, z, then keyword-only options."""
    from geometric_nn_ops_torch.triangle import attention_pair_bias

    sig = inspect.signature(attention_pair_bias)
    names = list(sig.parameters)
    assert names[:5] == ["s", "q", "k", "v", "z"]
    assert names[5:] == ["proj_g_weight", "proj_o_weight", "proj_z_weight", "ln_z_weight", "proj_g_bias",
                         "proj_o_bias", "mask", "scale", "inf", "eps", "z_is_projected", "return_z_proj"]
    assert all(sig.parameters[n].kind is inspect.Parameter.KEYWORD_ONLY for n in names[5:])
    assert sig.parameters["eps"].default == 1e-5 and sig.parameters["inf"].default is None


@pytest.mark.parametrize("mask_kind", [None, "batch", "copy"])
def test_attention_pair_bias_cpu_matches_oracle(mask_kind):
    from geometric_nn_ops_torch.triangle import attention_pair_bias
    from helpers import apb_inputs, apb_key_mask

    t = apb_inputs(2, 2, 3, 10, 10, 8, 16, seed=4, biases=True)
    mask = None if mask_kind is None else apb_key_mask(2 if mask_kind == "batch" else 4, 10, seed=6, frac_keep=0.6)
    out, pz = attention_pair_bias(**t, mask=mask, inf=1e6, return_z_proj=True)
    want, want_pz = O.attention_pair_bias(**{k: to_np(v) for k, v in t.items()},
                                          mask=None if mask is None else to_np(mask), inf=1e6, return_z_proj=True)
    assert O.rel_fro(to_np(out), want) < 1e-5 and O.rel_fro(to_np(pz), want_pz) < 1e-5
    cached, none = attention_pair_bias(**{**t, "z": pz}, mask=mask, inf=1e6, z_is_projected=True)
    assert none is None and torch.equal(cached, out)


def test_attention_pair_bias_errors():
    from geometric_nn_ops_torch.triangle import attention_pair_bias
    from helpers import apb_inputs

    t = apb_inputs(2, 2, 2, 6, 6, 8, 8, seed=1)
    with pytest.raises(ValueError, match="multiple of z batch"):
        attention_pair_bias(**{**t, "z": torch.randn(3, 6, 6, 8)})
    with pytest.raises(ValueError, match="must be B=2 or BM=4"):
        attention_pair_bias(**t, mask=torch.ones(3, 6))


def test_attention_pair_bias_operator_fake():
    from torch._subclasses.fake_tensor import FakeTensorMode

    import geometric_nn_ops_torch._ops  # noqa: F401

    with FakeTensorMode():
        s = torch.empty(6, 16, 32, dtype=torch.bfloat16)
        q = torch.empty(6, 4, 16, 8, dtype=torch.bfloat16)
        z = torch.empty(2, 16, 16, 24, dtype=torch.bfloat16)
        w = torch.empty(32, 32, dtype=torch.bfloat16)
        out, pz = torch.ops.gnn_amd.attention_pair_bias_fwd(s, q, q, q, z, w, w, torch.empty(4, 24, dtype=s.dtype),
                                                             None, None, None, None, None, None, 1e-5, False)
        assert out.shape == (6, 16, 32) and pz.shape == (2, 4, 16, 16)


def test_dbias_splits_follow_the_measured_optimum():
    """The pair-bias gradient's N_seq range count: within [1, min(N_seq, 64)], and at the
    shapes timed on an MI355X (fwd + bwd, bf16, D = 32, B = 1, H = 4) a count that measured
    at least as fast as the alternatives: N = 256: 16 ranges (0.305-0.312 ms; 32: 0.320-0.322);
    N = 384: 7 (0.508-0.568; 15: 0.539-0.561); N = 512: 4 (1.024; 8: 1.021-1.045);
    N = 768: 7 (3.117-3.160; 16: 3.151-3.167; 32: 3.25-3.30; 64: 3.45)."""
    from geometric_nn_ops_torch.triangle._kernels.triangle_attention import dbias_splits

    assert dbias_splits(1, 256, 256, 4) == 16
    assert dbias_splits(1, 384, 384, 4) == 7
    assert dbias_splits(1, 512, 512, 4) == 4
    assert dbias_splits(1, 768, 768, 4) == 7
    for B, S, N, H in ((1, 1, 32, 1), (1, 3, 72, 2), (2, 100, 300, 8), (1, 2048, 2048, 4), (4, 64, 64, 16)):
        assert 1 <= dbias_splits(B, S, N, H) <= min(S, 64)
