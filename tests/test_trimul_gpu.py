"""HIP triangle multiplicative update vs the CPU oracle, per stage and end to end.

Structural cases restate AMDResearch/geometric-nn-ops tests/test_trimul.py:70-404; accuracy
uses its tolerance table (testutil/metrics.py:96-101) against the fp64 oracle, plus this
build's rel-Frobenius <= 1e-2 for bf16. BASELINE config C3 (N=512, both directions, last
64 residues padded) runs at full size against the fp64 oracle.
"""

import contextlib
from unittest import mock

import numpy as np
import pytest
import torch

from helpers import (NORTH_STAR_REL_FRO, TRIMUL_TOL, Tolerance, assert_close_to_oracle, gen, np_weights,
                     pair_input, randn, to_np, trimul_weights)
from oracle import triangle_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
DIRECTIONS = pytest.mark.parametrize("direction", ["outgoing", "incoming"])
DTYPE_PRECISION = pytest.mark.parametrize(
    ("dtype", "precision"),
    [(torch.float32, "ieee"), (torch.float32, "tf32"), (torch.bfloat16, "ieee"), (torch.float16, "ieee")],
    ids=["fp32_ieee", "fp32_tf32", "bf16", "fp16"],
)


@contextlib.contextmanager
def matmul_precision(precision):
    prev = torch.backends.cuda.matmul.fp32_precision
    torch.backends.cuda.matmul.fp32_precision = precision
    try:
        yield
    finally:
        torch.backends.cuda.matmul.fp32_precision = prev


def hip(x, direction, mask, w):
    from geometric_nn_ops_torch.triangle._kernels.trimul import trimul_hip

    with torch.no_grad():
        return trimul_hip(x.to(DEV), direction, None if mask is None else mask.to(DEV),
                          **{k: v.to(DEV) for k, v in w.items()})


def oracle(x, direction, mask, w, **kw):
    return O.trimul(to_np(x), direction, None if mask is None else to_np(mask), **np_weights(w), **kw)


# ------------------------------------------------------------------------------- accuracy
@DIRECTIONS
@DTYPE_PRECISION
def test_accuracy(direction, dtype, precision):
    w = trimul_weights(32, 32, dtype, seed=3)
    x, mask = pair_input(1, 32, 32, dtype, seed=4)
    with matmul_precision(precision):
        got = hip(x, direction, mask, w)
    assert_close_to_oracle("out", got, oracle(x, direction, mask, w), TRIMUL_TOL[dtype, precision],
                           rel_fro_max=NORTH_STAR_REL_FRO)


@DIRECTIONS
@pytest.mark.parametrize(("dtype", "precision"),
                         [(torch.bfloat16, "ieee"), (torch.float32, "ieee"), (torch.float32, "tf32")],
                         ids=["bf16", "fp32", "fp32_tf32"])
def test_stages_against_oracle(direction, dtype, precision):
    """Each kernel's output region of the workspace against the oracle's intermediate:
    a, b (channel-major, transposed per channel for 'incoming'; k-blocked for 16-bit types,
    zero in the row padding), g and o. fp32 under 'tf32' takes the projection kernel that
    splits its operands into bf16 halves once (c_z = 64)."""
    from geometric_nn_ops_torch.triangle._kernels import trimul as K

    B, N, C, Ch = 2, 40, 64, 32
    w = trimul_weights(C, Ch, dtype, seed=5, biases=True, ln_random=True)
    x, mask = pair_input(B, N, C, dtype, seed=6)
    wd = {k: v.to(DEV) for k, v in w.items()}
    with torch.no_grad(), matmul_precision(precision):
        args, keep, out, ws, off = K.build_args(x.to(DEV), direction, mask.to(DEV), 1e-5, wd)
        K.run_stage("gnn_trimul_proj", args, x.device if x.is_cuda else torch.device(DEV))
        K.run_stage("gnn_trimul_contract", args, torch.device(DEV))
        K.run_stage("gnn_trimul_out", args, torch.device(DEV))
        torch.cuda.synchronize()
    NP = (N + 31) // 32 * 32
    el = x.element_size()

    def region(i, shape):
        n = int(np.prod(shape))
        return ws[off[i]:off[i] + n * el].view(dtype).reshape(shape)

    st = O.trimul_stages(to_np(x), direction, to_np(mask), **np_weights(w))
    tol = TRIMUL_TOL[dtype, precision]
    def operand(i):
        if dtype == torch.float32:  # row-major [B, Ch, N, NP]
            return region(i, (B, Ch, N, NP))
        # 16-bit: k-blocked [B, Ch, NP / 32, N, 32]
        return region(i, (B, Ch, NP // 32, N, 32)).permute(0, 1, 3, 2, 4).reshape(B, Ch, N, NP)

    a_full, b_full = operand(0), operand(1)
    if dtype != torch.float32:  # the contraction runs K to NP: columns N .. NP-1 must be zero
        assert torch.count_nonzero(a_full[..., N:]) == 0 and torch.count_nonzero(b_full[..., N:]) == 0
    a_cm, b_cm = a_full[..., :N], b_full[..., :N]
    o_cm = region(3, (B, Ch, N, NP))[..., :N]
    perm = (0, 2, 3, 1) if direction == "outgoing" else (0, 3, 2, 1)
    assert_close_to_oracle("a", a_cm.permute(*perm), st["a"], tol)
    assert_close_to_oracle("b", b_cm.permute(*perm), st["b"], tol)
    assert_close_to_oracle("g", region(2, (B, N, N, C)), st["g"], tol)
    assert_close_to_oracle("o", o_cm.permute(0, 2, 3, 1), st["o"], tol)
    assert_close_to_oracle("out", out, st["out"], tol,
                           rel_fro_max=NORTH_STAR_REL_FRO if dtype != torch.float32 else None)


@DIRECTIONS
@pytest.mark.parametrize("shape", [(2, 48, 48, 128), (2, 3, 40, 40, 128)], ids=["batched", "5D"])
def test_batched(direction, shape):
    *batch, N, _, C = shape
    w = trimul_weights(C, C, torch.bfloat16, seed=7)
    x, mask = pair_input(tuple(batch), N, C, torch.bfloat16, seed=11)
    assert_close_to_oracle("out", hip(x, direction, mask, w), oracle(x, direction, mask, w),
                           Tolerance(1 - 1e-4, 1.5e-2), rel_fro_max=NORTH_STAR_REL_FRO)


@DIRECTIONS
@pytest.mark.parametrize(("B", "N", "dtype", "precision"),
                         [(2, 70, torch.bfloat16, "ieee"), (1, 130, torch.float16, "ieee"), (3, 64, torch.bfloat16, "ieee"),
                          (2, 70, torch.float32, "tf32")],
                         ids=["b2_n70_bf16", "b1_n130_fp16", "b3_n64_bf16", "b2_n70_fp32_tf32"])
def test_output_stage_tiles_and_bounds(direction, B, N, dtype, precision):
    """The output stage at C = c_hidden = 128 (a fixed grid of workgroups walking 64-pixel
    tiles with the next tile's o and g in flight, out written by buffer stores whose range
    ends at the tile's last pixel; fp32 under 'tf32' with the operands split into bf16 halves
    once): rows whose last tile is partial, several batches, against the oracle; the stage run
    again into a buffer with a guard region after the output leaves the guard untouched and
    writes the same result."""
    from geometric_nn_ops_torch.triangle._kernels import trimul as K

    C = 128
    w = trimul_weights(C, C, dtype, seed=61, biases=True, ln_random=True)
    x, mask = pair_input(B, N, C, dtype, seed=62)
    wd = {k: v.to(DEV) for k, v in w.items()}
    with torch.no_grad(), matmul_precision(precision):
        args, keep, out, ws, off = K.build_args(x.to(DEV), direction, mask.to(DEV), 1e-5, wd)
        for stage in ("gnn_trimul_proj", "gnn_trimul_contract", "gnn_trimul_out"):
            K.run_stage(stage, args, torch.device(DEV))
        guard = torch.full((out.numel() + 4096,), 7.0, device=DEV, dtype=dtype)
        args.out = guard.data_ptr()
        K.run_stage("gnn_trimul_out", args, torch.device(DEV))
        torch.cuda.synchronize()
    tol = TRIMUL_TOL[torch.float32, "tf32"] if dtype == torch.float32 else Tolerance(1 - 1e-4, 2e-2)
    assert_close_to_oracle("out", out, oracle(x, direction, mask, w), tol,
                           rel_fro_max=None if dtype == torch.float32 else NORTH_STAR_REL_FRO)
    assert torch.equal(guard[:out.numel()].view(out.shape), out)
    assert bool((guard[out.numel():] == 7.0).all())


@DIRECTIONS
@pytest.mark.parametrize("true_length", [32, 48])
def test_block_padded(direction, true_length):
    N, C, batch = 64, 128, 2
    w = trimul_weights(C, C, torch.bfloat16, seed=11)
    x, _ = pair_input(batch, N, C, torch.bfloat16, seed=13)
    g = gen(13)
    mask = torch.zeros(batch, N, N, dtype=torch.bfloat16)
    for i in range(batch):
        live = max(1, true_length - 8 * i)
        mask[i, :live, :live] = (torch.rand(live, live, generator=g) < 0.9).to(torch.bfloat16)
    assert_close_to_oracle("out", hip(x, direction, mask, w), oracle(x, direction, mask, w),
                           Tolerance(1 - 1e-4, 1.5e-2), rel_fro_max=NORTH_STAR_REL_FRO)


@DIRECTIONS
@pytest.mark.parametrize("channels", [64, 96, 128, 256, 320, 512])
def test_channel_widths(direction, channels):
    """64 and 128 take the fixed-width projection kernel, the others the general one (up to
    8 x chunks per thread at 512)."""
    w = trimul_weights(channels, channels, torch.bfloat16, seed=17)
    x, mask = pair_input(1, 24, channels, torch.bfloat16, seed=18)
    assert_close_to_oracle("out", hip(x, direction, mask, w), oracle(x, direction, mask, w),
                           Tolerance(1 - 1e-4, 2e-2),
                           rel_fro_max=NORTH_STAR_REL_FRO)


@DIRECTIONS
@pytest.mark.parametrize("c_z,c_hidden", [(64, 32), (128, 256), (128, 32), (256, 64), (32, 160)])
def test_hidden_differs_from_channels(direction, c_z, c_hidden):
    """c_hidden = 256 gives a wave two projection units (weights reloaded per tile); 32 leaves
    waves idle."""
    w = trimul_weights(c_z, c_hidden, torch.bfloat16, seed=19)
    x, mask = pair_input(1, 24, c_z, torch.bfloat16, seed=20)
    assert_close_to_oracle("out", hip(x, direction, mask, w), oracle(x, direction, mask, w),
                           Tolerance(1 - 1e-4, 2e-2),
                           rel_fro_max=NORTH_STAR_REL_FRO)


@DIRECTIONS
@pytest.mark.parametrize("channels", [64, 128])
def test_fixed_width_fp16(direction, channels):
    w = trimul_weights(channels, channels, torch.float16, seed=21, biases=True)
    x, mask = pair_input(1, 40, channels, torch.float16, seed=22)
    assert_close_to_oracle("out", hip(x, direction, mask, w), oracle(x, direction, mask, w),
                           Tolerance(1 - 1e-4, 1e-2),
                           rel_fro_max=NORTH_STAR_REL_FRO)


@DIRECTIONS
@pytest.mark.parametrize("precision", ["ieee", "tf32"])
@pytest.mark.parametrize("channels", [128, 256])
def test_fp32_channel_widths(direction, precision, channels):
    w = trimul_weights(channels, channels, torch.float32, seed=23, biases=True)
    x, mask = pair_input(1, 24, channels, torch.float32, seed=24)
    with matmul_precision(precision):
        got = hip(x, direction, mask, w)
    assert_close_to_oracle("out", got, oracle(x, direction, mask, w), TRIMUL_TOL[torch.float32, precision])


@DIRECTIONS
@pytest.mark.parametrize("gamma", ["zero", "tiny", "learned"])
def test_layernorm_affine(direction, gamma):
    N, C = 24, 128
    dt = torch.bfloat16
    w = trimul_weights(C, C, dt, seed=19)
    g = gen(23)
    gin, gout = torch.ones(C), torch.ones(C)
    if gamma == "zero":
        gin[0] = gin[5] = 0.0
        gout[3] = 0.0
    elif gamma == "tiny":
        gin[:3] = torch.tensor([1e-2, 1e-3, 1e-4])
        gout[0] = 1e-3
    else:
        gin = torch.randn(C, generator=g) * 0.5 + 1
        gout = torch.randn(C, generator=g) * 0.5 + 1
    w["norm_in_weight"], w["norm_out_weight"] = gin.to(dt), gout.to(dt)
    w["norm_in_bias"] = (torch.randn(C, generator=g) * 0.1).to(dt)
    w["norm_out_bias"] = (torch.randn(C, generator=g) * 0.1).to(dt)
    x, mask = pair_input(1, N, C, dt, seed=20)
    assert_close_to_oracle("out", hip(x, direction, mask, w), oracle(x, direction, mask, w),
                           Tolerance(1 - 1e-4, 2e-2),
                           rel_fro_max=NORTH_STAR_REL_FRO)


def test_none_parameters():
    """LayerNorm weights/biases and projection biases may all be None."""
    w = trimul_weights(32, 32, torch.float32, seed=2)
    w = {k: v for k, v in w.items() if "norm" not in k}
    x, mask = pair_input(1, 20, 32, torch.float32, seed=3)
    for direction in ("outgoing", "incoming"):
        assert_close_to_oracle("out", hip(x, direction, mask, w), oracle(x, direction, mask, w),
                               TRIMUL_TOL[torch.float32, "ieee"])


# ---------------------------------------------------------------------------- structural
@pytest.mark.parametrize("biased", [False, True])
@DIRECTIONS
def test_fully_masked_input(biased, direction):
    N, C = 32, 128
    w = trimul_weights(C, C, torch.float32, seed=3, biases=biased)
    w["norm_out_bias"] = torch.full((C,), 0.25)
    w["g_out_weight"] = torch.zeros(C, C)
    x, _ = pair_input(1, N, C, torch.float32, seed=4)
    out = hip(x, direction, torch.zeros(1, N, N), w)
    torch.testing.assert_close(out, out[:, :1, :1].expand_as(out), rtol=0, atol=1e-6)
    assert out.abs().max() > 0.01


@pytest.mark.parametrize("which", ["p_in_bias", "g_in_bias", "p_out_bias", "g_out_bias"])
@DIRECTIONS
def test_each_projection_bias_contributes(which, direction):
    w = trimul_weights(32, 32, torch.float32, seed=47, biases=True)
    x, mask = pair_input(1, 16, 32, torch.float32, seed=49)
    out = hip(x, direction, mask, w)
    zeroed = hip(x, direction, mask, {**w, which: torch.zeros_like(w[which])})
    assert not torch.allclose(out, zeroed, atol=1e-5)


def test_direction_changes_the_result():
    w = trimul_weights(128, 128, torch.float32, seed=7)
    x, mask = pair_input(1, 32, 128, torch.float32, seed=8)
    assert not torch.allclose(hip(x, "outgoing", mask, w), hip(x, "incoming", mask, w), rtol=1e-2, atol=1e-2)


def test_unknown_direction_is_rejected():
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    w = trimul_weights(32, 32, torch.float32, seed=7)
    x, mask = pair_input(1, 12, 32, torch.float32, seed=8)
    with pytest.raises(ValueError, match="direction must be one of"):
        hip(x, "outgoin", mask, w)
    with pytest.raises(ValueError, match="direction must be one of"):
        triangle_multiplicative_update(x.to(DEV), "outgoin", mask.to(DEV), **{k: v.to(DEV) for k, v in w.items()})


@DIRECTIONS
def test_mask_none_matches_ones(direction):
    w = trimul_weights(32, 32, torch.float32, seed=37)
    x, _ = pair_input(1, 12, 32, torch.float32, seed=38)
    torch.testing.assert_close(hip(x, direction, None, w), hip(x, direction, torch.ones(1, 12, 12), w),
                               rtol=0, atol=0)


@DIRECTIONS
def test_broadcast_mask(direction):
    w = trimul_weights(32, 32, torch.float32, seed=31)
    x, mask = pair_input(2, 12, 32, torch.float32, seed=32)
    out = hip(x, direction, mask[0], w)
    assert out.shape == x.shape
    torch.testing.assert_close(out, hip(x, direction, mask[0].expand(x.shape[:-1]), w), rtol=0, atol=0)


def test_tf32_changes_the_result():
    w = trimul_weights(32, 32, torch.float32, seed=3)
    x, mask = pair_input(1, 32, 32, torch.float32, seed=4)
    with matmul_precision("ieee"):
        full = hip(x, "outgoing", mask, w)
    with matmul_precision("tf32"):
        reduced = hip(x, "outgoing", mask, w)
    assert not torch.equal(full, reduced)


# ------------------------------------------------------------------------------ dispatch
@contextlib.contextmanager
def dispatch_spy():
    from geometric_nn_ops_torch.triangle import _trimul
    from geometric_nn_ops_torch.triangle._kernels import trimul as _kt

    with mock.patch.object(_trimul, "trimul_torch", wraps=_trimul.trimul_torch) as ref, \
            mock.patch.object(_kt, "trimul_hip", wraps=_kt.trimul_hip) as kern:
        yield ref, kern


@pytest.mark.parametrize("no_backward", [torch.no_grad, torch.inference_mode])
def test_no_grad_modes_use_the_kernel(no_backward):
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    w = {k: v.to(DEV).requires_grad_() for k, v in trimul_weights(32, 32, torch.float32, seed=1).items()}
    x, mask = pair_input(1, 12, 32, torch.float32, seed=3)
    x = x.to(DEV).requires_grad_()
    with no_backward(), dispatch_spy() as (ref, kern):
        triangle_multiplicative_update(x, "outgoing", mask.to(DEV), **w)
    assert kern.called and not ref.called


def test_module_parameters_take_the_direct_implementation():
    """Weights held as nn.Parameter (what a module passes) run the operator's implementation
    directly in eager mode, not through the torch.library dispatch, with the same result."""
    from geometric_nn_ops_torch import _ops
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    w = {k: v.to(DEV) for k, v in trimul_weights(32, 32, torch.bfloat16, seed=1).items()}
    params = {k: torch.nn.Parameter(v) for k, v in w.items()}
    x, mask = pair_input(1, 12, 32, torch.bfloat16, seed=3)
    x, mask = x.to(DEV), mask.to(DEV)
    with torch.no_grad():
        want = triangle_multiplicative_update(x, "outgoing", mask, **w)
        with mock.patch.object(_ops, "trimul_fwd", side_effect=AssertionError("dispatched")), \
                mock.patch.object(_ops, "trimul_fwd_impl", wraps=_ops.trimul_fwd_impl) as impl:
            got = triangle_multiplicative_update(x, "outgoing", mask, **params)
    assert impl.called
    torch.testing.assert_close(got, want, rtol=0, atol=0)


@pytest.mark.parametrize("case", ["float64", "c_z_550", "fp32_c_z_288", "c_hidden_48_grad", "c_z_544_grad"])
def test_unsupported_configs_use_the_torch_path(case):
    """Configurations without kernels: fp64, widths above the fused tiles that are not
    multiples of 32 (the wide-width forward takes multiples of 32 only; fp32 above 256), and
    gradients with a width that is not a multiple of 32 or above 512 (the backward kernels'
    limits). (Other calls that need gradients run the HIP forward and backward:
    tests/test_trimul_bwd_gpu.py.)"""
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    dtype = {"float64": torch.float64, "c_z_550": torch.bfloat16, "c_z_544_grad": torch.bfloat16}.get(
        case, torch.float32)
    c_z = {"c_z_550": 550, "fp32_c_z_288": 288, "c_z_544_grad": 544}.get(case, 32)
    c_hidden = 48 if case == "c_hidden_48_grad" else 32
    w = {k: v.to(DEV) for k, v in trimul_weights(c_z, c_hidden, dtype, seed=1).items()}
    x, mask = pair_input(1, 12, c_z, dtype, seed=3)
    x = x.to(DEV)
    if case.endswith("_grad"):
        x.requires_grad_()
    with dispatch_spy() as (ref, kern):
        triangle_multiplicative_update(x, "outgoing", mask.to(DEV), **w)
    assert ref.called and not kern.called


@DIRECTIONS
@pytest.mark.parametrize(("dtype", "c_z", "c_hidden", "N"),
                         [(torch.bfloat16, 544, 576, 40), (torch.float16, 1024, 64, 32), (torch.bfloat16, 128, 640, 24)],
                         ids=["bf16_544_576_n40", "fp16_1024_64_n32", "bf16_128_640_n24"])
def test_wide_channel_widths(direction, dtype, c_z, c_hidden, N):
    """Widths above the fused kernels' 512 (the reference's Triton kernels take any width,
    trimul.py:310-314): the composed forward (trimul_wide_hip: the wide-row LayerNorm of
    gnn_layernorm_rows, the input linears on the vendor GEMM, gnn_trimul_relayout into the
    contraction's planes, gnn_trimul_contract at any width, LN_out, p_out and the gates) through
    the public op, with projection biases, random LayerNorm parameters and a padded mask;
    N = 40 and 24 take the pair grid to the next multiple of 32 with the padded pixels masked
    out. Against the fp64 oracle."""
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    w = trimul_weights(c_z, c_hidden, dtype, seed=37, biases=True, ln_random=True)
    x, mask = pair_input(1, N, c_z, dtype, seed=38)
    with dispatch_spy() as (ref, kern), torch.no_grad():
        got = triangle_multiplicative_update(x.to(DEV), direction, mask.to(DEV), **{k: v.to(DEV) for k, v in w.items()})
    assert kern.called and not ref.called
    assert got.shape == x.shape and got.dtype == dtype
    assert_close_to_oracle("out", got, oracle(x, direction, mask, w), Tolerance(1 - 1e-4, 2e-2),
                           rel_fro_max=NORTH_STAR_REL_FRO)


@DIRECTIONS
@pytest.mark.parametrize(("dtype", "c_z", "c_hidden"),
                         [(torch.bfloat16, 40, 24), (torch.bfloat16, 100, 70), (torch.bfloat16, 130, 128),
                          (torch.bfloat16, 120, 110), (torch.bfloat16, 496, 250), (torch.float16, 72, 40),
                          (torch.float32, 40, 20)],
                         ids=["bf16_40_24", "bf16_100_70", "bf16_130_128", "bf16_120_110", "bf16_496_250",
                              "fp16_72_40", "fp32_40_20"])
def test_odd_channel_widths(direction, dtype, c_z, c_hidden):
    """Widths that are not multiples of 32 (the reference's Triton kernels mask any width,
    trimul.py:310-314) on the forward kernels: x and the weights zero-padded to multiples of
    32 and the LayerNorms averaging over the real widths, with projection biases, random
    LayerNorm parameters and a padded mask, through the public op, against the fp64 oracle."""
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    w = trimul_weights(c_z, c_hidden, dtype, seed=27, biases=True, ln_random=True)
    x, mask = pair_input(1, 36, c_z, dtype, seed=28)
    with dispatch_spy() as (ref, kern), torch.no_grad():
        got = triangle_multiplicative_update(x.to(DEV), direction, mask.to(DEV), **{k: v.to(DEV) for k, v in w.items()})
    assert kern.called and not ref.called
    assert got.shape == x.shape and got.dtype == dtype
    tol = TRIMUL_TOL[torch.float32, "ieee"] if dtype == torch.float32 else Tolerance(1 - 1e-4, 2e-2)
    assert_close_to_oracle("out", got, oracle(x, direction, mask, w), tol,
                           rel_fro_max=None if dtype == torch.float32 else NORTH_STAR_REL_FRO)


@pytest.mark.parametrize(("b", "n", "direction"), [(2, 150, "incoming"), (1, 288, "outgoing")],
                         ids=["b2_n150_incoming", "b1_n288_outgoing"])
def test_fp32_tf32_contraction_tiles(b, n, direction):
    """fp32 under 'tf32' at sizes where the contraction takes 192-row tiles (on a 256-CU
    device the 192-row kernel holds two workgroups per CU, the 128-row one three; B = 2,
    N = 150: 256 tiles of 192 against 1024 of 128, one round against two; B = 1, N = 288:
    512 against 1152). N = 150 has one partial tile and guarded k-tail loads, N = 288 a
    whole tile, a ragged second one (96 rows) and unconditional loads; against the fp64
    oracle."""
    w = trimul_weights(128, 128, torch.float32, seed=45, biases=True, ln_random=True)
    x, mask = pair_input(b, n, 128, torch.float32, seed=46)
    with matmul_precision("tf32"):
        got = hip(x, direction, mask, w)
    assert_close_to_oracle("out", got, oracle(x, direction, mask, w), TRIMUL_TOL[torch.float32, "tf32"])


@DIRECTIONS
@pytest.mark.parametrize(("c_z", "c_hidden"), [(128, 128), (128, 64), (64, 32), (100, 70)],
                         ids=["128_128", "128_64", "64_32", "odd_100_70"])
def test_fp32_tf32_projection(direction, c_z, c_hidden):
    """fp32 under 'tf32' with c_z 64 or 128 (after padding) and c_hidden <= 128: the
    projection kernel that splits z, its weights and the gate weights into bf16 halves once.
    Ragged N (70: a partial last tile, row tails past N), batch 2, projection biases, random
    LayerNorm parameters and a padded mask, against the fp64 oracle."""
    w = trimul_weights(c_z, c_hidden, torch.float32, seed=41, biases=True, ln_random=True)
    x, mask = pair_input(2, 70, c_z, torch.float32, seed=42)
    with matmul_precision("tf32"):
        got = hip(x, direction, mask, w)
    assert_close_to_oracle("out", got, oracle(x, direction, mask, w), TRIMUL_TOL[torch.float32, "tf32"])


# ------------------------------------------------------------------ BASELINE configs (full size)
def test_config_c1_n64_fp32():
    """C1 shape (x [1,64,64,128] fp32, unit LN, weights N(0,1/128), all-ones mask) on the GPU."""
    w = trimul_weights(128, 128, torch.float32, seed=0)
    x = randn((1, 64, 64, 128), seed=1)
    mask = torch.ones(1, 64, 64)
    with matmul_precision("ieee"):
        got = hip(x, "outgoing", mask, w)
    assert_close_to_oracle("out", got, oracle(x, "outgoing", mask, w), TRIMUL_TOL[torch.float32, "ieee"])


@DIRECTIONS
def test_config_c3_n512(direction):
    """bf16 N=512, c_z = c_hidden = 128, LN gamma ~ 1+0.1N, beta ~ 0.1N, last 64 residues
    masked on both axes."""
    N, C = 512, 128
    w = trimul_weights(C, C, torch.bfloat16, seed=0, ln_random=True)
    x = randn((1, N, N, C), torch.bfloat16, seed=1)
    live = torch.arange(N) < N - 64
    mask = (live[:, None] & live[None, :]).to(torch.bfloat16)[None]
    got = hip(x, direction, mask, w)
    want = oracle(x, direction, mask, w)
    assert_close_to_oracle("out", got, want, TRIMUL_TOL[torch.bfloat16, "ieee"], rel_fro_max=NORTH_STAR_REL_FRO)
