"""the pair-stack block at full size on one GPU.

bf16, N=1024, c_z=128, in order: triangle multiplicative update outgoing, incoming, triangle
attention around the starting node, then around the ending node (H=4, D=32; the ending node
attends over the transposed pair tensor), each added to the residual pair stream. The same
block runs at N=384 with fp32 inputs under fp32_precision 'tf32' and 'ieee'. Inputs are
seeded N(0,1), weights N(0,1/fan_in), unit LayerNorm (config text in BASELINE.json).

Every op is called through the public API (so the HIP path is the one taken) on the input it
actually receives in the block, and checked against the fp64 oracle: trimul on a grid of
sampled pixels (oracle.trimul_grid, pinned against the full oracle in test_oracle.py),
attention on sampled N_seq rows (every query, head and channel of those rows).
"""

import numpy as np
import pytest
import torch

from helpers import (NORTH_STAR_REL_FRO, TRIANGLE_ATTENTION_TOL, TRIMUL_TOL, assert_close_to_oracle, gen,
                     np_weights, randn, to_np, trimul_weights)
from oracle import triangle_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
H, D = 4, 32


class fp32_precision:
    def __init__(self, precision):
        self.precision = precision

    def __enter__(self):
        self.prev = torch.backends.cuda.matmul.fp32_precision
        torch.backends.cuda.matmul.fp32_precision = self.precision

    def __exit__(self, *exc):
        torch.backends.cuda.matmul.fp32_precision = self.prev


def _attention_weights(c_z, dtype, seed):
    g = gen(seed)
    w = {k: randn((c_z, H * D), dtype, g=g, scale=c_z**-0.5) for k in ("q", "k", "v")}
    w["b"] = randn((c_z, H), dtype, g=g, scale=c_z**-0.5)
    w["o"] = randn((H * D, c_z), dtype, g=g, scale=(H * D) ** -0.5)
    return {k: v.to(DEV) for k, v in w.items()}


def _trimul_stage(z, direction, w, tol, rel_fro_max, rows, cols):
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update

    with torch.no_grad():
        out = triangle_multiplicative_update(z, direction, None, **{k: v.to(DEV) for k, v in w.items()})
    want = O.trimul_grid(to_np(z), direction, None, rows, cols, **np_weights(w))
    assert_close_to_oracle(f"trimul {direction}", out[:, rows][:, :, cols], want, tol, rel_fro_max=rel_fro_max)
    return z + out


def _attention_stage(z, w, ending, tol, rel_fro_max, rows):
    """Starting node: rows s of the pair stream attend along their columns. Ending node: the
    same on the transposed stream, passed as transpose(1, 2) views of q / k / v and a
    transpose(-1, -2) view of the bias (no copies), the output transposed back."""
    from geometric_nn_ops_torch.triangle import triangle_attention

    B, N = z.shape[0], z.shape[1]
    with torch.no_grad():
        q, k, v = ((z @ w[n]).view(B, N, N, H, D) for n in ("q", "k", "v"))
        bias = (z @ w["b"]).permute(0, 3, 1, 2).unsqueeze(1)  # [B, 1, H, N, N], a strided view
        if ending:
            q, k, v = (t.transpose(1, 2) for t in (q, k, v))
            bias = bias.transpose(-1, -2)
        o = triangle_attention(q, k, v, bias, None, D**-0.5)
    want = O.triangle_attention(to_np(q[:, rows]), to_np(k[:, rows]), to_np(v[:, rows]), to_np(bias), None,
                                D**-0.5)
    name = "attention " + ("ending" if ending else "starting")
    assert_close_to_oracle(name, o[:, rows], want, tol, rel_fro_max=rel_fro_max)
    with torch.no_grad():
        upd = o.reshape(B, N, N, H * D) @ w["o"]
    return z + (upd.transpose(1, 2) if ending else upd)


def _block(N, dtype, precision, rel_fro_max):
    C = 128
    z = randn((1, N, N, C), dtype, g=gen(5)).to(DEV)
    tw = trimul_weights(C, C, dtype, seed=6)
    aw = _attention_weights(C, dtype, seed=7)
    rows, cols = [0, N // 3, N - 1], [1, N // 2, N - 2]
    srows = [0, N // 2, N - 1]
    tm_tol = TRIMUL_TOL[dtype, precision]
    at_tol = TRIANGLE_ATTENTION_TOL[dtype, precision]
    with fp32_precision(precision):
        z = _trimul_stage(z, "outgoing", tw, tm_tol, rel_fro_max, rows, cols)
        z = _trimul_stage(z, "incoming", tw, tm_tol, rel_fro_max, rows, cols)
        z = _attention_stage(z, aw, False, at_tol, rel_fro_max, srows)
        z = _attention_stage(z, aw, True, at_tol, rel_fro_max, srows)
    assert torch.isfinite(z).all()


def test_pair_stack_n1024_bf16():
    _block(1024, torch.bfloat16, "ieee", NORTH_STAR_REL_FRO)


@pytest.mark.parametrize("precision", ["tf32", "ieee"])
def test_pair_stack_n384_fp32(precision):
    _block(384, torch.float32, precision, None)
