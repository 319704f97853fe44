"""Past 2^31 elements: the 64-bit offset paths of every forward kernel.

A 32-bit element or byte offset that wraps gives finite, wrong values, which only a tensor
with more than 2^31 elements can show (the reference's test_large_n_no_int32_overflow,
tests/test_trimul.py:406-434, runs trimul at N=4096, C=128 for this). Each case here is a
little past 2^31 elements, so the last rows sit beyond the 32-bit range, and is checked
  * against the fp64 oracle on the pixels / query rows that live past the boundary, and
  * (trimul) over the whole output against the package's own torch path on the GPU, with the
    reference test's bound (cos >= 1 - 1e-3, rel-Fro <= 3e-2, fp32 metrics), so a wrap
    anywhere in the tensor fails.
Inputs are drawn on the GPU from a seeded generator (tens of GB: a CPU draw would take
minutes); the oracle gets the slices it needs copied back.
"""

import numpy as np
import pytest
import torch

from helpers import TRIANGLE_ATTENTION_TOL, TRIMUL_TOL, assert_close_to_oracle, to_np, trimul_pixels
from oracle import triangle_oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.large]
DEV = "cuda"
INT31 = 1 << 31


def _gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def _free():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_past_int32_elements(direction):
    """bf16 trimul at N=4100, C=128: x holds 2.15e9 elements and every workspace operand as
    many (N is not a multiple of 32, so the a / b row padding is exercised too)."""
    from geometric_nn_ops_torch.triangle import triangle_multiplicative_update
    from geometric_nn_ops_torch.triangle._reference.trimul import trimul_torch

    N, C = 4100, 128
    assert N * N * C > INT31
    dt = torch.bfloat16
    g = _gen(13)
    w = {
        "norm_in_weight": 1 + 0.1 * torch.randn(C, device=DEV, generator=g),
        "norm_in_bias": 0.1 * torch.randn(C, device=DEV, generator=g),
        "p_in_weight": torch.randn(2 * C, C, device=DEV, generator=g) / C**0.5,
        "g_in_weight": torch.randn(2 * C, C, device=DEV, generator=g) / C**0.5,
        "norm_out_weight": 1 + 0.1 * torch.randn(C, device=DEV, generator=g),
        "norm_out_bias": 0.1 * torch.randn(C, device=DEV, generator=g),
        "p_out_weight": torch.randn(C, C, device=DEV, generator=g) / C**0.5,
        "g_out_weight": torch.randn(C, C, device=DEV, generator=g) / C**0.5,
    }
    w = {k: v.to(dt) for k, v in w.items()}
    x = torch.randn(1, N, N, C, device=DEV, generator=_gen(47), dtype=dt)
    live = torch.arange(N, device=DEV) < N - 37
    mask = (live[:, None] & live[None, :]).to(dt)[None]
    print(f"trimul {direction} N={N}: HIP forward", flush=True)
    with torch.inference_mode():
        out = triangle_multiplicative_update(x, direction, mask, **w)
    _free()

    # the oracle on pixels whose offsets lie past 2^31 elements (the last rows) and before it
    rows, cols = [1, N - 40, N - 1], [0, N - 38, N - 1]
    want = trimul_pixels(x, mask, w, direction, rows, cols)
    got = out[:, rows][:, :, cols]
    assert_close_to_oracle(f"pixels past 2^31 ({direction})", got, want, TRIMUL_TOL[dt, "ieee"], rel_fro_max=1e-2)

    # whole output against the package's torch path, fp32 metrics (reference test bound)
    print(f"trimul {direction} N={N}: torch path", flush=True)
    with torch.inference_mode():
        ref = trimul_torch(x, direction, mask, **w)
    del x
    _free()
    a, b = out.float(), ref.float()
    del out, ref
    rel = (torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b)).item()
    cos = torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0).item()
    del a, b
    _free()
    assert cos >= 1 - 1e-3 and rel <= 3e-2, (cos, rel)


@pytest.mark.parametrize("case", ["row_kernel", "tiled_kernel"])
def test_attention_past_int32_elements(case):
    """bf16 triangle attention with q / k / v / o of more than 2^31 elements each, on both
    forward kernels: D = 32, N_res = 1024 (row-resident kernel) with N_seq = 16400, and
    D = 128 (tiled kernel) with N_seq = 2100, N_res = 2048. Pair bias and a key mask; the
    first and the last N_seq rows are checked against the fp64 oracle."""
    from geometric_nn_ops_torch.triangle import triangle_attention

    S, N, H, D = (16400, 1024, 4, 32) if case == "row_kernel" else (2100, 2048, 4, 128)
    assert S * N * H * D > INT31
    dt = torch.bfloat16
    g = _gen(7)
    q, k, v = (torch.randn(1, S, N, H, D, device=DEV, generator=g, dtype=dt) for _ in range(3))
    bias = torch.randn(1, 1, H, N, N, device=DEV, generator=g, dtype=dt)
    mask = torch.rand(1, S, 1, 1, N, device=DEV, generator=g) < 0.8
    mask[..., 0] = True
    print(f"attention {case} S={S} N={N} D={D}", flush=True)
    with torch.inference_mode():
        o = triangle_attention(q, k, v, bias, mask)
    _free()
    for s in (0, S - 1):
        sl = slice(s, s + 1)
        want = O.triangle_attention(to_np(q[:, sl]), to_np(k[:, sl]), to_np(v[:, sl]), to_np(bias),
                                    mask[:, sl].cpu().numpy())
        assert_close_to_oracle(f"row {s}", o[:, sl], want, TRIANGLE_ATTENTION_TOL[dt, "ieee"], rel_fro_max=1e-2)
    assert np.isfinite(to_np(o[:, -1])).all()
