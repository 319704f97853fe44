"""Shared test helpers: seeded input builders, tolerance tables and oracle comparison.

Inputs are always drawn on the CPU from seeded generators and then moved to the device,
so the HIP kernels and the CPU oracle see identical bits. Tolerance tables restate the
reference's testutil/metrics.py:96-108 (cosine floor, relative-Frobenius ceiling against
the fp64 oracle).
"""

from typing import NamedTuple

import numpy as np
import torch

from oracle import triangle_oracle as O


class Tolerance(NamedTuple):
    cos_min: float
    rel_fro_max: float


TRIMUL_TOL = {
    (torch.float32, "ieee"): Tolerance(1.0 - 1e-6, 1.5e-3),
    (torch.float32, "tf32"): Tolerance(1.0 - 1e-6, 2e-3),
    (torch.float16, "ieee"): Tolerance(1.0 - 1e-6, 2e-3),
    (torch.bfloat16, "ieee"): Tolerance(1.0 - 1e-4, 1.5e-2),
}
TRIANGLE_ATTENTION_TOL = {
    (torch.float32, "ieee"): Tolerance(1.0 - 1e-5, 1.5e-3),
    (torch.float32, "tf32"): Tolerance(1.0 - 1e-5, 2e-3),
    (torch.float16, "ieee"): Tolerance(1.0 - 1e-4, 2e-2),
    (torch.bfloat16, "ieee"): Tolerance(1.0 - 1e-4, 5e-2),
}
ATTENTION_PAIR_BIAS_TOL = {
    (torch.float32, "ieee"): Tolerance(1.0 - 1e-5, 2e-3),
    (torch.float32, "tf32"): Tolerance(1.0 - 1e-5, 3e-3),
    (torch.float16, "ieee"): Tolerance(1.0 - 1e-4, 5e-3),
    (torch.bfloat16, "ieee"): Tolerance(1.0 - 1e-4, 2e-2),
}
# The build's own bar for 16-bit inputs: relative Frobenius <= 1e-2 against the
# fp32/fp64 reference on identical inputs.
NORTH_STAR_REL_FRO = 1e-2


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(shape, dtype=torch.float32, *, seed=0, scale=1.0, device="cpu", g=None):
    g = g or gen(seed)
    t = torch.randn(*shape, generator=g, dtype=torch.float32) * scale
    return t.to(dtype).to(device)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy()


def attention_inputs(b, n_seq, n_res, h, d, dtype, *, seed=0, with_bias=True, bias_scale=0.1,
                     device="cpu"):
    """q/k/v ``[b, N_seq, N_res, H, D]`` ~ N(0, 1) and bias ``[b, 1, H, N, N]``."""
    g = gen(seed)
    out = {name: randn((b, n_seq, n_res, h, d), dtype, g=g, device=device) for name in "qkv"}
    if with_bias:
        out["bias"] = randn((b, 1, h, n_res, n_res), dtype, g=g, scale=bias_scale, device=device)
    return out


def key_mask(b, n_seq, n_res, *, seed=0, frac_keep=0.75, device="cpu"):
    """Random boolean key mask ``[b, N_seq, 1, 1, N_res]`` with key 0 always kept."""
    m = torch.rand(b, n_seq, 1, 1, n_res, generator=gen(seed)) < frac_keep
    m[..., 0] = True
    return m.to(device)


def trimul_weights(c_z, c_hidden, dtype, *, seed=0, device="cpu", biases=False, ln_random=False):
    """LayerNorm + projection parameters (bias-free projections unless ``biases``)."""
    g = gen(seed)
    w = {
        "norm_in_weight": torch.ones(c_z),
        "norm_in_bias": torch.zeros(c_z),
        "p_in_weight": randn((2 * c_hidden, c_z), g=g, scale=c_z ** -0.5),
        "g_in_weight": randn((2 * c_hidden, c_z), g=g, scale=c_z ** -0.5),
        "norm_out_weight": torch.ones(c_hidden),
        "norm_out_bias": torch.zeros(c_hidden),
        "p_out_weight": randn((c_z, c_hidden), g=g, scale=c_hidden ** -0.5),
        "g_out_weight": randn((c_z, c_z), g=g, scale=c_z ** -0.5),
    }
    if ln_random:
        w["norm_in_weight"] = 1 + 0.1 * randn((c_z,), g=g)
        w["norm_in_bias"] = 0.1 * randn((c_z,), g=g)
        w["norm_out_weight"] = 1 + 0.1 * randn((c_hidden,), g=g)
        w["norm_out_bias"] = 0.1 * randn((c_hidden,), g=g)
    if biases:
        w["p_in_bias"] = randn((2 * c_hidden,), g=g, scale=0.05)
        w["g_in_bias"] = randn((2 * c_hidden,), g=g, scale=0.05)
        w["p_out_bias"] = randn((c_z,), g=g, scale=0.05)
        w["g_out_bias"] = randn((c_z,), g=g, scale=0.05)
    return {k: v.to(dtype).to(device) for k, v in w.items()}


def pair_input(batch, n, c_z, dtype, *, seed=0, frac_keep=0.9, device="cpu"):
    """Pair representation ``[*batch, N, N, C_z]`` ~ N(0, 1) and a random 0/1 mask."""
    lead = (batch,) if isinstance(batch, int) else tuple(batch)
    g = gen(seed)
    x = randn(lead + (n, n, c_z), dtype, g=g)
    mask = (torch.rand(*lead, n, n, generator=g) < frac_keep).to(dtype)
    return x.to(device), mask.to(device)


def np_weights(w: dict) -> dict:
    return {k: (None if v is None else to_np(v)) for k, v in w.items()}


def assert_close_to_oracle(name, got, want, tol: Tolerance, *, rel_fro_max=None):
    """Cosine and relative-Frobenius check of ``got`` (tensor) against ``want`` (numpy)."""
    g = to_np(got)
    assert g.shape == want.shape, f"{name}: shape {g.shape} vs oracle {want.shape}"
    assert np.isfinite(want).all(), f"{name}: oracle has non-finite values"
    assert np.isfinite(g).all(), f"{name}: candidate has non-finite values"
    c, f = O.cos(g, want), O.rel_fro(g, want)
    bound = tol.rel_fro_max if rel_fro_max is None else min(tol.rel_fro_max, rel_fro_max)
    assert c >= tol.cos_min, f"{name}: cos {c:.7f} < {tol.cos_min}"
    assert f <= bound, f"{name}: rel-fro {f:.3e} > {bound:.1e} (max-abs {np.abs(g - want).max():.3e})"
    return c, f


def apb_inputs(b, m, h, u, v, dh, zc, dtype=torch.float32, *, seed=0, biases=False, device="cpu"):
    """Attention-with-pair-bias op tensors (the reference's testutil/attention_pair_bias.py:
    make_op_tensors layout): s, pre-projected q/k/v, pair rep z and the weights."""
    g = gen(seed)
    d = h * dh
    t = {
        "s": randn((b * m, u, d), g=g),
        "q": randn((b * m, h, u, dh), g=g),
        "k": randn((b * m, h, v, dh), g=g),
        "v": randn((b * m, h, v, dh), g=g),
        "z": randn((b, u, v, zc), g=g),
        "proj_z_weight": randn((h, zc), g=g, scale=zc ** -0.5),
        "ln_z_weight": 1.0 + 0.1 * randn((zc,), g=g),
        "proj_g_weight": randn((d, d), g=g, scale=d ** -0.5),
        "proj_o_weight": randn((d, d), g=g, scale=d ** -0.5),
    }
    if biases:
        t["proj_g_bias"] = randn((d,), g=g, scale=0.1)
        t["proj_o_bias"] = randn((d,), g=g, scale=0.1)
    return {k: x.to(dtype).to(device) for k, x in t.items()}


def apb_key_mask(batch, v, *, seed=0, frac_keep=0.9, dtype=torch.float32, device="cpu"):
    """``[batch, V]`` 0 / 1 key mask, key 0 always kept."""
    m = torch.rand(batch, v, generator=gen(seed)) < frac_keep
    m[:, 0] = True
    return m.to(dtype).to(device)


def trimul_pixels(x, mask, w, direction, rows, cols):
    """``oracle.trimul`` at pixels ``(rows[i], cols[j])`` of a grid too large to copy whole.

    The pixels need only the pair-grid lines ``U = rows + cols`` of x (grid rows for
    'outgoing', columns for 'incoming'), so ``oracle.trimul_grid`` runs on x restricted to
    those lines with line indices into U. Its output gate is then taken from the restricted
    tensor at the compacted (line, line) position instead of at pixel (rows[i], cols[j]);
    the factor is replaced by the gate of the true pixel (both gates are sigmoids, > 0)."""
    wn = {k: to_np(v) for k, v in w.items()}
    lines = sorted(set(rows) | set(cols))
    pos = {r: i for i, r in enumerate(lines)}
    ri, ci = [pos[r] for r in rows], [pos[c] for c in cols]
    if direction == "outgoing":
        xs, ms = to_np(x[:, lines]), to_np(mask[:, lines])
    else:
        xs, ms = to_np(x[:, :, lines]), to_np(mask[:, :, lines])
    got = O.trimul_grid(xs, direction, ms, ri, ci, **wn)

    def gate(pix):
        z = O.layer_norm(pix, wn["norm_in_weight"], wn["norm_in_bias"])
        return O.sigmoid(O.linear(z, wn["g_out_weight"], wn.get("g_out_bias")))

    return got / gate(xs[:, ri][:, :, ci]) * gate(to_np(x[:, rows][:, :, cols]))
