"""Pins the CPU oracle (oracle/triangle_oracle.py) without running the reference.

Each oracle function is checked against something independent of its own formula:
pure-Python loop implementations at tiny sizes, closed forms and the reference's
known-answer cases (tests/test_triangle_attention.py:88-338 and tests/test_trimul.py:70-131
of AMDResearch/geometric-nn-ops), chosen so that a dropped term, a wrong sign, a swapped
index or a transposed operand fails at least one of them.
"""

import math

import numpy as np
import pytest
import torch

from oracle import triangle_oracle as O

RNG = np.random.default_rng


# ---------------------------------------------------------------------------------- masking
def test_mask_val_values():
    """Reference _masking.py:32-39: 1e18 fp64, 1e9 fp32/bf16, finfo(fp16).max/2 fp16."""
    assert O.mask_val("float64") == 1e18
    assert O.mask_val("float32") == 1e9 and O.mask_val("bfloat16") == 1e9
    assert O.mask_val("float16") == 65504.0 / 2
    with pytest.raises(ValueError):
        O.mask_val("int8")


def test_masked_key_bias_signs():
    """Kept keys get +0.0 (not -0.0); masked keys get exactly -mask_val."""
    m = np.array([True, False, True])
    b = O.masked_key_bias(m)
    assert b[1] == -1e18
    assert b[0] == 0 and not np.signbit(b[0]) and not np.signbit(b[2])


@pytest.mark.parametrize("name", ["float32", "bfloat16", "float16"])
def test_mask_val_suppresses_any_realistic_logit(name):
    """exp underflows to 0 below ~-104 in fp32: needs mask_val/2 - 52 > 1e4
    (reference test_triangle_attention.py:316-338)."""
    assert O.mask_val(name) / 2 - 52 > 1e4


# ---------------------------------------------------------------------- triangle attention
def _attention_loops(q, k, v, bias, mask, scale):
    """Softmax attention with explicit Python loops: o[b,s,i,h,:] = sum_j p_ij v[b,s,j,h,:]."""
    B, S, N, H, D = q.shape
    out = np.zeros_like(q)
    for b in range(B):
        for s in range(S):
            for h in range(H):
                for i in range(N):
                    logits = []
                    for j in range(N):
                        dot = sum(q[b, s, i, h, d] * scale * k[b, s, j, h, d] for d in range(D))
                        if bias is not None:
                            dot += bias[b, 0, h, i, j]
                        if mask is not None and not mask[b, s, 0, 0, j]:
                            dot += -1e18
                        logits.append(dot)
                    mx = max(logits)
                    ws = [math.exp(x - mx) for x in logits]
                    tot = sum(ws)
                    for d in range(D):
                        out[b, s, i, h, d] = sum(ws[j] * v[b, s, j, h, d] for j in range(N)) / tot
    return out


def test_attention_matches_loops():
    r = RNG(0)
    B, S, N, H, D = 2, 2, 5, 2, 3
    q, k, v = (r.standard_normal((B, S, N, H, D)) for _ in range(3))
    bias = r.standard_normal((B, 1, H, N, N))
    mask = r.random((B, S, 1, 1, N)) < 0.7
    mask[..., 0] = True
    scale = 0.37
    want = _attention_loops(q, k, v, bias, mask, scale)
    got = O.triangle_attention(q, k, v, bias, mask, scale)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # 4D bias gains the N_seq axis; chunking over N_seq changes nothing
    np.testing.assert_allclose(O.triangle_attention(q, k, v, bias[:, 0], mask, scale, s_chunk=1),
                               want, rtol=1e-12, atol=1e-12)


def _lse_max_loops(q, k, bias, mask, scale, mask_value):
    """Per-query log-sum-exp and maximum of the logits, with explicit Python loops."""
    B, S, N, H, D = q.shape
    lse = np.zeros((B, S, H, N))
    mx = np.zeros((B, S, H, N))
    for b in range(B):
        for s in range(S):
            for h in range(H):
                for i in range(N):
                    row = []
                    for j in range(N):
                        x = sum(q[b, s, i, h, d] * scale * k[b, s, j, h, d] for d in range(D))
                        x += bias[b, 0, h, i, j] if bias is not None else 0.0
                        x += 0.0 if mask is None or mask[b, s, 0, 0, j] else mask_value
                        row.append(x)
                    mx[b, s, h, i] = max(row)
                    lse[b, s, h, i] = math.log(sum(math.exp(x) for x in row))
    return lse, mx


def test_lse_max_match_loops():
    """Known answers too: one live key -> both equal its logit; equal logits -> lse = max +
    log(number of keys)."""
    r = RNG(7)
    B, S, N, H, D = 1, 2, 6, 2, 3
    q, k = (r.standard_normal((B, S, N, H, D)) for _ in range(2))
    bias = r.standard_normal((B, 1, H, N, N))
    mask = r.random((B, S, 1, 1, N)) < 0.7
    mask[..., 1] = True
    lse, mx = O.triangle_attention_lse_max(q, k, bias, mask, 0.4, mask_value=-30.0)
    want = _lse_max_loops(q, k, bias, mask, 0.4, -30.0)
    np.testing.assert_allclose(lse, want[0], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mx, want[1], rtol=1e-12, atol=1e-12)
    assert not np.allclose(lse, mx)
    one = np.zeros((1, 1, 1, 1, N), dtype=bool)
    one[..., 2] = True
    lse1, mx1 = O.triangle_attention_lse_max(q[:, :1], k[:, :1], bias, one)
    logit = np.einsum("bihd,bhd->bhi", q[:, 0] * 3 ** -0.5, k[:, 0, 2]) + bias[:, 0, :, :, 2]
    np.testing.assert_allclose(mx1[:, 0], logit, rtol=1e-12)
    np.testing.assert_allclose(lse1[:, 0], logit, rtol=1e-12)
    lse0, mx0 = O.triangle_attention_lse_max(np.zeros((1, 1, N, H, D)), k[:, :1])
    np.testing.assert_allclose(lse0, mx0 + math.log(N), rtol=1e-12)


def test_attention_transposes_are_not_symmetric():
    """Swapping q and k (a transposed product) must change the result."""
    r = RNG(1)
    q, k, v = (r.standard_normal((1, 1, 6, 1, 4)) for _ in range(3))
    assert not np.allclose(O.triangle_attention(q, k, v), O.triangle_attention(k, q, v))


@pytest.mark.parametrize("kept", [0, 7, 31])
def test_one_live_key_returns_that_value(kept):
    r = RNG(3)
    q, k, v = (r.standard_normal((1, 2, 32, 4, 8)) for _ in range(3))
    mask = np.zeros((1, 2, 1, 1, 32), bool)
    mask[..., kept] = True
    out = O.triangle_attention(q, k, v, r.standard_normal((1, 1, 4, 32, 32)), mask)
    np.testing.assert_array_equal(out, np.broadcast_to(v[:, :, kept:kept + 1], out.shape))


def test_uniform_logits_give_the_mean():
    r = RNG(5)
    v = r.integers(-4, 5, (1, 1, 32, 4, 16)).astype(np.float64)
    z = np.zeros_like(v)
    out = O.triangle_attention(z, z, v, np.zeros((1, 1, 4, 32, 32)))
    np.testing.assert_array_equal(out, np.broadcast_to(v.mean(axis=2, keepdims=True), out.shape))


def test_masked_values_are_bit_invariant():
    r = RNG(7)
    q, k, v = (r.standard_normal((1, 1, 32, 4, 8)) for _ in range(3))
    bias = r.standard_normal((1, 1, 4, 32, 32)) * 0.1
    mask = r.random((1, 1, 1, 1, 32)) < 0.75
    mask[..., 0] = True
    dead = ~mask.reshape(1, 1, 32, 1, 1)
    noisy_v = np.where(dead, v + 1e3 * r.standard_normal(v.shape), v)
    noisy_k = np.where(dead, k + 1e3 * r.standard_normal(k.shape), k)
    noisy_b = np.where(~mask.reshape(1, 1, 1, 1, 32), bias + 1e3, bias)
    base = O.triangle_attention(q, k, v, bias, mask)
    np.testing.assert_array_equal(base, O.triangle_attention(q, noisy_k, noisy_v, noisy_b, mask))
    assert not np.allclose(O.triangle_attention(q, k, v, bias), O.triangle_attention(q, k, noisy_v, bias))


def test_fully_masked_row_gives_the_mean():
    """The finite sentinel collapses every logit of a dead row to one value."""
    r = RNG(9)
    q, k = r.standard_normal((1, 1, 32, 4, 16)), r.standard_normal((1, 1, 32, 4, 16))
    v = r.integers(-4, 5, (1, 1, 32, 4, 16)).astype(np.float64)
    out = O.triangle_attention(q, k, v, None, np.zeros((1, 1, 1, 1, 32), bool))
    np.testing.assert_array_equal(out, np.broadcast_to(v.mean(axis=2, keepdims=True), out.shape))


def test_optional_arguments():
    r = RNG(11)
    q, k, v = (r.standard_normal((1, 2, 8, 2, 4)) for _ in range(3))
    keep = np.ones((1, 2, 1, 1, 8), bool)
    np.testing.assert_array_equal(O.triangle_attention(q, k, v), O.triangle_attention(q, k, v, None, keep))
    np.testing.assert_array_equal(O.triangle_attention(q, k, v),
                                  O.triangle_attention(q, k, v, np.zeros((1, 1, 2, 8, 8))))
    np.testing.assert_array_equal(O.triangle_attention(q, k, v), O.triangle_attention(q, k, v, scale=0.5))
    assert not np.allclose(O.triangle_attention(q, k, v), O.triangle_attention(q, k, v, scale=0.9))


# --------------------------------------------------------------------------------- trimul
def test_combine_matches_loops():
    r = RNG(13)
    a, b = r.standard_normal((2, 4, 4, 3)), r.standard_normal((2, 4, 4, 3))
    out_l = np.zeros_like(a)
    in_l = np.zeros_like(a)
    for n in range(2):
        for i in range(4):
            for j in range(4):
                for c in range(3):
                    out_l[n, i, j, c] = sum(a[n, i, kk, c] * b[n, j, kk, c] for kk in range(4))
                    in_l[n, i, j, c] = sum(a[n, kk, i, c] * b[n, kk, j, c] for kk in range(4))
    np.testing.assert_allclose(O.combine(a, b, True), out_l, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(O.combine(a, b, False), in_l, rtol=1e-13, atol=1e-13)
    assert not np.allclose(out_l, in_l)


def test_layer_norm_closed_forms():
    r = RNG(15)
    x = r.standard_normal((5, 7, 16)) * 3 + 2
    y = O.layer_norm(x, eps=0.0)
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-13)
    np.testing.assert_allclose((y ** 2).mean(-1), 1, atol=1e-12)  # biased variance
    w, b = r.standard_normal(16), r.standard_normal(16)
    np.testing.assert_allclose(O.layer_norm(x, w, b, eps=0.0), y * w + b, rtol=1e-13, atol=1e-13)
    # eps inside the square root: a constant row normalises to exactly 0, giving beta
    np.testing.assert_array_equal(O.layer_norm(np.zeros((2, 16)), w, b), np.broadcast_to(b, (2, 16)))
    xs = np.array([[1.0, 3.0]])
    np.testing.assert_allclose(O.layer_norm(xs, eps=1.0), [[-1 / math.sqrt(2), 1 / math.sqrt(2)]])


def _weights(r, c, ch, biases=False):
    w = dict(
        norm_in_weight=1 + 0.1 * r.standard_normal(c), norm_in_bias=0.1 * r.standard_normal(c),
        p_in_weight=r.standard_normal((2 * ch, c)) / math.sqrt(c),
        g_in_weight=r.standard_normal((2 * ch, c)) / math.sqrt(c),
        norm_out_weight=1 + 0.1 * r.standard_normal(ch), norm_out_bias=0.1 * r.standard_normal(ch),
        p_out_weight=r.standard_normal((c, ch)) / math.sqrt(ch),
        g_out_weight=r.standard_normal((c, c)) / math.sqrt(c),
    )
    if biases:
        w.update(p_in_bias=r.standard_normal(2 * ch), g_in_bias=r.standard_normal(2 * ch),
                 p_out_bias=r.standard_normal(c), g_out_bias=r.standard_normal(c))
    return w


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_single_residue_closed_form(direction):
    """At N = 1 both directions reduce to out = p_out(LN(a * b)) * sigmoid(g_out(z)),
    written here with explicit per-channel loops."""
    r = RNG(17)
    c, ch = 6, 4
    w = _weights(r, c, ch, biases=True)
    x = r.standard_normal((1, 1, c))
    xs = x[0, 0]
    mu = sum(xs) / c
    var = sum((t - mu) ** 2 for t in xs) / c
    z = [(xs[i] - mu) / math.sqrt(var + 1e-5) * w["norm_in_weight"][i] + w["norm_in_bias"][i] for i in range(c)]

    def lin(W, bvec, inp):
        return [sum(W[o][i] * inp[i] for i in range(len(inp))) + (bvec[o] if bvec is not None else 0)
                for o in range(len(W))]

    sig = lambda t: 1 / (1 + math.exp(-t))  # noqa: E731
    p = [pi * sig(gi) for pi, gi in zip(lin(w["p_in_weight"], w["p_in_bias"], z),
                                         lin(w["g_in_weight"], w["g_in_bias"], z))]
    o = [p[i] * p[ch + i] for i in range(ch)]
    mo = sum(o) / ch
    vo = sum((t - mo) ** 2 for t in o) / ch
    on = [(o[i] - mo) / math.sqrt(vo + 1e-5) * w["norm_out_weight"][i] + w["norm_out_bias"][i] for i in range(ch)]
    g = [sig(t) for t in lin(w["g_out_weight"], w["g_out_bias"], z)]
    want = np.array([t * gg for t, gg in zip(lin(w["p_out_weight"], w["p_out_bias"], on), g)])
    got = O.trimul(x, direction, **w)[0, 0]
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_fully_masked_is_a_constant_field(direction):
    """Zero mask zeroes the contraction and a zero g_out weight fixes the gate, so every
    position holds the same vector (reference test_trimul.py:70-90)."""
    r = RNG(19)
    w = _weights(r, 16, 16, biases=True)
    w["norm_out_bias"] = np.full(16, 0.25)
    w["g_out_weight"] = np.zeros((16, 16))
    out = O.trimul(r.standard_normal((1, 8, 8, 16)), direction, np.zeros((1, 8, 8)), **w)
    np.testing.assert_allclose(out, np.broadcast_to(out[:, :1, :1], out.shape), rtol=0, atol=1e-12)
    assert np.abs(out).max() > 0.01


def test_trimul_direction_and_biases_matter():
    r = RNG(21)
    w = _weights(r, 8, 8, biases=True)
    x = r.standard_normal((1, 6, 6, 8))
    base = O.trimul(x, "outgoing", **w)
    assert not np.allclose(base, O.trimul(x, "incoming", **w))
    for key in ("p_in_bias", "g_in_bias", "p_out_bias", "g_out_bias"):
        assert not np.allclose(base, O.trimul(x, "outgoing", **{**w, key: np.zeros_like(w[key])}))
    with pytest.raises(ValueError, match="direction must be one of"):
        O.trimul(x, "outgoin", **w)


def test_trimul_stages_are_consistent():
    """The staged intermediates recombine into the final output."""
    r = RNG(23)
    w = _weights(r, 8, 4)
    x = r.standard_normal((2, 5, 5, 8))
    mask = (r.random((2, 5, 5)) < 0.8).astype(float)
    st = O.trimul_stages(x, "incoming", mask, **w)
    np.testing.assert_allclose(st["o"], O.combine(st["a"], st["b"], False))
    np.testing.assert_array_equal(st["a"][mask == 0], 0)
    np.testing.assert_allclose(st["out"], O.linear(st["on"], w["p_out_weight"]) * st["g"])


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_grid_is_the_full_oracle_sampled(direction):
    """The sampled-pixel oracle used at large N equals the full oracle at those pixels
    (rows and columns repeated and unsorted on purpose; batched; masked; with biases)."""
    r = RNG(29)
    w = _weights(r, 8, 4, biases=True)
    x = r.standard_normal((2, 7, 7, 8))
    mask = (r.random((2, 7, 7)) < 0.7).astype(float)
    rows, cols = [5, 0, 5, 3], [6, 2, 0]
    full = O.trimul(x, direction, mask, **w)
    grid = O.trimul_grid(x, direction, mask, rows, cols, **w)
    np.testing.assert_allclose(grid, full[:, rows][:, :, cols], rtol=1e-12, atol=1e-12)


# --------------------------------------------- oracle vs the product's torch fallback (fp64)
def test_oracle_agrees_with_torch_fallback():
    """Two independent restatements (numpy loops-free oracle here, torch einsum in the
    package) agree in fp64, which pins the package's differentiable path too."""
    from geometric_nn_ops_torch.triangle._reference.triangle_attention import triangle_attention_torch
    from geometric_nn_ops_torch.triangle._reference.trimul import trimul_torch

    r = RNG(25)
    q, k, v = (r.standard_normal((2, 3, 9, 2, 8)) for _ in range(3))
    bias = r.standard_normal((2, 1, 2, 9, 9))
    mask = r.random((2, 3, 1, 1, 9)) < 0.7
    mask[..., 0] = True
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    got = triangle_attention_torch(t(q), t(k), t(v), t(bias), t(mask), 0.3).numpy()
    np.testing.assert_allclose(got, O.triangle_attention(q, k, v, bias, mask, 0.3), rtol=1e-12, atol=1e-12)

    w = _weights(r, 16, 8, biases=True)
    x = r.standard_normal((2, 7, 7, 16))
    m = (r.random((7, 7)) < 0.8).astype(float)
    for direction in ("outgoing", "incoming"):
        got = trimul_torch(t(x), direction, t(m), **{kk: t(vv) for kk, vv in w.items()}).numpy()
        np.testing.assert_allclose(got, O.trimul(x, direction, m, **w), rtol=1e-11, atol=1e-11)


# ------------------------------------------------------------- attention with pair bias
def _apb_inputs(B=2, M=2, H=2, U=3, V=3, DH=2, Zc=4, seed=0, biases=True):
    rng = np.random.default_rng(seed)
    D = H * DH
    t = {
        "s": rng.standard_normal((B * M, U, D)),
        "q": rng.standard_normal((B * M, H, U, DH)),
        "k": rng.standard_normal((B * M, H, V, DH)),
        "v": rng.standard_normal((B * M, H, V, DH)),
        "z": rng.standard_normal((B, U, V, Zc)),
        "proj_z_weight": rng.standard_normal((H, Zc)) * Zc ** -0.5,
        "ln_z_weight": 1.0 + 0.1 * rng.standard_normal(Zc),
        "proj_g_weight": rng.standard_normal((D, D)) * D ** -0.5,
        "proj_o_weight": rng.standard_normal((D, D)) * D ** -0.5,
    }
    if biases:
        t["proj_g_bias"] = 0.1 * rng.standard_normal(D)
        t["proj_o_bias"] = 0.1 * rng.standard_normal(D)
    return t


def _apb_loops(t, mask=None, scale=None, inf=1e18, eps=1e-5):
    """Element-by-element restatement in pure Python (math module only)."""
    s, q, k, v, z = (t[n].tolist() for n in ("s", "q", "k", "v", "z"))
    BM, H, U, DH = t["q"].shape
    V = t["k"].shape[2]
    B, Zc = t["z"].shape[0], t["z"].shape[3]
    M = BM // B
    D = H * DH
    scale = DH ** -0.5 if scale is None else scale
    wz, lw = t["proj_z_weight"].tolist(), t["ln_z_weight"].tolist()
    wg, wo = t["proj_g_weight"].tolist(), t["proj_o_weight"].tolist()
    bg = t.get("proj_g_bias", np.zeros(D)).tolist()
    bo = t.get("proj_o_bias", np.zeros(D)).tolist()
    bias = [[[[0.0] * V for _ in range(U)] for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for u in range(U):
            for j in range(V):
                x = z[b][u][j]
                mu = sum(x) / Zc
                var = sum((e - mu) ** 2 for e in x) / Zc
                zn = [(e - mu) / math.sqrt(var + eps) * lw[c] for c, e in enumerate(x)]
                for h in range(H):
                    bias[b][h][u][j] = sum(zn[c] * wz[h][c] for c in range(Zc))
    out = [[[0.0] * D for _ in range(U)] for _ in range(BM)]
    for n in range(BM):
        b = n // M
        o = [[0.0] * D for _ in range(U)]
        for h in range(H):
            for u in range(U):
                logit = []
                for j in range(V):
                    l_ = sum(q[n][h][u][d] * k[n][h][j][d] for d in range(DH)) * scale + bias[b][h][u][j]
                    if mask is not None:
                        keep = mask[b][j] if len(mask) == B else mask[n][j]
                        l_ += (keep - 1.0) * inf
                    logit.append(l_)
                mx = max(logit)
                e = [math.exp(x - mx) for x in logit]
                tot = sum(e)
                for d in range(DH):
                    o[u][h * DH + d] = sum(e[j] / tot * v[n][h][j][d] for j in range(V))
        for u in range(U):
            gated = [o[u][c] / (1.0 + math.exp(-(sum(s[n][u][i] * wg[c][i] for i in range(D)) + bg[c])))
                     for c in range(D)]
            for c in range(D):
                out[n][u][c] = sum(gated[i] * wo[c][i] for i in range(D)) + bo[c]
    return np.array(out), np.array(bias)


@pytest.mark.parametrize("mask_kind", [None, "batch", "copy"])
def test_attention_pair_bias_matches_loops(mask_kind):
    t = _apb_inputs()
    B, M, V = 2, 2, 3
    mask = None
    if mask_kind == "batch":
        mask = np.array([[1.0, 0.0, 1.0], [1.0, 1.0, 0.0]])
    elif mask_kind == "copy":
        mask = np.array([[1.0, 0.0, 1.0], [0.0, 1.0, 1.0], [1.0, 1.0, 0.0], [1.0, 0.0, 0.0]])
    out, pz = O.attention_pair_bias(**t, mask=mask, scale=0.7, inf=30.0, return_z_proj=True)
    want, want_pz = _apb_loops(t, None if mask is None else mask.tolist(), scale=0.7, inf=30.0)
    np.testing.assert_allclose(pz, want_pz, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out, want, rtol=1e-11, atol=1e-12)
    assert out.shape == (B * M, 3, 4) and V == 3


def test_attention_pair_bias_is_triangle_attention_with_multiplicity_rows():
    """The attention core equals triangle attention with N_seq = M: q [B*M, H, U, DH] is the
    canonical [B, M, U, H, DH] by a permutation, the bias is shared across the M rows."""
    B, M, H, U, DH, Zc = 2, 3, 2, 5, 4, 6
    t = _apb_inputs(B=B, M=M, H=H, U=U, V=U, DH=DH, Zc=Zc, seed=3, biases=False)
    D = H * DH
    t["proj_g_weight"] = np.zeros((D, D))  # gate = 1/2
    t["proj_o_weight"] = 2.0 * np.eye(D)   # out = o
    keep = (np.random.default_rng(5).random((B, U)) < 0.7).astype(np.float64)
    keep[:, 0] = 1.0
    out, pz = O.attention_pair_bias(**t, mask=keep, return_z_proj=True)
    canon = lambda a: np.transpose(a.reshape(B, M, H, U, DH), (0, 1, 3, 2, 4))  # noqa: E731
    o = O.triangle_attention(canon(t["q"]), canon(t["k"]), canon(t["v"]), bias=pz,
                             mask=keep.astype(bool)[:, None, None, None, :])
    np.testing.assert_allclose(out, o.reshape(B * M, U, D), rtol=1e-12, atol=1e-12)


def test_attention_pair_bias_known_answers():
    t = _apb_inputs(B=2, M=3, H=2, U=4, V=4, DH=3, Zc=5, seed=7)
    mask = np.ones((2, 4))
    mask[0, 2] = mask[1, 1] = 0.0
    out, pz = O.attention_pair_bias(**t, mask=mask, return_z_proj=True)
    # masked keys: v (and k) noise there changes nothing
    noisy = dict(t)
    for name in ("v", "k"):
        a = t[name].copy().reshape(2, 3, 2, 4, 3)
        a[0, :, :, 2] += 1e3
        a[1, :, :, 1] -= 1e3
        noisy[name] = a.reshape(t[name].shape)
    np.testing.assert_array_equal(O.attention_pair_bias(**noisy, mask=mask)[0], out)
    # the cached bias reproduces the uncached call exactly
    cached, _ = O.attention_pair_bias(**{**t, "z": pz}, mask=mask, z_is_projected=True)
    np.testing.assert_array_equal(cached, out)
    # a per-batch mask equals its per-copy repetition
    np.testing.assert_array_equal(O.attention_pair_bias(**t, mask=np.repeat(mask, 3, axis=0))[0], out)
    # copies with equal inputs give equal outputs; batch elements differ
    same = dict(t)
    for name in ("s", "q", "k", "v"):
        g = t[name].reshape(2, 3, *t[name].shape[1:])
        same[name] = np.broadcast_to(g[:, :1], g.shape).reshape(t[name].shape).copy()
    o2 = O.attention_pair_bias(**same)[0].reshape(2, 3, 4, 6)
    np.testing.assert_array_equal(o2[:, 1], o2[:, 0])
    assert not np.array_equal(o2[0, 0], o2[1, 0])
    # zero q and a zero pair bias: uniform attention, o = mean(v)
    flat = {**t, "q": np.zeros_like(t["q"]), "z": np.zeros((2, 2, 4, 4))}
    base = O.attention_pair_bias(**flat, z_is_projected=True)[0]
    o_mean = np.transpose(t["v"].mean(axis=2, keepdims=True).repeat(4, axis=2), (0, 2, 1, 3)).reshape(6, 4, 6)
    g = 1.0 / (1.0 + np.exp(-(t["s"] @ t["proj_g_weight"].T + t["proj_g_bias"])))
    np.testing.assert_allclose(base, (o_mean * g) @ t["proj_o_weight"].T + t["proj_o_bias"], rtol=1e-12)
    with pytest.raises(ValueError, match="multiple"):
        O.attention_pair_bias(**{**t, "z": t["z"][:1].repeat(4, axis=0)})


# ------------------------------------------------------------- attention gradients
def test_attention_grad_matches_finite_differences():
    """Central differences of the (loop-pinned) forward oracle: every entry of dq, dk, dv and
    of the N_seq-summed dbias."""
    rng = np.random.default_rng(17)
    B, S, N, H, D = 2, 2, 5, 2, 3
    q, k, v = (rng.standard_normal((B, S, N, H, D)) for _ in range(3))
    bias = 0.5 * rng.standard_normal((B, 1, H, N, N))
    mask = rng.random((B, S, 1, 1, N)) < 0.7
    mask[..., 0] = True
    dout = rng.standard_normal((B, S, N, H, D))
    scale = 0.6
    grads = O.triangle_attention_grad(q, k, v, bias, mask, scale, dout)
    inputs = {"q": q, "k": k, "v": v, "bias": bias}

    def loss(**kw):
        return float(np.sum(O.triangle_attention(kw["q"], kw["k"], kw["v"], kw["bias"], mask, scale) * dout))

    eps = 1e-6
    for name, g in zip(("q", "k", "v", "bias"), grads):
        base = inputs[name]
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            plus, minus = base.copy(), base.copy()
            plus[idx] += eps
            minus[idx] -= eps
            num[idx] = (loss(**{**inputs, name: plus}) - loss(**{**inputs, name: minus})) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-8, err_msg=name)
    # masked keys receive no k / v gradient at all
    dropped = ~mask[:, :, 0, 0, :]
    assert np.all(grads[1][dropped] == 0) and np.all(grads[2][dropped] == 0)


# ------------------------------------------------------------- trimul gradients
def _trimul_case(rng, B, N, C, Ch):
    w = {
        "norm_in_weight": 1 + 0.3 * rng.standard_normal(C), "norm_in_bias": 0.3 * rng.standard_normal(C),
        "p_in_weight": rng.standard_normal((2 * Ch, C)) / np.sqrt(C), "p_in_bias": 0.3 * rng.standard_normal(2 * Ch),
        "g_in_weight": rng.standard_normal((2 * Ch, C)) / np.sqrt(C), "g_in_bias": 0.3 * rng.standard_normal(2 * Ch),
        "norm_out_weight": 1 + 0.3 * rng.standard_normal(Ch), "norm_out_bias": 0.3 * rng.standard_normal(Ch),
        "p_out_weight": rng.standard_normal((C, Ch)) / np.sqrt(Ch), "p_out_bias": 0.3 * rng.standard_normal(C),
        "g_out_weight": rng.standard_normal((C, C)) / np.sqrt(C), "g_out_bias": 0.3 * rng.standard_normal(C),
    }
    x = rng.standard_normal((B, N, N, C))
    mask = (rng.random((B, N, N)) < 0.8).astype(np.float64)
    dout = rng.standard_normal((B, N, N, C))
    return x, mask, dout, w


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_grad_matches_finite_differences(direction):
    """Central differences of the (loop-pinned) forward oracle: every entry of dx and of every
    weight gradient, with a mask, at a size where the contraction, both LayerNorms and the
    gates all matter (a transposed contraction index or a dropped gate term fails here)."""
    rng = np.random.default_rng(23 if direction == "outgoing" else 29)
    x, mask, dout, w = _trimul_case(rng, 2, 3, 4, 2)
    grads = O.trimul_grad(x, direction, mask, dout, **w)

    def loss(xx, ww):
        return float(np.sum(O.trimul(xx, direction, mask, **ww) * dout))

    h = 1e-6
    params = {"x": x, **w}
    for name, base in params.items():
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            plus, minus = base.copy(), base.copy()
            plus[idx] += h
            minus[idx] -= h
            if name == "x":
                num[idx] = (loss(plus, w) - loss(minus, w)) / (2 * h)
            else:
                num[idx] = (loss(x, {**w, name: plus}) - loss(x, {**w, name: minus})) / (2 * h)
        np.testing.assert_allclose(grads[name], num, rtol=1e-5, atol=1e-7, err_msg=name)


def test_trimul_grad_without_optional_weights():
    """LayerNorm affines and projection biases omitted: their gradients are None and the rest
    still match finite differences of the forward."""
    rng = np.random.default_rng(31)
    x, mask, dout, w = _trimul_case(rng, 1, 3, 4, 2)
    w = {k: v for k, v in w.items() if k.endswith("weight") and not k.startswith("norm")}
    grads = O.trimul_grad(x, "incoming", None, dout, **w)
    assert grads["norm_in_weight"] is None and grads["p_out_bias"] is None
    h = 1e-6
    num = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        plus, minus = x.copy(), x.copy()
        plus[idx] += h
        minus[idx] -= h
        num[idx] = (np.sum(O.trimul(plus, "incoming", None, **w) * dout)
                    - np.sum(O.trimul(minus, "incoming", None, **w) * dout)) / (2 * h)
    np.testing.assert_allclose(grads["x"], num, rtol=1e-5, atol=1e-7)


def test_layer_norm_grad_matches_finite_differences():
    rng = np.random.default_rng(37)
    x = rng.standard_normal((3, 7))
    wt = 1 + 0.3 * rng.standard_normal(7)
    b = 0.3 * rng.standard_normal(7)
    dy = rng.standard_normal((3, 7))
    dx, dw, db = O.layer_norm_grad(x, dy, wt)
    h = 1e-6
    for name, base, g in (("x", x, dx), ("w", wt, dw), ("b", b, db)):
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            args = {"x": x, "w": wt, "b": b}
            plus, minus = base.copy(), base.copy()
            plus[idx] += h
            minus[idx] -= h
            num[idx] = (np.sum(O.layer_norm(**{**{"x": x, "weight": wt, "bias": b},
                                                **{{"x": "x", "w": "weight", "b": "bias"}[name]: plus}}) * dy)
                        - np.sum(O.layer_norm(**{**{"x": x, "weight": wt, "bias": b},
                                                  **{{"x": "x", "w": "weight", "b": "bias"}[name]: minus}}) * dy)
                        ) / (2 * h)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-8, err_msg=name)


# ---------------------------------------------------------------------------------- metrics
def test_rel_fro_known_answers():
    """``rel_fro(a, b) = ||a - b|| / ||b||`` with ``b`` the reference (testutil/metrics.py:40-47):
    the denominator is the second argument, so (2b, b) gives 1 and (b, 2b) gives 1/2."""
    b = RNG(0).standard_normal((4, 8))
    assert O.rel_fro(b, b) == 0.0
    assert O.rel_fro(2 * b, b) == pytest.approx(1.0, abs=1e-15)
    assert O.rel_fro(b, 2 * b) == pytest.approx(0.5, abs=1e-15)
    assert O.rel_fro(-b, b) == pytest.approx(2.0, abs=1e-15)
    # a 3-4-5 triangle: ||(3, 4) - (0, 0)|| against a unit reference
    assert O.rel_fro(np.array([3.0, 4.0, 1.0]), np.array([0.0, 0.0, 1.0])) == pytest.approx(5.0, abs=1e-15)
    # shape-agnostic: the Frobenius norm of the flattened arrays
    assert O.rel_fro(2 * b.reshape(32), b.reshape(32)) == pytest.approx(1.0, abs=1e-15)
    # a zero reference is clamped, not divided by (the reference clamps at 1e-30)
    assert O.rel_fro(np.zeros(3), np.zeros(3)) == 0.0
    assert O.rel_fro(np.full(3, 1e-20), np.zeros(3)) > 1e9


def test_cos_known_answers():
    """Cosine of the flattened arrays; two zero arrays count as 1 and one zero side as 0
    (testutil/metrics.py:26-37, tests/test_metrics.py:14-38)."""
    b = RNG(1).standard_normal((4, 8))
    zero = np.zeros((4, 8))
    assert O.cos(zero, zero) == 1.0
    assert O.cos(zero, np.ones((4, 8))) == 0.0
    assert O.cos(np.ones((4, 8)), zero) == 0.0
    assert O.cos(b, b) == pytest.approx(1.0, abs=1e-15)
    assert O.cos(3 * b, b) == pytest.approx(1.0, abs=1e-15)
    assert O.cos(-b, b) == pytest.approx(-1.0, abs=1e-15)
    assert O.cos(np.array([1.0, 0.0]), np.array([0.0, 1.0])) == 0.0
    assert O.cos(np.array([1.0, 1.0]), np.array([1.0, 0.0])) == pytest.approx(2 ** -0.5, abs=1e-15)
    assert math.isnan(O.cos(np.array([np.nan, 1.0]), np.array([1.0, 1.0])))


def test_assert_close_to_oracle_rejects_mismatches():
    """The GPU parity gate (tests/helpers.py) fails on a scaled, sign-flipped, non-finite or
    reshaped candidate and on a zero candidate against a non-zero oracle, and passes the exact
    match and two zero tensors (tests/test_metrics.py:14-38)."""
    from helpers import Tolerance, assert_close_to_oracle

    tol = Tolerance(1.0 - 1e-4, 1e-2)
    want = RNG(2).standard_normal((4, 8))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    assert assert_close_to_oracle("exact", t(want), want, tol) == (pytest.approx(1.0), 0.0)
    assert assert_close_to_oracle("zeros", t(np.zeros((4, 8))), np.zeros((4, 8)), tol) == (1.0, 0.0)
    bad = {
        "scaled": 1.05 * want,  # cosine 1, rel-Fro 0.05
        "negated": -want,
        "zero": np.zeros_like(want),
        "nan": np.where(np.arange(32).reshape(4, 8) == 5, np.nan, want),
        "transposed": want.T,
    }
    for name, got in bad.items():
        with pytest.raises(AssertionError):
            assert_close_to_oracle(name, t(got), want, tol)
    # the north star's 1e-2 cap tightens a looser table entry
    with pytest.raises(AssertionError):
        assert_close_to_oracle("capped", t(1.02 * want), want, Tolerance(1.0 - 1e-4, 5e-2), rel_fro_max=1e-2)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_pixels_from_lines_is_the_full_oracle(direction):
    """The large-N tests' pixel oracle (helpers.trimul_pixels: trimul_grid on the needed grid
    lines with the output gate re-taken at the true pixel) equals the full oracle there."""
    from helpers import pair_input, trimul_pixels, trimul_weights

    N = 14
    w = trimul_weights(32, 16, torch.float64, seed=5, biases=True, ln_random=True)
    x, mask = pair_input(1, N, 32, torch.float64, seed=6)
    full = O.trimul(x.numpy(), direction, mask.numpy(), **{k: v.numpy() for k, v in w.items()})
    rows, cols = [1, N - 4, N - 1], [0, N - 3, N - 1]
    got = trimul_pixels(x, mask, w, direction, rows, cols)
    np.testing.assert_allclose(got, full[:, rows][:, :, cols], rtol=1e-12, atol=1e-12)
