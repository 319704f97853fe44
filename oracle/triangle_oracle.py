"""CPU oracle for the triangle hot path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's pure-torch math, used by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, and only as the checker (or
the timed CPU baseline). The product (geometric-nn-ops_amd/) never imports it.

Reference files followed (paths relative to AMDResearch/geometric-nn-ops):
  * mask_val / masked_key_bias          geometric_nn_ops_torch/triangle/_masking.py:13-42
  * triangle_attention                  geometric_nn_ops_torch/triangle/_reference/triangle_attention.py:11-44
  * trimul (LayerNorm, gated projection, mask, combine, output LN, projection, gate)
                                        geometric_nn_ops_torch/triangle/_reference/trimul.py:27-97
  * layer_norm semantics                torch.nn.functional.layer_norm (biased variance,
                                        1/sqrt(var + eps)), called at _reference/trimul.py:85,94
  * triangle_attention_grad (dq, dk, dv, N_seq-summed dbias): the autograd of
    _reference/triangle_attention.py:11-44 written out
  * trimul_grad / layer_norm_grad (dx and every weight gradient): the autograd of
    _reference/trimul.py:57-97 written out (the reference itself has no other backward)
  * attention_pair_bias (pair-bias projection, multiplicity broadcast, key mask with a
    caller-given magnitude, gate from s, output projection)
                                        geometric_nn_ops_torch/triangle/_reference/attention_pair_bias.py:17-89

Everything is computed in ``dtype`` (float64 by default). How each function is pinned
(tests/test_oracle.py): triangle_attention against a pure-Python loop softmax-attention
at tiny sizes and the reference's known-answer cases (one live key gives v, zero q gives
mean(v), masked keys are bit-invariant to noise, fully masked rows give mean(v));
combine against pure-Python triple loops for both directions; layer_norm against its
closed-form moments and the zero-vector -> beta case; trimul end to end against the
N = 1 closed form and the fully-masked constant field; mask_val against the reference's
stated sentinel values; attention_pair_bias against a pure-Python per-element loop at tiny
sizes, against triangle_attention with N_seq = the multiplicity (the shared-bias
identity), and the reference's known answers (masked keys ignored, cached bias equal to the
recomputed one, copies with equal inputs equal, a per-batch mask equal to its per-copy
repetition); triangle_attention_grad against central finite differences of
triangle_attention (every input, with bias and mask); trimul_grad and layer_norm_grad against
central finite differences of trimul / layer_norm (every input and weight, both directions,
with a mask).
"""

from __future__ import annotations

import numpy as np

DIRECTIONS = ("outgoing", "incoming")


# ---------------------------------------------------------------- masking (_masking.py:13-42)
def mask_val(dtype_name: str) -> float:
    """Sentinel magnitude per dtype name: fp64 1e18, fp32/bf16 1e9, fp16 finfo.max/2."""
    if dtype_name == "float64":
        return 1e18
    if dtype_name in ("float32", "bfloat16"):
        return 1e9
    if dtype_name == "float16":
        return float(np.finfo(np.float16).max) / 2
    raise ValueError(f"Unsupported dtype {dtype_name}")


def masked_key_bias(mask: np.ndarray, dtype=np.float64, dtype_name: str = "float64") -> np.ndarray:
    """``mask_val * (mask - 1)``: +0.0 on kept keys, -mask_val on masked ones."""
    return mask_val(dtype_name) * (mask.astype(dtype) - 1)


# ------------------------------------------- triangle attention (_reference/triangle_attention.py)
def _softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def triangle_attention(q, k, v, bias=None, mask=None, scale=None, *, dtype=np.float64,
                       s_chunk: int | None = None) -> np.ndarray:
    """Triangle attention on the canonical 5D layout ``[B, N_seq, N_res, H, D]``.

    ``bias`` broadcastable to ``[B, 1, H, N, N]`` (4D ``[B, H, N, N]`` gains the N_seq
    axis); ``mask`` boolean broadcastable to ``[B, N_seq, 1, 1, N]``. Logits are
    ``(q * scale) . k + bias + masked_key_bias(mask)`` (triangle_attention.py:34-40), the
    softmax runs over keys (:42) and the output is ``P @ v`` (:43). ``s_chunk`` processes
    the N_seq axis in chunks to bound memory (the math is row-independent).
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    B, S, N, H, D = q.shape
    if scale is None:
        scale = D ** -0.5
    if bias is not None:
        bias = np.asarray(bias, dtype=dtype)
        if bias.ndim == 4:
            bias = bias[:, None]
        bias = np.broadcast_to(bias, (B, 1, H, N, N))
    if mask is not None:
        mask = np.broadcast_to(np.asarray(mask, dtype=bool), (B, S, 1, 1, N))
        name = "float64" if dtype == np.float64 else "float32"
        mbias = masked_key_bias(mask, dtype, name)  # [B, S, 1, 1, N]
    out = np.empty((B, S, N, H, D), dtype=dtype)
    step = s_chunk or S
    for s0 in range(0, S, step):
        s1 = min(S, s0 + step)
        qs = np.transpose(q[:, s0:s1], (0, 1, 3, 2, 4)) * dtype(scale)  # [B, s, H, N, D]
        ks = np.transpose(k[:, s0:s1], (0, 1, 3, 2, 4))
        vs = np.transpose(v[:, s0:s1], (0, 1, 3, 2, 4))
        logits = qs @ np.swapaxes(ks, -1, -2)  # [B, s, H, N, N]
        if bias is not None:
            logits = logits + bias
        if mask is not None:
            logits = logits + mbias[:, s0:s1]
        probs = _softmax(logits, -1)
        out[:, s0:s1] = np.transpose(probs @ vs, (0, 1, 3, 2, 4))
    return out


def triangle_attention_lse_max(q, k, bias=None, mask=None, scale=None, *, mask_value=None,
                               dtype=np.float64):
    """Per-query natural-log log-sum-exp and maximum of triangle_attention's logits, each
    ``[B, N_seq, H, N_res]``: the auxiliary outputs of cueq's triangle_attention(return_aux)
    (the reference's shim refuses them, hipequivariance_ops_torch/cuequivariance_ops_torch/
    triangle_attention.py:34-38). Masked keys get ``mask_value`` (default: the dtype's
    sentinel, as in ``triangle_attention``)."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    B, S, N, H, D = q.shape
    if scale is None:
        scale = D ** -0.5
    qs = np.transpose(q, (0, 1, 3, 2, 4)) * dtype(scale)
    ks = np.transpose(k, (0, 1, 3, 2, 4))
    logits = qs @ np.swapaxes(ks, -1, -2)  # [B, S, H, N, N]
    if bias is not None:
        bias = np.asarray(bias, dtype=dtype)
        if bias.ndim == 4:
            bias = bias[:, None]
        logits = logits + np.broadcast_to(bias, (B, 1, H, N, N))
    if mask is not None:
        mask = np.broadcast_to(np.asarray(mask, dtype=bool), (B, S, 1, 1, N))
        if mask_value is None:
            name = "float64" if dtype == np.float64 else "float32"
            logits = logits + masked_key_bias(mask, dtype, name)
        else:
            logits = logits + np.where(mask, 0.0, mask_value).astype(dtype)
    mx = logits.max(-1)
    lse = mx + np.log(np.exp(logits - mx[..., None]).sum(-1))
    return lse, mx


# ------------------------------------------------------------- trimul (_reference/trimul.py)
def is_outgoing(direction: str) -> bool:
    if direction not in DIRECTIONS:
        raise ValueError(f"direction must be one of {DIRECTIONS}, got {direction!r}")
    return direction == "outgoing"


def layer_norm(x, weight=None, bias=None, eps=1e-5, *, dtype=np.float64) -> np.ndarray:
    """LayerNorm over the last axis with torch's semantics: biased variance and
    ``(x - mean) / sqrt(var + eps) * weight + bias``."""
    x = np.asarray(x, dtype=dtype)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + dtype(eps))
    if weight is not None:
        y = y * np.asarray(weight, dtype=dtype)
    if bias is not None:
        y = y + np.asarray(bias, dtype=dtype)
    return y


def linear(x, weight, bias=None, *, dtype=np.float64) -> np.ndarray:
    """``x @ weight.T + bias`` with ``weight`` in nn.Linear layout ``[out, in]``."""
    y = np.asarray(x, dtype=dtype) @ np.asarray(weight, dtype=dtype).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=dtype)
    return y


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def combine(a, b, outgoing: bool) -> np.ndarray:
    """outgoing ``o[..., i, j, c] = sum_k a[..., i, k, c] b[..., j, k, c]``;
    incoming ``o[..., i, j, c] = sum_k a[..., k, i, c] b[..., k, j, c]``
    (_reference/trimul.py:44-54), evaluated as one matmul per channel. The channel-major
    copies are contiguous: numpy's matmul on the strided moveaxis views takes a non-BLAS
    loop (about 100x slower at N = 256)."""
    am = np.ascontiguousarray(np.moveaxis(a, -1, -3))  # [..., C, N, N]
    bm = np.ascontiguousarray(np.moveaxis(b, -1, -3))
    if outgoing:
        o = am @ np.swapaxes(bm, -1, -2)
    else:
        o = np.swapaxes(am, -1, -2) @ bm
    return np.moveaxis(o, -3, -1)


def trimul_stages(x, direction="outgoing", mask=None, *, eps=1e-5, dtype=np.float64, **w):
    """Every intermediate of the triangle multiplicative update, as a dict:
    z (LN-in), a, b (masked gated projections), g (output gate), o (contraction),
    on (LN-out), out (the op's result). Weight keywords as the public op."""
    outgoing = is_outgoing(direction)
    x = np.asarray(x, dtype=dtype)
    c_hidden = np.asarray(w["p_in_weight"]).shape[0] // 2
    z = layer_norm(x, w.get("norm_in_weight"), w.get("norm_in_bias"), eps, dtype=dtype)
    p = linear(z, w["p_in_weight"], w.get("p_in_bias"), dtype=dtype) * sigmoid(
        linear(z, w["g_in_weight"], w.get("g_in_bias"), dtype=dtype))
    if mask is not None:
        p = p * np.asarray(mask, dtype=dtype)[..., None]
    a, b = p[..., :c_hidden], p[..., c_hidden:]
    o = combine(a, b, outgoing)
    on = layer_norm(o, w.get("norm_out_weight"), w.get("norm_out_bias"), eps, dtype=dtype)
    g = sigmoid(linear(z, w["g_out_weight"], w.get("g_out_bias"), dtype=dtype))
    out = linear(on, w["p_out_weight"], w.get("p_out_bias"), dtype=dtype) * g
    return dict(z=z, a=a, b=b, g=g, o=o, on=on, out=out)


def trimul(x, direction="outgoing", mask=None, *, eps=1e-5, dtype=np.float64, **w) -> np.ndarray:
    """Triangle multiplicative update (_reference/trimul.py:57-97)."""
    return trimul_stages(x, direction, mask, eps=eps, dtype=dtype, **w)["out"]


def trimul_grid(x, direction="outgoing", mask=None, rows=(0,), cols=(0,), *, eps=1e-5,
                dtype=np.float64, **w) -> np.ndarray:
    """``trimul(...)[..., rows, :, :][..., :, cols, :]`` computed from the rows / columns of
    x those pixels depend on, for checking sizes where the full N^3 product is too slow on
    the CPU. Same math as trimul_stages (_reference/trimul.py:57-97): out[i, j] needs
    a[i, k] and b[j, k] for all k ('outgoing', rows i and j of the pair grid) or a[k, i] and
    b[k, j] ('incoming', columns), plus the gate of pixel (i, j) itself."""
    outgoing = is_outgoing(direction)
    x = np.asarray(x, dtype=dtype)
    rows, cols = list(rows), list(cols)
    c_hidden = np.asarray(w["p_in_weight"]).shape[0] // 2
    m = None if mask is None else np.broadcast_to(np.asarray(mask, dtype=dtype), x.shape[:-1])

    def gated(sel_x, sel_m):
        z = layer_norm(sel_x, w.get("norm_in_weight"), w.get("norm_in_bias"), eps, dtype=dtype)
        p = linear(z, w["p_in_weight"], w.get("p_in_bias"), dtype=dtype) * sigmoid(
            linear(z, w["g_in_weight"], w.get("g_in_bias"), dtype=dtype))
        return p if sel_m is None else p * sel_m[..., None]

    if outgoing:  # [..., R, N, 2Ch] from rows, contract over the column index k
        pr = gated(x[..., rows, :, :], None if m is None else m[..., rows, :])
        pc = gated(x[..., cols, :, :], None if m is None else m[..., cols, :])
        o = np.einsum("...ikc,...jkc->...ijc", pr[..., :c_hidden], pc[..., c_hidden:])
    else:  # [..., N, R, 2Ch] from columns, contract over the row index k
        pr = gated(x[..., :, rows, :], None if m is None else m[..., :, rows])
        pc = gated(x[..., :, cols, :], None if m is None else m[..., :, cols])
        o = np.einsum("...kic,...kjc->...ijc", pr[..., :c_hidden], pc[..., c_hidden:])
    on = layer_norm(o, w.get("norm_out_weight"), w.get("norm_out_bias"), eps, dtype=dtype)
    xg = x[..., rows, :, :][..., :, cols, :]
    zg = layer_norm(xg, w.get("norm_in_weight"), w.get("norm_in_bias"), eps, dtype=dtype)
    g = sigmoid(linear(zg, w["g_out_weight"], w.get("g_out_bias"), dtype=dtype))
    return linear(on, w["p_out_weight"], w.get("p_out_bias"), dtype=dtype) * g


# ------------------------------------------------ trimul gradients (autograd of the reference's
# trimul_torch, _reference/trimul.py:57-97, written out)
def layer_norm_grad(x, dy, weight=None, eps=1e-5, *, dtype=np.float64):
    """``(dx, dweight, dbias)`` of ``sum(layer_norm(x, weight, bias) * dy)`` over the last
    axis; the weight / bias gradients are summed over every leading axis."""
    x = np.asarray(x, dtype=dtype)
    dy = np.asarray(dy, dtype=dtype)
    mean = x.mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(((x - mean) ** 2).mean(axis=-1, keepdims=True) + dtype(eps))
    xh = (x - mean) * rstd
    g = dy if weight is None else dy * np.asarray(weight, dtype=dtype)
    dx = rstd * (g - g.mean(axis=-1, keepdims=True) - xh * (g * xh).mean(axis=-1, keepdims=True))
    lead = tuple(range(x.ndim - 1))
    return dx, (dy * xh).sum(axis=lead), dy.sum(axis=lead)


def trimul_grad(x, direction="outgoing", mask=None, dout=None, *, eps=1e-5, dtype=np.float64, **w):
    """Gradients of ``sum(trimul(x, ...) * dout)``: a dict with ``"x"`` and one entry per
    weight keyword (None where the weight is None). Weight gradients are summed over the
    pixels and every batch axis; the mask gets none (the reference's mask is data)."""
    outgoing = is_outgoing(direction)
    x = np.asarray(x, dtype=dtype)
    dout = np.asarray(dout, dtype=dtype)
    W = {k: (None if v is None else np.asarray(v, dtype=dtype)) for k, v in w.items()}
    c_hidden = W["p_in_weight"].shape[0] // 2
    lead = tuple(range(x.ndim - 1))

    def lin(t, wk, bk):
        return linear(t, W[wk], W.get(bk), dtype=dtype)

    z = layer_norm(x, W.get("norm_in_weight"), W.get("norm_in_bias"), eps, dtype=dtype)
    lp, lg, lgo = lin(z, "p_in_weight", "p_in_bias"), lin(z, "g_in_weight", "g_in_bias"), \
        lin(z, "g_out_weight", "g_out_bias")
    sg, sgo = sigmoid(lg), sigmoid(lgo)
    m = np.ones(x.shape[:-1] + (1,), dtype) if mask is None else \
        np.broadcast_to(np.asarray(mask, dtype=dtype), x.shape[:-1])[..., None]
    ab = lp * sg * m
    a, b = ab[..., :c_hidden], ab[..., c_hidden:]
    o = combine(a, b, outgoing)
    on = layer_norm(o, W.get("norm_out_weight"), W.get("norm_out_bias"), eps, dtype=dtype)
    y = lin(on, "p_out_weight", "p_out_bias")
    # out = y * sgo
    dy = dout * sgo
    dlgo = dout * y * sgo * (1 - sgo)
    def outer(d, t):  # sum over every leading axis of d[..., o] t[..., i]
        return d.reshape(-1, d.shape[-1]).T @ t.reshape(-1, t.shape[-1])

    gr = {"p_out_weight": outer(dy, on), "p_out_bias": dy.sum(axis=lead)}
    don = dy @ W["p_out_weight"]
    do, gr["norm_out_weight"], gr["norm_out_bias"] = layer_norm_grad(o, don, W.get("norm_out_weight"), eps,
                                                                     dtype=dtype)
    if outgoing:  # o[i, j] = sum_k a[i, k] b[j, k]
        da = np.einsum("...ijc,...jkc->...ikc", do, b)
        db = np.einsum("...ijc,...ikc->...jkc", do, a)
    else:  # o[i, j] = sum_k a[k, i] b[k, j]
        da = np.einsum("...ijc,...kjc->...kic", do, b)
        db = np.einsum("...ijc,...kic->...kjc", do, a)
    dab = np.concatenate([da, db], axis=-1)
    dlp = dab * sg * m
    dlg = dab * lp * m * sg * (1 - sg)
    for name, d in (("p_in", dlp), ("g_in", dlg), ("g_out", dlgo)):
        gr[f"{name}_weight"] = outer(d, z)
        gr[f"{name}_bias"] = d.sum(axis=lead)
    dz = dlp @ W["p_in_weight"] + dlg @ W["g_in_weight"] + dlgo @ W["g_out_weight"]
    dx, gr["norm_in_weight"], gr["norm_in_bias"] = layer_norm_grad(x, dz, W.get("norm_in_weight"), eps,
                                                                   dtype=dtype)
    out = {"x": dx}
    for key in ("norm_in_weight", "norm_in_bias", "p_in_weight", "p_in_bias", "g_in_weight", "g_in_bias",
                "norm_out_weight", "norm_out_bias", "p_out_weight", "p_out_bias", "g_out_weight",
                "g_out_bias"):
        out[key] = None if W.get(key) is None else gr[key]
    return out


# ------------------------------------------------------------------------- metrics
def rel_fro(a, b) -> float:
    """``||a - b|| / ||b||`` in fp64; ``b`` is the reference (testutil/metrics.py:40-47)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm((a - b).ravel()) / max(np.linalg.norm(b.ravel()), 1e-30))


def cos(a, b) -> float:
    """Cosine similarity of the flattened arrays; two zero arrays count as 1
    (testutil/metrics.py:26-37)."""
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / max(na * nb, 1e-300))


# ------------------------------- attention with pair bias (_reference/attention_pair_bias.py)
def pair_bias_projection(z, ln_z_weight, proj_z_weight, eps=1e-5, *, dtype=np.float64) -> np.ndarray:
    """``z [B, U, V, Zc]`` -> per-head bias ``[B, H, U, V]``: LayerNorm over ``Zc`` with no
    beta, then the bias-free projection to H heads (attention_pair_bias.py:17-22)."""
    zc = layer_norm(z, ln_z_weight, None, eps, dtype=dtype)
    pz = linear(zc, proj_z_weight, None, dtype=dtype)  # [B, U, V, H]
    return np.ascontiguousarray(np.transpose(pz, (0, 3, 1, 2)))


def attention_pair_bias(s, q, k, v, z, *, proj_g_weight, proj_o_weight, proj_z_weight=None,
                        ln_z_weight=None, proj_g_bias=None, proj_o_bias=None, mask=None,
                        scale=None, inf=None, eps=1e-5, z_is_projected=False,
                        return_z_proj=False, dtype=np.float64):
    """Attention with pair bias (attention_pair_bias.py:25-89).

    q ``[B*M, H, U, DH]``, k / v ``[B*M, H, V, DH]``, s ``[B*M, U, H*DH]``; z the pair rep
    ``[B, U, V, Zc]`` (or the projected bias ``[B, H, U, V]`` with ``z_is_projected``);
    mask ``[B, V]`` or ``[B*M, V]`` with 1 = keep, pushing masked logits down by ``inf``
    (``None``: the dtype's mask_val). Returns ``(out [B*M, U, H*DH], bias or None)``.
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    BM, H, U, DH = q.shape
    V = k.shape[2]
    B = np.asarray(z).shape[0]
    if BM % B != 0:
        raise ValueError(f"q batch {BM} is not a multiple of z batch {B}")
    M = BM // B
    if scale is None:
        scale = DH ** -0.5
    pz = np.asarray(z, dtype=dtype) if z_is_projected else pair_bias_projection(
        z, ln_z_weight, proj_z_weight, eps, dtype=dtype)
    qm = q.reshape(B, M, H, U, DH)
    km = k.reshape(B, M, H, V, DH)
    vm = v.reshape(B, M, H, V, DH)
    logits = (qm @ np.swapaxes(km, -1, -2)) * dtype(scale) + pz[:, None]  # [B, M, H, U, V]
    if mask is not None:
        mask = np.asarray(mask, dtype=dtype)
        if mask.shape[0] == B:
            keep = mask.reshape(B, 1, 1, 1, V)
        elif mask.shape[0] == BM:
            keep = mask.reshape(B, M, 1, 1, V)
        else:
            raise ValueError(f"mask batch {mask.shape[0]} must be B={B} or BM={BM}")
        if inf is None:
            inf = mask_val("float64" if dtype == np.float64 else "float32")
        logits = logits + (keep - 1.0) * dtype(inf)
    o = _softmax(logits, -1) @ vm  # [B, M, H, U, DH]
    o = np.transpose(o.reshape(BM, H, U, DH), (0, 2, 1, 3)).reshape(BM, U, H * DH)
    g = sigmoid(linear(s, proj_g_weight, proj_g_bias, dtype=dtype))
    out = linear(o * g, proj_o_weight, proj_o_bias, dtype=dtype)
    return out, (pz if return_z_proj else None)


# --------------------------------------------- triangle attention gradients (autograd of the
# reference's triangle_attention_torch, _reference/triangle_attention.py:11-44)
def triangle_attention_grad(q, k, v, bias, mask, scale, dout, *, dtype=np.float64):
    """Gradients ``(dq, dk, dv, dbias)`` of ``sum(triangle_attention(...) * dout)`` on the
    canonical layout; ``dbias`` has the bias's ``[B, 1, H, N, N]`` shape (summed over
    N_seq, where the bias is broadcast), ``None`` without a bias."""
    q, k, v, dout = (np.asarray(t, dtype=dtype) for t in (q, k, v, dout))
    B, S, N, H, D = q.shape
    if scale is None:
        scale = D ** -0.5
    tr = lambda t: np.transpose(t, (0, 1, 3, 2, 4))  # noqa: E731  [B, S, H, N, D]
    qs, ks, vs, dos = tr(q), tr(k), tr(v), tr(dout)
    logits = (qs * dtype(scale)) @ np.swapaxes(ks, -1, -2)
    if bias is not None:
        bias = np.broadcast_to(np.asarray(bias, dtype=dtype), (B, 1, H, N, N))
        logits = logits + bias
    if mask is not None:
        mask = np.broadcast_to(np.asarray(mask, dtype=bool), (B, S, 1, 1, N))
        logits = logits + masked_key_bias(mask, dtype, "float64" if dtype == np.float64 else "float32")
    p = _softmax(logits, -1)                          # [B, S, H, N, N]
    o = p @ vs
    dv = np.swapaxes(p, -1, -2) @ dos
    dp = dos @ np.swapaxes(vs, -1, -2)
    delta = np.sum(dos * o, axis=-1, keepdims=True)
    ds = p * (dp - delta)
    dq = (ds @ ks) * dtype(scale)
    dk = (np.swapaxes(ds, -1, -2) @ qs) * dtype(scale)
    dbias = None if bias is None else ds.sum(axis=1, keepdims=True)
    return tr(dq), tr(dk), tr(dv), dbias
