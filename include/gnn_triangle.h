/*
 * gnn_triangle.h -- C ABI of libgnn_hip.so, the gfx950 (MI355X) implementation of the
 * inference forward of geometric_nn_ops_torch.triangle.{triangle_attention,
 * triangle_multiplicative_update}.
 *
 * Boundary rules
 *   - Plain pointers, sizes and strides only; no torch or HIP types in the signatures.
 *     `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *   - The caller owns every buffer: inputs, outputs and the trimul workspace. The
 *     library never allocates or frees device memory and keeps no global state except
 *     the thread-local error message, so every entry point is reentrant.
 *   - Strides are in ELEMENTS, not bytes. The innermost (head-dim / channel) stride
 *     must be 1.
 *   - Return value: GNN_OK (0), a negative GNN_ERR_* code, or a positive hipError_t
 *     from the launch. gnn_last_error() returns a message for the calling thread.
 *
 * Which reference interface each entry point replaces (paths relative to the
 * AMDResearch/geometric-nn-ops source tree):
 *   gnn_triattn_fwd   -> triangle_attention_triton / EvoformerAttention.forward /
 *                        _attn_fwd[grid] launch
 *                        (geometric_nn_ops_torch/triangle/_kernels/triangle_attention.py:1447,
 *                        :1091, :1213) plus masked_key_bias (triangle/_masking.py:35)
 *   gnn_trimul_fwd    -> trimul_triton (geometric_nn_ops_torch/triangle/_kernels/trimul.py:404)
 *   gnn_trimul_proj   -> triton_layernorm(x) + the g_in / p_in / g_out triton_linear_fused
 *                        calls (trimul.py:435-439, :445-447)
 *   gnn_trimul_contract -> _combine_projections' torch.einsum
 *                        (geometric_nn_ops_torch/triangle/_reference/trimul.py:44-54, called
 *                        from trimul.py:442)
 *   gnn_trimul_out    -> triton_layernorm(o) + p_out linear + the o*g gate (trimul.py:443-448)
 *   gnn_triattn_bwd   -> EvoformerAttention.backward (triangle_attention.py:1278-1442)
 *   gnn_pair_bias_proj -> _project_pair_bias of attention_pair_bias
 *                        (geometric_nn_ops_torch/triangle/_reference/attention_pair_bias.py:17-22)
 *   gnn_apb_gate_out   -> its gate and output projection (attention_pair_bias.py:86-89)
 *   gnn_layernorm_rows, gnn_trimul_gate_bwd -> the LayerNorm and gate nodes of autograd
 *                        through trimul_torch (triangle/_trimul.py:31-36,
 *                        triangle/_reference/trimul.py:57-97): the reference's trimul
 *                        backward, which has no native kernel
 *   gnn_trimul_contract_bwd, gnn_trimul_relayout -> the autograd products of the
 *                        contraction's einsum (triangle/_reference/trimul.py:44-54) and the
 *                        strided copies around them, in that same backward
 */
#ifndef GNN_TRIANGLE_H
#define GNN_TRIANGLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum gnn_dtype { GNN_F32 = 0, GNN_BF16 = 1, GNN_F16 = 2 };

/* Dot-product mode for fp32 operands (ignored for bf16/fp16, which always use their
 * native MFMA). IEEE = full fp32 MFMA; BF16X3 = each fp32 operand split into
 * hi+lo bf16 with three bf16 MFMAs (hi*hi + hi*lo + lo*hi), the mode torch's "tf32"
 * setting resolves to on gfx950 (geometric_nn_ops_torch/_precision.py:36-39). */
enum gnn_precision { GNN_PREC_IEEE = 0, GNN_PREC_BF16X3 = 1 };

enum gnn_status {
  GNN_OK = 0,
  GNN_ERR_ARG = -1,         /* bad shape / stride / pointer combination */
  GNN_ERR_UNSUPPORTED = -2, /* valid request this build does not implement */
  GNN_ERR_WORKSPACE = -3    /* workspace missing or too small */
};

/* ---------------------------------------------------------------------------------
 * Triangle attention forward.
 *   o[b,s,i,h,:] = softmax_j( scale * q[b,s,i,h,:].k[b,s,j,h,:] + mask_bias[b,s,j]
 *                             + bias[b,h,i,j] ) @ v[b,s,:,h,:]
 * Logical layouts are the public API's canonical 5D [B, S=N_seq, N=N_res, H, D]
 * (triangle/_triattn.py:64-73), addressed through explicit strides, so transposed
 * views (ending-node attention) need no copy.
 * mask_bias[b,s,j] = 0 where mask[b,s,j] != 0, else mask_value, added in fp32
 * (mask_value is the caller's mask_val(dtype) already rounded to the input dtype,
 * triangle/_masking.py:13-42, triangle_attention.py:1470).
 */
typedef struct gnn_triattn_args {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const void* bias;     /* [B,H,N,N] in the input dtype, or NULL for no pair bias */
  const uint8_t* mask;  /* bool [B,S,N] (nonzero = keep), or NULL for all-keep */
  float* lse;           /* optional fp32 [B,S,H,N] log-sum-exp (natural log), or NULL */
  float* row_max;       /* optional fp32 [B,S,H,N] largest logit of each query row, or NULL */
  int64_t B, S, N, H, D; /* D a multiple of 8, at most 256 (fp32: 128); N at most 32768 */
  int64_t q_stride[4];  /* strides of dims b, s, n, h (d stride must be 1) */
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  int64_t bias_stride[4]; /* b, h, i, j (any strides for 16-bit inputs with D <= 32 and
                             N <= 1024; otherwise j stride 1, i stride a multiple of 8) */
  int64_t mask_stride[3]; /* b, s, j */
  float scale;
  float mask_value;
  int32_t dtype;     /* enum gnn_dtype, shared by q, k, v, o, bias */
  int32_t precision; /* enum gnn_precision */
  void* workspace;   /* caller scratch of gnn_triattn_workspace_bytes(args) bytes (NULL when 0) */
  size_t workspace_bytes;
} gnn_triattn_args;

/* Replaces the forward launch of EvoformerAttention (triangle_attention.py:1091-1276). */
int gnn_triattn_fwd(const gnn_triattn_args* args, void* stream);

/* Bytes of device scratch gnn_triattn_fwd needs for these arguments (shapes, dtype, bias
 * present): the pair bias rewritten in the order the 16-bit row-resident kernel reads it
 * (B * H * ceil(N/32) * ceil(N/64) * 4 KB), 0 for calls that need none. No reference
 * counterpart: the reference's launcher reads the bias in place (triangle_attention.py:
 * 1231-1262). The scratch is only used during the call. */
size_t gnn_triattn_workspace_bytes(const gnn_triattn_args* args);

/* gnn_triattn_fwd without any allocation by the caller or the library: the scratch that
 * gnn_triattn_workspace_bytes() would ask for lives in a static 16 MiB device array of the
 * library instead (args->workspace is ignored). No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid it). Calls needing more scratch than 16 MiB (B * H * ceil(N/32) *
 * ceil(N/64) * 4 KB, e.g. B * H > 16 at N_res = 1024) return GNN_ERR_UNSUPPORTED. Every
 * call on one device shares that device's array: calls that overlap on one device (other
 * streams or threads) race. */
int gnn_triattn_fwd_noalloc(const gnn_triattn_args* args, void* stream);

/* ---------------------------------------------------------------------------------
 * Triangle attention backward (head dim a multiple of 8: bf16 / fp16 up to 128; fp32 up to
 * 64, its products full fp32 (precision GNN_PREC_IEEE) or split into bf16 hi / lo parts
 * (GNN_PREC_BF16X3), as the forward that wrote the lse ran them).
 * Given the forward's inputs, its output o, the upstream gradient dout and the forward's
 * lse (fp32 [B, S, H, N] contiguous, natural log; gnn_triattn_fwd writes it when args->lse
 * is set), writes dq, dk, dv (input dtype, [B, S, N, H, D] by strides) and, when both bias
 * and dbias are given, the pair-bias gradient summed over N_seq into dbias (fp32
 * [B, H, N, N] contiguous). delta is caller-provided fp32 scratch of B * S * H * N floats;
 * with dbias_splits > 1 the N_seq rows are split into that many ranges whose partial sums
 * go to dbias_ws (dbias_splits * B * H * N * N floats) and are added in range order, so
 * the result does not depend on scheduling.
 * Same layout rules as gnn_triattn_args; scale, mask_value and the mask are the forward's.
 */
typedef struct gnn_triattn_bwd_args {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const void* bias;      /* [B,H,N,N] or NULL */
  const uint8_t* mask;   /* bool [B,S,N] or NULL */
  const float* lse;      /* fp32 [B,S,H,N] */
  void* dq;
  void* dk;
  void* dv;
  float* dbias;          /* fp32 [B,H,N,N] or NULL */
  float* delta;          /* fp32 scratch [B,S,H,N] */
  float* dbias_ws;       /* fp32 scratch [dbias_splits,B,H,N,N] when dbias_splits > 1 */
  int32_t dbias_splits;  /* N_seq ranges summed separately (1..min(N_seq, 64)), then added in order */
  int64_t B, S, N, H, D;
  int64_t q_stride[4];   /* b, s, n, h for every [B,S,N,H,D] tensor (d stride 1) */
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  int64_t do_stride[4];
  int64_t dq_stride[4];
  int64_t dk_stride[4];
  int64_t dv_stride[4];
  int64_t bias_stride[4]; /* b, h, i, j (j stride must be 1) */
  int64_t mask_stride[3]; /* b, s, j */
  float scale;
  float mask_value;
  int32_t dtype;
  int32_t precision;
} gnn_triattn_bwd_args;

/* Replaces the backward of EvoformerAttention
 * (geometric_nn_ops_torch/triangle/_kernels/triangle_attention.py:1278-1442: the
 * _attn_bwd_preprocess, _attn_bwd_dk_dv and _attn_bwd_dbias_dq launches). */
int gnn_triattn_bwd(const gnn_triattn_bwd_args* args, void* stream);

/* ---------------------------------------------------------------------------------
 * Triangle multiplicative update forward (reference math:
 * geometric_nn_ops_torch/triangle/_reference/trimul.py:57-97):
 *   z = LN_in(x);  p = (z Wp_in^T + bp_in) * sigmoid(z Wg_in^T + bg_in) * mask
 *   a = p[..., :Ch], b = p[..., Ch:]
 *   outgoing: o[i,j,c] = sum_k a[i,k,c] b[j,k,c];  incoming: o[i,j,c] = sum_k a[k,i,c] b[k,j,c]
 *   out = (LN_out(o) Wp_out^T + bp_out) * sigmoid(z Wg_out^T + bg_out)
 * x and out are contiguous [B, N, N, C]. Every weight is contiguous in nn.Linear
 * layout ([out, in]) and in the input dtype; any bias / LayerNorm parameter may be
 * NULL (zero bias, unit LayerNorm weight). p_in_w and g_in_w are the concatenated
 * [a; b] projections, [2*Ch, C].
 */
typedef struct gnn_trimul_args {
  const void* x;
  void* out;
  const void* mask;   /* [B,N,N] in the input dtype via strides, or NULL */
  int64_t mask_stride[3]; /* b, i, j */
  const void* ln_in_w;
  const void* ln_in_b;
  const void* p_in_w;
  const void* p_in_b;
  const void* g_in_w;
  const void* g_in_b;
  const void* ln_out_w;
  const void* ln_out_b;
  const void* p_out_w;
  const void* p_out_b;
  const void* g_out_w;
  const void* g_out_b;
  void* workspace;
  size_t workspace_bytes;
  int64_t B, N, C, Ch;
  float eps;
  int32_t outgoing;  /* 1 = "outgoing", 0 = "incoming" */
  int32_t dtype;     /* enum gnn_dtype */
  int32_t precision; /* enum gnn_precision */
  /* Optional buffer for the output gate g ([B, N, N, C], input dtype, 16-byte aligned),
   * written by the projection stage and read by the output stage. NULL: the gate region of
   * the workspace. When set, the workspace needs only off[2] bytes (the gate region is laid
   * out last), so a caller keeping a, b and o for a backward can release g after the
   * forward. No reference counterpart. */
  void* gate;
  /* Channels the LayerNorms average over: LN-in over the first ln_in_channels of C, LN-out
   * over the first ln_out_channels of Ch (0: all). A caller whose widths are not multiples
   * of 32 pads x and the weights with zeros up to the next multiple (and the LayerNorm
   * weights and biases too, so the padded channels normalise to zero) and passes the real
   * widths here; the padded output channels then come out as zeros. No reference
   * counterpart: the reference's Triton kernels mask any width (trimul.py:310-314). */
  int64_t ln_in_channels;
  int64_t ln_out_channels;
} gnn_trimul_args;

/* Workspace size in bytes for one call (a, b, the output gate and o, each in the
 * input dtype), and the byte offsets of those four regions:
 *   off[0] a  channel-major, (i, k) of channel c (incoming: stored transposed per channel);
 *             bf16 / fp16: k-blocked [B, Ch, NP/32, N, 32], columns N .. NP-1 zero;
 *             fp32: row-major [B, Ch, N, NP]
 *   off[1] b  the same for b
 *   off[2] g  pixel-major   [B, N, N, C]    sigmoid(z Wg_out^T + bg_out); the last region
 *             (unused when gnn_trimul_args.gate is set)
 *   off[3] o  channel-major [B, Ch, N, NP]  the contraction output
 * where NP = N rounded up to a multiple of 32 (the row pitch; columns >= N of o unused).
 * No reference counterpart: the reference allocates its intermediates through torch
 * (trimul.py:253, :308). */
size_t gnn_trimul_workspace_bytes(int64_t B, int64_t N, int64_t C, int64_t Ch, int32_t dtype,
                                  size_t off[4]);

/* All three stages (the whole op) on one stream. Replaces trimul_triton (trimul.py:404-448). */
int gnn_trimul_fwd(const gnn_trimul_args* args, void* stream);

/* Stage 1: LayerNorm-in + [p_in; g_in] projections with sigmoid gate and mask, writing a
 * and b channel-major, and the output gate g. Replaces trimul.py:435-439, :445-447. */
int gnn_trimul_proj(const gnn_trimul_args* args, void* stream);

/* Stage 2: per-channel N x N x N contraction of a and b into o. It depends on the B * Ch
 * planes and N only, so it takes c_z and c_hidden above the 512 of stages 1 and 3 (the
 * wide-channel forward composes it with gnn_layernorm_rows and gnn_trimul_relayout).
 * Replaces _combine_projections (_reference/trimul.py:44-54) as called at trimul.py:442. */
int gnn_trimul_contract(const gnn_trimul_args* args, void* stream);

/* Stage 3: LayerNorm-out + p_out projection, multiplied by the gate g.
 * Replaces trimul.py:443-448. */
int gnn_trimul_out(const gnn_trimul_args* args, void* stream);

/* ---------------------------------------------------------------------------------
 * Pair-bias projection of attention with pair bias:
 *   out[b, h, u, v] = sum_c LN(z[b, u, v, :])[c] * proj_w[h, c]
 *   LN(x) = (x - mean) / sqrt(var + eps) * ln_w   (biased variance, no beta; the result is
 *   rounded to the input dtype before the projection, as F.layer_norm returns it)
 * z contiguous [B, U, V, Zc]; proj_w contiguous [H, Zc]; ln_w [Zc] or NULL (ones); out
 * [B, H, U, V] by strides (v stride 1), all in the input dtype. Zc a multiple of 8 and at
 * most 256, H * Zc at most 8192.
 */
typedef struct gnn_pair_bias_args {
  const void* z;
  const void* ln_w;
  const void* proj_w;
  void* out;
  int64_t B, U, V, Zc, H;
  int64_t out_stride[3]; /* b, h, u (v stride must be 1) */
  float eps;
  int32_t dtype; /* enum gnn_dtype, shared by every tensor */
} gnn_pair_bias_args;

/* Replaces _project_pair_bias (geometric_nn_ops_torch/triangle/_reference/
 * attention_pair_bias.py:17-22: F.layer_norm + F.linear + permute to [B, H, U, V]), the
 * pair-rep half of attention_pair_bias (triangle/_attention_pair_bias.py:11-98); the
 * attention itself runs on gnn_triattn_fwd with N_seq = the multiplicity. */
int gnn_pair_bias_proj(const gnn_pair_bias_args* args, void* stream);

/* Gate and output projection of attention with pair bias, fused:
 *   out = ( o * sigmoid(s g_w^T + g_b) ) o_w^T + o_b
 * with each product rounded to the input dtype as the reference's F.linear, torch.sigmoid
 * and multiply return it. s [M, Cs] (row pitch s_ld), o [M, D] (the attention output with
 * heads merged, row pitch o_ld), g_w [D, Cs], o_w [Co, D] contiguous, g_b [D] / o_b [Co] or
 * NULL, out [M, Co] (row pitch out_ld); one dtype for every tensor; fp32 products follow
 * `precision` like the other fp32 kernels. Cs, D and Co multiples of 32, rows 16-byte
 * aligned, and (Cs + D) small enough for the LDS tiles (up to 1024 + 1024 for 16-bit types,
 * 512 + 512 for fp32). */
typedef struct gnn_apb_gate_out_args {
  const void* s;
  const void* o;
  const void* g_w;
  const void* g_b;
  const void* o_w;
  const void* o_b;
  void* out;
  int64_t M, Cs, D, Co;
  int64_t s_ld, o_ld, out_ld;
  int32_t dtype;     /* enum gnn_dtype */
  int32_t precision; /* enum gnn_precision */
} gnn_apb_gate_out_args;

/* Replaces the gate and output projection of attention_pair_bias_torch
 * (geometric_nn_ops_torch/triangle/_reference/attention_pair_bias.py:86-89). */
int gnn_apb_gate_out(const gnn_apb_gate_out_args* args, void* stream);

/* ---------------------------------------------------------------------------------
 * Backward of the triangle multiplicative update. The reference has no native backward:
 * with gradients it runs trimul_torch under autograd (geometric_nn_ops_torch/triangle/
 * _trimul.py:31-36; math in triangle/_reference/trimul.py:57-97). The library's backward
 * differentiates that math with these two kernels plus vendor GEMMs for the plain matrix
 * products (geometric_nn_ops_torch/triangle/_kernels/trimul.py::trimul_bwd_hip).
 *
 * Row LayerNorm over the last K columns (F.layer_norm semantics: biased variance,
 * 1/sqrt(var + eps)), forward or backward:
 *   forward  (dy == NULL): out = (x - mean) * rstd * weight + bias
 *   backward (dy != NULL): xh = (x - mean) * rstd, g = dy * weight,
 *                          out = dx = rstd * (g - mean(g) - xh * mean(g * xh));
 *            and, if `partial` is set, partial[w][0][k] / partial[w][1][k] = the sums of
 *            dy * xh / dy over the rows workgroup w handled (w < gnn_layernorm_partials):
 *            the weight / bias gradients are their sums over w.
 * Every tensor in `dtype` except `partial` (fp32); rows addressed by row strides (elements),
 * columns contiguous; K a multiple of 32 and at most 512 (forward: at most 8192; rows wider
 * than 512 then need 16-byte aligned rows).
 */
typedef struct gnn_layernorm_args {
  const void* x;      /* [rows, K] */
  const void* dy;     /* NULL = forward; else [rows, K], the gradient of the output */
  const void* weight; /* [K] or NULL (ones) */
  const void* bias;   /* [K] or NULL (zeros); forward only */
  void* out;          /* [rows, K]: LN(x) (forward) or dx (backward) */
  float* partial;     /* backward, optional: [gnn_layernorm_partials(rows, K)][2][K] */
  int64_t rows, K;
  int64_t x_stride, dy_stride, out_stride;
  float eps;
  int32_t dtype; /* enum gnn_dtype */
} gnn_layernorm_args;

/* Replaces the LayerNorm autograd nodes of the reference's trimul_torch backward (the
 * F.layer_norm calls at triangle/_reference/trimul.py:85 and :94); no native counterpart. */
int64_t gnn_layernorm_partials(int64_t rows, int64_t K);
int gnn_layernorm_rows(const gnn_layernorm_args* args, void* stream);

/* Backward of out = value * sigmoid(gate_pre) * mask (mask per row, NULL = 1):
 *   d_value = grad * s * mask,  d_gate_pre = grad * value * mask * s * (1 - s),  s = sigmoid(gate_pre)
 * (with gate_is_sigmoid nonzero, gate_pre holds s itself: the forward's saved gate, which is
 * what torch's sigmoid backward uses).
 * [rows, K] tensors by row strides (columns contiguous, rows and bases 16-byte aligned),
 * mask [rows] by mask_stride, all in `dtype`; K a multiple of 8.
 * If `partial` is set, partial[w][0][k] / partial[w][1][k] receive the sums of the stored
 * (rounded) d_value / d_gate_pre over the rows workgroup w handled, w < gnn_gate_bwd_partials
 * (rows, K): the bias gradients of the two linear layers behind value and gate_pre are their
 * sums over w. gnn_gate_bwd_partials returns 0 for the K it cannot split this way (K / 8
 * must divide 256). */
typedef struct gnn_gate_bwd_args {
  const void* grad;
  const void* value;
  const void* gate_pre;
  const void* mask;
  void* d_value;
  void* d_gate_pre;
  float* partial; /* optional fp32 [gnn_gate_bwd_partials(rows, K)][2][K] */
  int64_t rows, K;
  int64_t grad_stride, value_stride, gate_stride, mask_stride, dv_stride, dg_stride;
  int32_t dtype;           /* enum gnn_dtype */
  int32_t gate_is_sigmoid; /* gate_pre holds sigmoid(gate_pre) */
} gnn_gate_bwd_args;

/* Replaces the sigmoid / multiply autograd nodes of the gated projections in the reference's
 * trimul_torch backward (triangle/_reference/trimul.py:86-90 and :95-97: p * sigmoid(g) * mask
 * and p_out(o) * sigmoid(g_out(z))); no native counterpart. */
int64_t gnn_gate_bwd_partials(int64_t rows, int64_t K);
int gnn_trimul_gate_bwd(const gnn_gate_bwd_args* args, void* stream);

/* The input side of the trimul backward in one pass over the pixel rows (16-bit dtypes,
 * C in {64, 128}, c_hidden <= 128): z = LN_in(x) is recomputed and written, the gated input
 * projections p = z p_in_w^T + p_in_b and g = z g_in_w^T + g_in_b (each rounded to the dtype)
 * are recomputed on MFMA tile by tile and never stored, and the backward of
 * a|b = p * sigmoid(g) * mask is applied to d_ab:
 *   d_p = d_ab * s * mask,  d_g = d_ab * p * mask * s * (1 - s),  s = sigmoid(g).
 * Replaces, in the reference's trimul_torch backward under autograd (triangle/_reference/
 * trimul.py:85-90), the recompute of F.layer_norm(x) and of the two input linears and the
 * sigmoid / multiply nodes behind a and b; no native counterpart (the reference has no trimul
 * backward kernel). Rows are pixels (any order); x [rows, C] by x_ld, mask [rows] by
 * mask_stride (NULL = 1), d_ab [rows, 2 Ch] by dab_ld, d_p / d_g [rows, 2 Ch] by dl_ld, z
 * [rows, C] contiguous; rows, bases and strides 16-byte aligned. partial[w][0][c] /
 * partial[w][1][c] receive the sums of the stored d_p / d_g over the rows workgroup w
 * handled, w < gnn_trimul_proj_bwd_partials(rows): the bias gradients of p_in and g_in are
 * their sums over w. */
typedef struct gnn_trimul_proj_bwd_args {
  const void* x;
  const void* ln_w; /* LN_in gamma [C] or NULL (ones) */
  const void* ln_b; /* LN_in beta [C] or NULL (zeros) */
  const void* p_in_w; /* [2 Ch, C] */
  const void* p_in_b; /* [2 Ch] or NULL */
  const void* g_in_w; /* [2 Ch, C] */
  const void* g_in_b; /* [2 Ch] or NULL */
  const void* mask;
  const void* d_ab;
  void* d_p;
  void* d_g;
  void* z;
  float* partial; /* fp32 [gnn_trimul_proj_bwd_partials(rows)][2][2 Ch] */
  int64_t rows, C, Ch;
  int64_t x_ld, dab_ld, dl_ld, mask_stride;
  float eps;
  int32_t dtype; /* GNN_BF16 or GNN_F16 */
} gnn_trimul_proj_bwd_args;
int64_t gnn_trimul_proj_bwd_partials(int64_t rows);
int gnn_trimul_proj_bwd(const gnn_trimul_proj_bwd_args* args, void* stream);

/* The output side of the trimul backward in one pass over 64-pixel tiles of the pair grid
 * (16-bit dtypes, C in {64, 128}, c_hidden in {32, 64, 128}): on = LN_out(o) from the
 * forward's channel-major o, y = on p_out_w^T + p_out_b (rounded to the dtype) recomputed on
 * MFMA, the backward of out = y * gate against the forward's saved gate,
 *   dy = dout * gate,  d_go = dout * y * gate * (1 - gate),
 * d(on) = dy p_out_w (rounded to the dtype) on MFMA and the LN_out backward
 *   x^ = (o - mean) * rstd,  g = d(on) * ln_w,  d_o = rstd * (g - mean(g) - x^ * mean(g * x^)).
 * Replaces, in the reference's trimul_torch backward under autograd (triangle/_reference/
 * trimul.py:91-97), the recompute of F.layer_norm(o) and of the p_out linear, the sigmoid-
 * gate / multiply nodes of the output gate, the input gradient of p_out and the LayerNorm's
 * backward; no native counterpart. o is [B, Ch, N, NP] (NP = round_up(N, 32), the
 * gnn_trimul_fwd workspace layout); gate, dout [B N N, C] and on, d_o [B N N, Ch] are
 * pixel-major rows (pixel (b, i, j) at (b N + i) N + j) in the dtype, dy [B N N, C]
 * contiguous, d_go [B N N, C] by dgo_ld (e.g. the g_out block of the input side's
 * [M, 4 Ch + C] gradient). partial[w][k][c] (k = 0: sum of dy, 1: of d_go over column c < C;
 * 2: of d(on) * x^, 3: of d(on) over column c < Ch) over the pixels workgroup w handled,
 * w < gnn_trimul_out_bwd_partials(B, N): the p_out / g_out bias gradients and the LN_out
 * weight / bias gradients are their sums over w. All pointers 16-byte aligned. */
typedef struct gnn_trimul_out_bwd_args {
  const void* o;
  const void* ln_w;    /* LN_out gamma [Ch] or NULL (ones) */
  const void* ln_b;    /* LN_out beta [Ch] or NULL (zeros) */
  const void* p_out_w; /* [C, Ch] */
  const void* p_out_b; /* [C] or NULL */
  const void* gate;
  const void* dout;
  void* on;
  void* dy;
  void* d_go;
  void* d_o;
  float* partial; /* fp32 [gnn_trimul_out_bwd_partials(B, N)][4][128] */
  int64_t B, N, C, Ch;
  int64_t dgo_ld;
  float eps;
  int32_t dtype; /* GNN_BF16 or GNN_F16 */
} gnn_trimul_out_bwd_args;
int64_t gnn_trimul_out_bwd_partials(int64_t B, int64_t N);
int gnn_trimul_out_bwd(const gnn_trimul_out_bwd_args* args, void* stream);

/* The two N^3 products of the contraction's backward, per (batch, channel) plane p < planes
 * (16-bit dtypes):
 *   dA_p[i][k] = sum_j dO_p[i][j] B_p[j][k],   dB_p[j][k] = sum_i dO_p[i][j] A_p[i][k].
 * A and B are the forward's workspace operands as gnn_trimul_fwd left them (k-blocked,
 * [planes][NP / 32][N][32], NP = round_up(N, 32): element (i, k) at ((k / 32) N + i) 32 + k % 32
 * of its plane). dO is given twice, column-blocked with its rows zero-padded to NP:
 *   do_i = [planes][NP / 32][NP][32], element (i, j) at ((i / 32) NP + j) 32 + i % 32 (zero for j >= N),
 *   do_j = [planes][NP / 32][NP][32], element (i, j) at ((j / 32) NP + i) 32 + j % 32 (zero for i >= N).
 * da / db = [planes][N][NP] row-major (columns N .. NP-1 not written). All pointers 16-byte
 * aligned, in `dtype`. */
typedef struct gnn_trimul_contract_bwd_args {
  const void* a;
  const void* b;
  const void* do_i;
  const void* do_j;
  void* da;
  void* db;
  int64_t planes; /* B * Ch */
  int64_t N;
  int32_t dtype;  /* GNN_BF16 or GNN_F16 */
  int32_t reserved;
} gnn_trimul_contract_bwd_args;

/* Replaces the autograd products of the einsum in _combine_projections
 * (triangle/_reference/trimul.py:44-54), which the reference differentiates with torch;
 * no native counterpart. */
int gnn_trimul_contract_bwd(const gnn_trimul_contract_bwd_args* args, void* stream);

/* Relayouts between the pixel-major rows of the op ([B, N, N] pixels, channels contiguous) and
 * per-channel planes, for 16-bit dtypes (B * Ch planes, channel c of batch b = plane b Ch + c):
 *   GNN_RELAYOUT_PLANES_TO_PIXELS:  src = planes [B * Ch][N][src_ld] (row r, column s);
 *       dst[pixel][dst_c0 + c] with pixel (r, s), or (s, r) when `transposed`; dst rows of
 *       dst_ld elements. src_ld >= round_up(N, 8).
 *   GNN_RELAYOUT_PIXELS_TO_BLOCKED: src[pixel (i, j)][src_c0 + c] (rows of src_ld elements) ->
 *       dst = [B * Ch][NP / 32][NP][32], NP = round_up(N, 32): element (i, j) at
 *       ((i / 32) NP + j) 32 + i % 32, or at ((j / 32) NP + i) 32 + j % 32 when `transposed`;
 *       every element with i >= N or j >= N is written as zero (the dO operands of
 *       gnn_trimul_contract_bwd: do_i untransposed, do_j transposed).
 * Ch, the row pitches and channel offsets multiples of 8; pointers 16-byte aligned. */
enum gnn_relayout_mode { GNN_RELAYOUT_PLANES_TO_PIXELS = 0, GNN_RELAYOUT_PIXELS_TO_BLOCKED = 1 };

typedef struct gnn_trimul_relayout_args {
  const void* src;
  void* dst;
  int64_t B, N, Ch;
  int64_t src_ld, dst_ld;
  int64_t src_c0, dst_c0;
  int32_t mode;       /* enum gnn_relayout_mode */
  int32_t transposed;
  int32_t dtype;      /* GNN_BF16 or GNN_F16 */
  int32_t reserved;
} gnn_trimul_relayout_args;

/* Replaces the strided copies (permute / contiguous) between the trimul backward's pixel-major
 * tensors and the contraction's planes; no counterpart in the reference, whose backward is
 * autograd through trimul_torch (triangle/_reference/trimul.py:57-97). */
int gnn_trimul_relayout(const gnn_trimul_relayout_args* args, void* stream);

/* Message for the last failing call on this thread ("" if none). */
const char* gnn_last_error(void);

/* Library version string, e.g. "0.1.0 gfx950". */
const char* gnn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GNN_TRIANGLE_H */
