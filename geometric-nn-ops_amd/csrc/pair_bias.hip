// Pair-bias projection of attention with pair bias, for gfx950.
//
//   bias[b, h, u, v] = round( sum_c round(LN(z[b, u, v, :]))[c] * W[h, c] )
//   LN(x)[c] = (x[c] - mean) / sqrt(var + eps) * gamma[c]      (biased variance, no beta)
//
// which is _project_pair_bias of the reference (geometric_nn_ops_torch/triangle/_reference/
// attention_pair_bias.py:17-22: F.layer_norm without bias, rounded to z's dtype as
// F.layer_norm returns it, then F.linear with fp32 accumulation and the permute to
// [B, H, U, V]). One pass over the pair tensor z replaces the reference's LayerNorm
// output, linear output and permuted copy.
//
// Layout: eight lanes per pixel (a wave holds 8 consecutive pixels of the flattened
// [B, U, V] grid), lane j of a pixel loading the 16-byte channel chunks j, j + 8, ... of its
// row, so a wave's loads cover 8 whole contiguous pixel rows. Mean and variance are reduced
// over the 8 lanes with xor shuffles (two passes over the registers). The projection
// weights sit in LDS as fp32 [H][Zc]; each lane forms its channels' partial dot product for
// a head, the 8 partials meet through three xor shuffles, and lane h % 8 stores head h.
// The kernel is HBM-bound (Zc * e bytes read per pixel against H * e written).
#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

constexpr int PB_THREADS = 256;              // 4 waves
constexpr int PB_PIX = PB_THREADS / 8;       // pixels per workgroup iteration
constexpr int PB_MAX_CHUNKS = 4;             // Zc <= 256
constexpr int PB_MAX_W = 8192;               // H * Zc <= 8192 (32 KB of fp32 weights)

template <typename T>
__global__ __launch_bounds__(PB_THREADS) void pair_bias_proj_kernel(const gnn_pair_bias_args a) {
  __shared__ float ws[PB_MAX_W];
  __shared__ float gs[PB_MAX_CHUNKS * 64];
  const int Zc = (int)a.Zc, H = (int)a.H, V = (int)a.V, U = (int)a.U;
  const int tid = threadIdx.x;
  for (int i = tid; i < H * Zc; i += PB_THREADS) ws[i] = TypeOps<T>::to_f32(((const T*)a.proj_w)[i]);
  for (int i = tid; i < Zc; i += PB_THREADS)
    gs[i] = a.ln_w ? TypeOps<T>::to_f32(((const T*)a.ln_w)[i]) : 1.0f;
  __syncthreads();

  const int j = tid & 7;
  const int nch = Zc / 8;
  const int64_t npix = a.B * (int64_t)U * V;
  const float inv_zc = 1.0f / (float)Zc;
  for (int64_t p0 = (int64_t)blockIdx.x * PB_PIX; p0 < npix; p0 += (int64_t)gridDim.x * PB_PIX) {
    const int64_t p = p0 + (tid >> 3);
    const bool ok = p < npix;
    const T* row = (const T*)a.z + (ok ? p : 0) * Zc;
    f32x8 x[PB_MAX_CHUNKS];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < PB_MAX_CHUNKS; ++c) {
      const int ch = j + 8 * c;
      if (ch < nch) {
        x[c] = TypeOps<T>::to_f32(load8(row + 8 * ch));
#pragma unroll
        for (int e = 0; e < 8; ++e) s += x[c][e];
      }
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    const float mean = s * inv_zc;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < PB_MAX_CHUNKS; ++c) {
      if (j + 8 * c < nch) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = x[c][e] - mean;
          q += d * d;
        }
      }
    }
    q += __shfl_xor(q, 1);
    q += __shfl_xor(q, 2);
    q += __shfl_xor(q, 4);
    const float rstd = 1.0f / sqrtf(q * inv_zc + a.eps);
    // normalised, gamma-scaled and rounded to the input dtype (F.layer_norm's output)
#pragma unroll
    for (int c = 0; c < PB_MAX_CHUNKS; ++c) {
      const int ch = j + 8 * c;
      if (ch < nch) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          x[c][e] = TypeOps<T>::to_f32(TypeOps<T>::from_f32((x[c][e] - mean) * rstd * gs[8 * ch + e]));
      }
    }
    int64_t b = 0, u = 0, v = 0;
    if (ok) {
      v = p % V;
      const int64_t r = p / V;
      u = r % U;
      b = r / U;
    }
    T* orow = (T*)a.out + b * a.out_stride[0] + u * a.out_stride[2] + v;
    for (int h = 0; h < H; ++h) {
      const float* wh = ws + h * Zc;
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < PB_MAX_CHUNKS; ++c) {
        const int ch = j + 8 * c;
        if (ch < nch) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(x[c][e], wh[8 * ch + e], acc);
        }
      }
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      acc += __shfl_xor(acc, 4);
      if (ok && (h & 7) == j) orow[h * a.out_stride[1]] = TypeOps<T>::from_f32(acc);
    }
  }
}

template <typename T>
int launch_pb(const gnn_pair_bias_args& a, hipStream_t stream) {
  const int64_t npix = a.B * a.U * a.V;
  const int64_t want = (npix + PB_PIX - 1) / PB_PIX;
  const int grid = (int)std::min<int64_t>(want, (int64_t)persistent_grid((const void*)pair_bias_proj_kernel<T>,
                                                                          PB_THREADS, 0) * 4);
  hipLaunchKernelGGL(pair_bias_proj_kernel<T>, dim3(grid < 1 ? 1 : grid), dim3(PB_THREADS), 0, stream, a);
  return (int)hipGetLastError();
}

}  // namespace

int pair_bias_proj(const gnn_pair_bias_args& a, hipStream_t stream) {
  if (a.Zc % 8 != 0 || a.Zc > 8 * PB_MAX_CHUNKS * 8)
    return set_error(GNN_ERR_UNSUPPORTED, "pair_bias_proj: c_z must be a multiple of 8 and at most 256");
  if (a.H * a.Zc > PB_MAX_W)
    return set_error(GNN_ERR_UNSUPPORTED, "pair_bias_proj: heads * c_z must be at most 8192");
  switch (a.dtype) {
    case GNN_BF16: return launch_pb<bf16>(a, stream);
    case GNN_F16: return launch_pb<f16>(a, stream);
    case GNN_F32: return launch_pb<float>(a, stream);
  }
  return set_error(GNN_ERR_ARG, "pair_bias_proj: unknown dtype");
}

}  // namespace gnn
