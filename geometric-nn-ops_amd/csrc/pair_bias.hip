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
//
// Also here: the gate and output projection of attention with pair bias (apb_gate_out_kernel,
// below), the part of the op after the attention itself.
#include <type_traits>

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

// ---- gate and output projection ------------------------------------------------------
//   out = ( T(o) * T(sigmoid(T(s Wg^T + bg))) ) Wo^T + bo,
// each product's result rounded to T as the reference's F.linear / torch.sigmoid / multiply
// return it (attention_pair_bias.py:86-89). One workgroup (4 waves) per GT = 32 tokens:
// the tile's s rows and its o rows (the attention output, heads merged) are staged in LDS;
// gate pre-activations run on MFMA in passes of 128 channels (wave w: channels 32 w ..,
// A = Wg rows from global memory, fetched a chunk of k-steps ahead, B = s fragments from
// LDS), and each lane writes o * g over
// the o values it read, so the gated tile never leaves LDS; the output product then reads it
// as its B operand and its results leave through an LDS staging tile as 16-byte rows. No
// intermediate (g, o * g) reaches memory.
constexpr int GT = 32;       // tokens per workgroup
constexpr int GOC = 128;     // output channels per pass (4 waves x 32)
constexpr int GO_THREADS = 256;

struct GateOutLds {
  size_t s, og, y, bias, total;
};
template <typename T>
__host__ __device__ inline GateOutLds gate_out_lds(int64_t Cs, int64_t D) {
  constexpr int pad = 16 / (int)sizeof(T);
  GateOutLds L;
  L.s = 0;
  L.og = L.s + (size_t)GT * (Cs + pad) * sizeof(T);
  L.y = L.og + (size_t)GT * (D + pad) * sizeof(T);
  L.bias = L.y + (size_t)GT * (GOC + pad) * sizeof(T);
  return L;
}
// the biases follow as fp32 [D] and [Co]
__host__ __device__ inline size_t gate_out_lds_total(const GateOutLds& L, int64_t D, int64_t Co) {
  return L.bias + (size_t)(D + Co) * sizeof(float);
}

// acc += W[rows wrow.., k] * tile[token l32][k] over nk k-steps of 16 (nk a multiple of GK):
// the weight fragments (global memory, L2-resident) in chunks of GK k-steps, the next chunk
// requested before the current one's MFMAs so that the loads stay ahead of the products.
// Branches only around whole chunks, so a chunk's LDS reads and counter waits are straight
// code the compiler can schedule.
template <typename T, int PREC, int GK>
__device__ __forceinline__ void gate_out_gemm(f32x16& acc, const T* __restrict__ wrow, int nk, const T* tile, int ld,
                                              int l32, int g) {
  typedef typename TypeOps<T>::V8 V8;
  V8 wa[GK], wb[GK];
  auto load = [&](V8 (&w)[GK], int k0) {
#pragma unroll
    for (int j = 0; j < GK; ++j) w[j] = load8(wrow + 16 * (k0 + j));
  };
  auto mma = [&](const V8 (&w)[GK], int k0) {
#pragma unroll
    for (int j = 0; j < GK; ++j) Mma<T, PREC>::step(acc, w[j], load8(&tile[l32 * ld + 16 * (k0 + j) + 8 * g]));
  };
  load(wa, 0);
  for (int k0 = 0; k0 < nk; k0 += 2 * GK) {
    const bool second = k0 + GK < nk;  // uniform
    if (second) load(wb, k0 + GK);
    mma(wa, k0);
    if (second) {
      if (k0 + 2 * GK < nk) load(wa, k0 + 2 * GK);
      mma(wb, k0 + GK);
    }
  }
}
template <typename T, int PREC>
__device__ __forceinline__ void gate_out_gemm(f32x16& acc, const T* __restrict__ wrow, int nk, const T* tile, int ld,
                                              int l32, int g) {
  if (nk % 8 == 0) gate_out_gemm<T, PREC, 8>(acc, wrow, nk, tile, ld, l32, g);
  else gate_out_gemm<T, PREC, 2>(acc, wrow, nk, tile, ld, l32, g);  // widths are multiples of 32: nk is even
}

template <typename T, int PREC>
__global__ __launch_bounds__(GO_THREADS) void apb_gate_out_kernel(const gnn_apb_gate_out_args a) {
  typedef typename TypeOps<T>::V8 V8;
  typedef typename TypeOps<T>::V4 V4;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int pad = 16 / (int)sizeof(T);
  constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  const int Cs = (int)a.Cs, D = (int)a.D, Co = (int)a.Co;
  const int SR = Cs + pad, OR = D + pad, YR = GOC + pad;
  const GateOutLds L = gate_out_lds<T>(Cs, D);
  T* ss = reinterpret_cast<T*>(smem_raw + L.s);
  T* og = reinterpret_cast<T*>(smem_raw + L.og);
  T* ys = reinterpret_cast<T*>(smem_raw + L.y);
  float* gb_s = reinterpret_cast<float*>(smem_raw + L.bias);
  float* ob_s = gb_s + D;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int64_t t0 = (int64_t)blockIdx.x * GT;
  const int ntok = a.M - t0 < GT ? (int)(a.M - t0) : GT;

  // stage s [GT][Cs] and o [GT][D] (16-byte chunks, zeros past the last token), SB chunks
  // per thread loaded before any is stored, so their latencies overlap
  constexpr int SB = 8;
  typedef typename std::conditional<sizeof(T) == 2, V8, V4>::type Vc;  // 16 bytes of T
  auto stage = [&](const T* src, int64_t ld, int C, T* dst, int R) {
    const int cpr = C / EPC, n = GT * cpr;
    for (int base = 0; base < n; base += SB * GO_THREADS) {
      Vc v[SB];
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int c = base + i * GO_THREADS + tid, r = c / cpr, k = (c - r * cpr) * EPC;
        v[i] = Vc{};
        if (c < n && r < ntok) {
          if constexpr (sizeof(T) == 2) v[i] = load8(src + (t0 + r) * ld + k);
          else v[i] = load4(src + (t0 + r) * ld + k);
        }
      }
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int c = base + i * GO_THREADS + tid, r = c / cpr, k = (c - r * cpr) * EPC;
        if (c < n) {
          if constexpr (sizeof(T) == 2) store8(&dst[r * R + k], v[i]);
          else store4(&dst[r * R + k], v[i]);
        }
      }
    }
  };
  stage((const T*)a.s, a.s_ld, Cs, ss, SR);
  stage((const T*)a.o, a.o_ld, D, og, OR);
  for (int c = tid; c < D; c += GO_THREADS) gb_s[c] = a.g_b ? TypeOps<T>::to_f32(((const T*)a.g_b)[c]) : 0.f;
  for (int c = tid; c < Co; c += GO_THREADS) ob_s[c] = a.o_b ? TypeOps<T>::to_f32(((const T*)a.o_b)[c]) : 0.f;
  __syncthreads();

  // ---- gate: acc = [channel][token], channel = c0 + 32 wave + 8(r/4) + 4g + r%4, token l32
  for (int c0 = 0; c0 < D; c0 += GOC) {
    const int cw = c0 + 32 * wave;
    if (cw < D) {
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
      gate_out_gemm<T, PREC>(acc, (const T*)a.g_w + (int64_t)(cw + l32) * Cs + 8 * g, Cs / 16, ss, SR, l32, g);
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int ch = cw + 8 * rg + 4 * g;
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&gb_s[ch]);
        f32x4 pre;
#pragma unroll
        for (int e = 0; e < 4; ++e) pre[e] = acc[4 * rg + e] + b4[e];
        // T(linear) -> T(sigmoid) -> T(o * g)
        const f32x4 pr = TypeOps<T>::to_f32(TypeOps<T>::from_f32(pre));
        f32x4 gv;
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e] = 1.0f / (1.0f + __expf(-pr[e]));
        const f32x4 gr = TypeOps<T>::to_f32(TypeOps<T>::from_f32(gv));
        T* op = &og[l32 * OR + ch];
        const f32x4 ov = TypeOps<T>::to_f32(load4(op));
        store4(op, TypeOps<T>::from_f32(ov * gr));
      }
    }
  }
  __syncthreads();

  // ---- output: acc = [out channel][token], passes of GOC channels staged through ys
  T* obase = (T*)a.out + t0 * a.out_ld;
  for (int c0 = 0; c0 < Co; c0 += GOC) {
    const int W = Co - c0 < GOC ? Co - c0 : GOC;
    const int cw = c0 + 32 * wave;
    if (32 * wave < W) {
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
      gate_out_gemm<T, PREC>(acc, (const T*)a.o_w + (int64_t)(cw + l32) * D + 8 * g, D / 16, og, OR, l32, g);
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int ch = cw + 8 * rg + 4 * g;
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&ob_s[ch]);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[4 * rg + e] + b4[e];
        store4(&ys[l32 * YR + 32 * wave + 8 * rg + 4 * g], TypeOps<T>::from_f32(v));
      }
    }
    __syncthreads();
    const int cpr = W / EPC;
    for (int c = tid; c < GT * cpr; c += GO_THREADS) {
      const int r = c / cpr, k = (c - r * cpr) * EPC;
      if (r < ntok) {
        if constexpr (sizeof(T) == 2)
          store8(obase + (int64_t)r * a.out_ld + c0 + k, load8(&ys[r * YR + k]));
        else
          store4(obase + (int64_t)r * a.out_ld + c0 + k, load4(&ys[r * YR + k]));
      }
    }
    if (c0 + GOC < Co) __syncthreads();  // the next pass rewrites ys
  }
}

template <typename T, int PREC>
int launch_gate_out(const gnn_apb_gate_out_args& a, hipStream_t stream) {
  const size_t smem = gate_out_lds_total(gate_out_lds<T>(a.Cs, a.D), a.D, a.Co);
  const void* fn = (const void*)apb_gate_out_kernel<T, PREC>;
  if (smem > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  hipLaunchKernelGGL((apb_gate_out_kernel<T, PREC>), dim3((uint32_t)((a.M + GT - 1) / GT)), dim3(GO_THREADS), smem,
                     stream, a);
  return (int)hipGetLastError();
}

}  // namespace

int apb_gate_out(const gnn_apb_gate_out_args& a, hipStream_t stream) {
  if (a.Cs % 32 != 0 || a.D % 32 != 0 || a.Co % 32 != 0)
    return set_error(GNN_ERR_UNSUPPORTED, "apb_gate_out: c_s, the attention width and c_out must be multiples of 32");
  const size_t e = a.dtype == GNN_F32 ? 4 : 2;
  const size_t lds = gate_out_lds_total(e == 2 ? gate_out_lds<bf16>(a.Cs, a.D) : gate_out_lds<float>(a.Cs, a.D), a.D,
                                        a.Co);
  if (lds > 160 * 1024)
    return set_error(GNN_ERR_UNSUPPORTED, "apb_gate_out: c_s + attention width too large for the LDS tiles");
  if (a.M >= ((int64_t)1 << 31) * GT) return set_error(GNN_ERR_UNSUPPORTED, "apb_gate_out: too many tokens");
  switch (a.dtype) {
    case GNN_BF16: return launch_gate_out<bf16, PREC_NATIVE>(a, stream);
    case GNN_F16: return launch_gate_out<f16, PREC_NATIVE>(a, stream);
    case GNN_F32:
      return a.precision == GNN_PREC_BF16X3 ? launch_gate_out<float, PREC_BF16X3>(a, stream)
                                            : launch_gate_out<float, PREC_IEEE>(a, stream);
  }
  return set_error(GNN_ERR_ARG, "apb_gate_out: unknown dtype");
}

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
