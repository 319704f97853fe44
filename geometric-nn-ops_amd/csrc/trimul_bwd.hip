// Element-wise and LayerNorm kernels of the triangle multiplicative update's backward, for
// gfx950.
//
// The reference has no native trimul backward: a forward that needs gradients runs its
// pure-torch trimul_torch under autograd (geometric_nn_ops_torch/triangle/_trimul.py:31-36,
// math in triangle/_reference/trimul.py:57-97). This library differentiates that same math.
// The plain matrix products of the backward (weight gradients, input gradients of the
// linear layers, the contraction's two products per channel) go to the vendor GEMM; the
// rest is here:
//
//   layernorm_rows   y = (x - mean) * rstd * w + b per row, or its backward
//                      xh = (x - mean) * rstd,  g = dy * w,
//                      dx = rstd * (g - mean(g) - xh * mean(g * xh)),
//                    plus per-workgroup column sums of dy * xh (-> dw) and dy (-> db), so
//                    the weight gradients need no atomics and sum in a fixed order.
//   gate_bwd         the backward of  out = value * sigmoid(gate_pre) [* mask per row]:
//                      d_value = grad * s * m,   d_gate_pre = grad * value * m * s * (1 - s).
//                    Used for the output gate (value = p_out(LN(o)), no mask) and for the
//                    gated input projection (value = p_in(z), mask = the pair mask).
//
// Layout: one 32-lane half-wave per row (K a multiple of 32, at most 512: each lane holds
// K / 32 consecutive columns, reduced with xor shuffles inside the half-wave); 16 rows per
// 256-thread workgroup in flight (two per half-wave, loads issued together), a grid of at most
// 4096 workgroups striding over the rows. Every tensor is
// read once and written once, so both kernels are bound by HBM bandwidth.
#include <algorithm>

#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

constexpr int LN_THREADS = 256;                 // 8 half-waves: 8 rows at a time
constexpr int LN_ROWS = LN_THREADS / 32;
constexpr int LN_MAX_K = 512;
constexpr int LN_UNROLL = 4;                    // rows per half-wave step
constexpr int LN_MAX_GRID = 4096;               // partial rows of the weight gradients

template <typename T>
__device__ __forceinline__ float ld1(const void* p, int64_t i, float dflt) {
  return p ? TypeOps<T>::to_f32(((const T*)p)[i]) : dflt;
}

// Sum over a half-wave (lanes 32h .. 32h + 31; every lane gets it) in VALU lane moves, no
// LDS-routed shuffle: DPP pairs (quad_perm 1,0,3,2), quads (2,3,0,1), half-rows
// (row_half_mirror) and rows (row_mirror) -- each mirror pairs a lane with one holding the
// complementary partial sum -- then v_permlane16_swap joins the half-wave's two rows.
__device__ __forceinline__ float half_wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// KPL columns per lane (K = 32 * KPL), lane c of a half-wave owning columns KPL c .. KPL c + KPL-1.
// A half-wave takes LN_UNROLL rows per step, their loads issued together.
template <typename T, int KPL, bool BWD>
__global__ __launch_bounds__(LN_THREADS) void layernorm_rows_kernel(const gnn_layernorm_args a) {
  const int K = 32 * KPL;
  const int tid = threadIdx.x, hw = tid >> 5, c = tid & 31;
  const int k0 = c * KPL;
  float w[KPL], bv[KPL], bsum[KPL], wsum[KPL];
#pragma unroll
  for (int e = 0; e < KPL; ++e) {
    w[e] = ld1<T>(a.weight, k0 + e, 1.f);
    bv[e] = BWD ? 0.f : ld1<T>(a.bias, k0 + e, 0.f);
    bsum[e] = 0.f;  // backward: column sums of dy
    wsum[e] = 0.f;  // backward: column sums of dy * xh
  }
  const float inv_k = 1.0f / (float)K;
  // K = 128 (four columns per lane) with rows aligned to four elements: one vector access
  // per lane and row instead of four scalar ones
  typedef typename TypeOps<T>::V4 TV4;
  constexpr bool V4 = KPL == 4;
  constexpr int64_t VB = sizeof(TV4);
  auto al = [&](const void* p, int64_t stride) {
    return (uintptr_t)p % VB == 0 && (stride * (int64_t)sizeof(T)) % VB == 0;
  };
  const bool vec = V4 && al(a.x, a.x_stride) && al(a.out, a.out_stride) && (!BWD || al(a.dy, a.dy_stride));
  const int64_t step = (int64_t)gridDim.x * LN_ROWS * LN_UNROLL;
  for (int64_t r0 = ((int64_t)blockIdx.x * LN_ROWS + hw) * LN_UNROLL; r0 < a.rows; r0 += step) {
    float x[LN_UNROLL][KPL], dy[LN_UNROLL][KPL];
#pragma unroll
    for (int u = 0; u < LN_UNROLL; ++u) {
      const int64_t r = min(r0 + u, a.rows - 1);  // a row past the end repeats the last (not stored)
      const T* xr = (const T*)a.x + r * a.x_stride + k0;
      if (V4 && vec) {
        const f32x4 xv = TypeOps<T>::to_f32(*reinterpret_cast<const TV4*>(xr));
#pragma unroll
        for (int e = 0; e < KPL; ++e) x[u][e] = xv[e % 4];
      } else {
#pragma unroll
        for (int e = 0; e < KPL; ++e) x[u][e] = TypeOps<T>::to_f32(xr[e]);
      }
      if constexpr (BWD) {
        const T* dyr = (const T*)a.dy + r * a.dy_stride + k0;
        if (V4 && vec) {
          const f32x4 dv = TypeOps<T>::to_f32(*reinterpret_cast<const TV4*>(dyr));
#pragma unroll
          for (int e = 0; e < KPL; ++e) dy[u][e] = dv[e % 4];
        } else {
#pragma unroll
          for (int e = 0; e < KPL; ++e) dy[u][e] = TypeOps<T>::to_f32(dyr[e]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < LN_UNROLL; ++u) {
      const int64_t r = r0 + u;
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < KPL; ++e) s += x[u][e];
      const float mean = half_wave_sum(s) * inv_k;
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < KPL; ++e) {
        x[u][e] -= mean;
        q += x[u][e] * x[u][e];
      }
      const float rstd = 1.0f / sqrtf(half_wave_sum(q) * inv_k + a.eps);
      if (r >= a.rows) continue;  // uniform over the half-wave (after its shuffles)
      T* orow = (T*)a.out + r * a.out_stride + k0;
      if constexpr (!BWD) {
        float y[KPL];
#pragma unroll
        for (int e = 0; e < KPL; ++e) y[e] = x[u][e] * rstd * w[e] + bv[e];
        if (V4 && vec) {
          *reinterpret_cast<TV4*>(orow) = TypeOps<T>::from_f32(f32x4{y[0], y[1 % KPL], y[2 % KPL], y[3 % KPL]});
        } else {
#pragma unroll
          for (int e = 0; e < KPL; ++e) orow[e] = TypeOps<T>::from_f32(y[e]);
        }
      } else {
        float g[KPL];
        float sg = 0.f, sgx = 0.f;
#pragma unroll
        for (int e = 0; e < KPL; ++e) {
          const float xh = x[u][e] * rstd;
          bsum[e] += dy[u][e];
          wsum[e] += dy[u][e] * xh;
          g[e] = dy[u][e] * w[e];
          sg += g[e];
          sgx += g[e] * xh;
          x[u][e] = xh;
        }
        const float mg = half_wave_sum(sg) * inv_k, mgx = half_wave_sum(sgx) * inv_k;
#pragma unroll
        for (int e = 0; e < KPL; ++e) g[e] = rstd * (g[e] - mg - x[u][e] * mgx);
        if (V4 && vec) {
          *reinterpret_cast<TV4*>(orow) = TypeOps<T>::from_f32(f32x4{g[0], g[1 % KPL], g[2 % KPL], g[3 % KPL]});
        } else {
#pragma unroll
          for (int e = 0; e < KPL; ++e) orow[e] = TypeOps<T>::from_f32(g[e]);
        }
      }
    }
  }
  if constexpr (BWD) {
    if (!a.partial) return;  // uniform over the workgroup
    // the 8 half-waves' column sums meet in LDS, summed in half-wave order
    __shared__ float red[LN_ROWS][2][LN_MAX_K];
#pragma unroll
    for (int e = 0; e < KPL; ++e) {
      red[hw][0][k0 + e] = wsum[e];
      red[hw][1][k0 + e] = bsum[e];
    }
    __syncthreads();
    float* part = a.partial + (int64_t)blockIdx.x * 2 * K;
    for (int i = tid; i < 2 * K; i += LN_THREADS) {
      const int which = i / K, col = i % K;
      float acc = 0.f;
#pragma unroll
      for (int h = 0; h < LN_ROWS; ++h) acc += red[h][which][col];
      part[i] = acc;
    }
  }
}

// ---- forward LayerNorm of wide rows (512 < K <= LN_WIDE_MAX_K, K a multiple of 32): one
// wave per row, walking it in 512-column chunks (8 consecutive columns per lane, 16-byte
// loads) three times -- the sum, the squared deviations from the mean, the normalised output
// -- so that nothing of the row is held in registers; the row (at most 16 KB) is re-read
// from the caches. The same two-pass statistics as the narrow kernel.
constexpr int LN_WIDE_MAX_K = 8192;
constexpr int LN_WIDE_WAVES = 4;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <typename T>
__global__ __launch_bounds__(64 * LN_WIDE_WAVES) void layernorm_wide_kernel(const gnn_layernorm_args a) {
  const int K = (int)a.K, lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * LN_WIDE_WAVES + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * LN_WIDE_WAVES;
  const float inv_k = 1.0f / (float)K;
  for (int64_t r = wave; r < a.rows; r += nwaves) {
    const T* xr = (const T*)a.x + r * a.x_stride;
    float s = 0.f;
    for (int k = 8 * lane; k < K; k += 512) {
      const f32x8 v = TypeOps<T>::to_f32(load8(xr + k));
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[e];
    }
    const float mean = wave_sum(s) * inv_k;
    float q = 0.f;
    for (int k = 8 * lane; k < K; k += 512) {
      const f32x8 v = TypeOps<T>::to_f32(load8(xr + k));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[e] - mean;
        q += d * d;
      }
    }
    const float rstd = 1.0f / sqrtf(wave_sum(q) * inv_k + a.eps);
    T* orow = (T*)a.out + r * a.out_stride;
    for (int k = 8 * lane; k < K; k += 512) {
      const f32x8 v = TypeOps<T>::to_f32(load8(xr + k));
      f32x8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (v[e] - mean) * rstd * ld1<T>(a.weight, k + e, 1.f) + ld1<T>(a.bias, k + e, 0.f);
      store8(orow + k, TypeOps<T>::from_f32(y));
    }
  }
}

template <typename T>
int launch_ln_wide(const gnn_layernorm_args& a, hipStream_t st) {
  const int64_t grid = std::min<int64_t>((a.rows + LN_WIDE_WAVES - 1) / LN_WIDE_WAVES, 8192);
  hipLaunchKernelGGL((layernorm_wide_kernel<T>), dim3((uint32_t)grid), dim3(64 * LN_WIDE_WAVES), 0, st, a);
  return (int)hipGetLastError();
}

template <typename T, bool BWD>
int launch_ln(const gnn_layernorm_args& a, hipStream_t st) {
  const int grid = (int)layernorm_partials(a.rows, a.K);
  switch (a.K / 32) {
#define GNN_LN_CASE(KPL)                                                                              \
  case KPL:                                                                                           \
    hipLaunchKernelGGL((layernorm_rows_kernel<T, KPL, BWD>), dim3(grid), dim3(LN_THREADS), 0, st, a); \
    break;
    GNN_LN_CASE(1)
    GNN_LN_CASE(2)
    GNN_LN_CASE(3)
    GNN_LN_CASE(4)
    GNN_LN_CASE(5)
    GNN_LN_CASE(6)
    GNN_LN_CASE(7)
    GNN_LN_CASE(8)
    GNN_LN_CASE(9)
    GNN_LN_CASE(10)
    GNN_LN_CASE(11)
    GNN_LN_CASE(12)
    GNN_LN_CASE(13)
    GNN_LN_CASE(14)
    GNN_LN_CASE(15)
    GNN_LN_CASE(16)
#undef GNN_LN_CASE
    default:
      return set_error(GNN_ERR_UNSUPPORTED, "layernorm_rows: K must be a multiple of 32, at most 512");
  }
  return (int)hipGetLastError();
}

// ---- gate backward: 8 consecutive elements per thread ----------------------------------
// With partial sums (PART), K / 8 divides the block, so a thread keeps the same 8 columns over
// its whole grid-stride walk: it sums the values it stores in registers, and the workgroup
// adds up the threads of each column through LDS once at the end (a fixed order, no atomics).
constexpr int GB_THREADS = 256;
constexpr int GB_MAX_GRID = 1024;  // partial rows of the bias gradients

template <typename T, bool PART>
__global__ __launch_bounds__(GB_THREADS) void gate_bwd_kernel(const gnn_gate_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  const int64_t kc = a.K / 8;  // 8-element chunks per row
  const int64_t total = a.rows * kc;
  f32x8 sdv = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, sdg = sdv;
  for (int64_t i = (int64_t)blockIdx.x * GB_THREADS + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * GB_THREADS) {
    const int64_t r = i / kc, k = (i % kc) * 8;
    const f32x8 gr = TypeOps<T>::to_f32(load8((const T*)a.grad + r * a.grad_stride + k));
    const f32x8 v = TypeOps<T>::to_f32(load8((const T*)a.value + r * a.value_stride + k));
    const f32x8 gp = TypeOps<T>::to_f32(load8((const T*)a.gate_pre + r * a.gate_stride + k));
    const float m = a.mask ? TypeOps<T>::to_f32(((const T*)a.mask)[r * a.mask_stride]) : 1.f;
    f32x8 dv, dg;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // sigmoid with the hardware exp2 and reciprocal, as the forward's gates (or the saved
      // gate itself)
      const float s = a.gate_is_sigmoid ? gp[e]
                                        : __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gp[e] * -1.4426950408889634f));
      const float gm = gr[e] * m;
      dv[e] = gm * s;
      dg[e] = gm * v[e] * s * (1.0f - s);
    }
    const V8 dvr = TypeOps<T>::from_f32(dv), dgr = TypeOps<T>::from_f32(dg);
    store8((T*)a.d_value + r * a.dv_stride + k, dvr);
    store8((T*)a.d_gate_pre + r * a.dg_stride + k, dgr);
    if constexpr (PART) {
      sdv += TypeOps<T>::to_f32(dvr);
      sdg += TypeOps<T>::to_f32(dgr);
    }
  }
  if constexpr (PART) {
    __shared__ float red[GB_THREADS][17];  // padded rows: the column walk below spreads over banks
    const int tid = threadIdx.x;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      red[tid][e] = sdv[e];
      red[tid][8 + e] = sdg[e];
    }
    __syncthreads();
    const int K = (int)a.K, nkc = (int)kc;
    for (int c = tid; c < 2 * K; c += GB_THREADS) {
      const int which = c / K, col = c % K;
      float sum = 0.f;
      for (int t = col / 8; t < GB_THREADS; t += nkc) sum += red[t][8 * which + col % 8];
      a.partial[((int64_t)blockIdx.x * 2 + which) * K + col] = sum;
    }
  }
}

template <typename T>
int launch_gate(const gnn_gate_bwd_args& a, hipStream_t st) {
  if (a.partial) {
    const int64_t grid = gate_bwd_partials(a.rows, a.K);
    if (grid < 1) return set_error(GNN_ERR_UNSUPPORTED, "gate_bwd: partial sums need K / 8 to divide 256");
    hipLaunchKernelGGL((gate_bwd_kernel<T, true>), dim3((uint32_t)grid), dim3(GB_THREADS), 0, st, a);
    return (int)hipGetLastError();
  }
  const int64_t chunks = a.rows * (a.K / 8);
  const int64_t want = (chunks + GB_THREADS - 1) / GB_THREADS;
  const int grid = (int)std::min<int64_t>(
      want, (int64_t)persistent_grid((const void*)gate_bwd_kernel<T, false>, GB_THREADS, 0) * 4);
  hipLaunchKernelGGL((gate_bwd_kernel<T, false>), dim3(grid < 1 ? 1 : grid), dim3(GB_THREADS), 0, st, a);
  return (int)hipGetLastError();
}

// ---- the input side of the backward in one pass (16-bit, C = CK in {64, 128}) -----------
// Per 64-pixel tile: LN_in of the tile's x rows (fp32 statistics, two barriers, the partials
// merged as in the forward's projection kernel), z rounded to T, written to z and kept in LDS;
// wave w owns the 32 stacked channels 32 w .. 32 w + 31 of p_in and g_in (2 Ch <= 256, their
// weight fragments in registers for the whole launch) and recomputes p and g for the tile's two
// 32-pixel halves on MFMA as [channel][pixel] blocks (A = the weights, B = z), so that a lane
// holds one pixel and 4 consecutive channels per register group: d_ab is read and d_p / d_g
// written 8 bytes at a time straight from the accumulators, each pixel row's 64 bytes per wave
// covered by its two lanes. The next tile's x is requested before the current tile's MFMAs.
// The per-channel sums of the stored d_p / d_g stay in registers until the workgroup ends.
constexpr int PB_W = 8;              // waves
constexpr int PB_NT = 64 * PB_W;     // threads
constexpr int PB_TP = 64;            // pixels per tile
constexpr int PB_MAX_GRID = 512;     // partial rows of the bias gradients

template <typename T, int CK>
struct PbLds {
  static constexpr int ZR = CK + (int)(16 / sizeof(T));  // z row pitch (elements)
  static constexpr size_t zs = 0;
  static constexpr size_t red = zs + (size_t)PB_TP * ZR * sizeof(T);
  static constexpr size_t lnw = red + 8 * (size_t)PB_TP * 8;
  static constexpr size_t lnb = lnw + CK * 4;
  static constexpr size_t bias = lnb + CK * 4;  // [2][256]: p_in, g_in biases
  static constexpr size_t mk = bias + 2 * 256 * 4;
  static constexpr size_t total = mk + PB_TP * 4;
};

// ALLU: 2 c_hidden = 256, so every wave owns a unit; its tile loop then holds no load or
// store in a branch (loads of the workgroup's last tile repeat that tile; stores are buffer
// stores whose range ends at the last row), and the compiler's memory-counter wait for the
// next tile's x and d_ab leaves the stores just issued in flight.
template <typename T, int CK, bool ALLU>
__global__ __launch_bounds__(PB_NT, 1) void trimul_proj_bwd_kernel(const gnn_trimul_proj_bwd_args a) {
  typedef PbLds<T, CK> S;
  typedef typename TypeOps<T>::V8 V8;
  typedef typename TypeOps<T>::V4 V4;
  constexpr int XM = CK / 64, NK = CK / 16, ZR = S::ZR;
  __shared__ __align__(16) unsigned char smem[S::total];
  T* zs = reinterpret_cast<T*>(smem + S::zs);
  float2* red = reinterpret_cast<float2*>(smem + S::red);
  float* lnw = reinterpret_cast<float*>(smem + S::lnw);
  float* lnb = reinterpret_cast<float*>(smem + S::lnb);
  float* bias = reinterpret_cast<float*>(smem + S::bias);
  float* mk = reinterpret_cast<float*>(smem + S::mk);
  const int64_t rows = a.rows;
  const int Ch2 = 2 * (int)a.Ch;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int64_t ntiles = (rows + PB_TP - 1) / PB_TP;

  for (int c = tid; c < CK; c += PB_NT) {
    lnw[c] = a.ln_w ? TypeOps<T>::to_f32(((const T*)a.ln_w)[c]) : 1.f;
    lnb[c] = a.ln_b ? TypeOps<T>::to_f32(((const T*)a.ln_b)[c]) : 0.f;
  }
  for (int c = tid; c < Ch2; c += PB_NT) {
    bias[c] = a.p_in_b ? TypeOps<T>::to_f32(((const T*)a.p_in_b)[c]) : 0.f;
    bias[256 + c] = a.g_in_b ? TypeOps<T>::to_f32(((const T*)a.g_in_b)[c]) : 0.f;
  }
  // this wave's channels: A fragments, row = channel 32 wave + l32, k = 16 kk + 8 g + e
  const bool has_unit = ALLU || 32 * wave < Ch2;  // uniform over the wave
  V8 wpf[NK], wgf[NK];
  {
    const int ch = has_unit ? 32 * wave + l32 : 0;
    const T* wprow = (const T*)a.p_in_w + (int64_t)ch * CK + 8 * g;
    const T* wgrow = (const T*)a.g_in_w + (int64_t)ch * CK + 8 * g;
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      wpf[k] = load8(wprow + 16 * k);
      wgf[k] = load8(wgrow + 16 * k);
    }
  }
  float sp[16], sg[16];  // sums of the stored d_p / d_g, channel 32 wave + 8 (i / 4) + 4 g + i % 4
#pragma unroll
  for (int i = 0; i < 16; ++i) sp[i] = sg[i] = 0.f;

  // ---- tile load + LayerNorm: thread = (pixel xpl, part xpart) holding chunks xpart + 8j;
  // rows past the end read the last row (in bounds; never stored)
  const int xpl = tid >> 3, xpart = tid & 7;
  V8 xr[XM];
  T mraw = TypeOps<T>::from_f32(1.f);
  auto load_x = [&](int64_t t) {
    const int64_t r = min(t * PB_TP + xpl, rows - 1);
    const T* src = (const T*)a.x + r * a.x_ld;
#pragma unroll
    for (int j = 0; j < XM; ++j) xr[j] = load8(src + 8 * (xpart + 8 * j));
    if (a.mask && tid < PB_TP) mraw = ((const T*)a.mask)[min(t * PB_TP + tid, rows - 1) * a.mask_stride];
  };
  auto ln_partial = [&]() {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < XM; ++j) {
      const f32x8 v = TypeOps<T>::to_f32(xr[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[e];
    }
    const float mean = s * (1.0f / (8 * XM));
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < XM; ++j) {
      const f32x8 v = TypeOps<T>::to_f32(xr[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[e] - mean;
        m2 += d * d;
      }
    }
    red[xpart * PB_TP + xpl] = make_float2(mean, m2);
  };
  auto ln_finish = [&](int64_t t) {
    float mean = 0.f;
    float2 pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pr[j] = red[j * PB_TP + xpl];
      mean += pr[j].x;
    }
    mean *= 0.125f;  // every part holds 8 * XM channels
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = pr[j].x - mean;
      m2 += pr[j].y + (float)(8 * XM) * d * d;
    }
    const float rstd = 1.0f / sqrtf(m2 * (1.0f / CK) + a.eps);
    const int64_t r = t * PB_TP + xpl;
#pragma unroll
    for (int j = 0; j < XM; ++j) {
      const int ci = xpart + 8 * j;
      const f32x8 v = TypeOps<T>::to_f32(xr[j]);
      f32x8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (v[e] - mean) * rstd * lnw[8 * ci + e] + lnb[8 * ci + e];
      const V8 yr = TypeOps<T>::from_f32(y);
      store8(&zs[xpl * ZR + 8 * ci], yr);
      if constexpr (ALLU) {  // the range ends at the last row
        const int64_t r0 = t * PB_TP;
        buffer_store(yr, buffer_rsrc((T*)a.z + r0 * CK, (int)(min<int64_t>(PB_TP, rows - r0) * CK * sizeof(T))),
                     (uint32_t)((xpl * CK + 8 * ci) * (int)sizeof(T)));
      } else {
        if (r < rows) store8((T*)a.z + r * CK + 8 * ci, yr);
      }
    }
    if (tid < PB_TP) mk[tid] = TypeOps<T>::to_f32(mraw);
  };

  // d_ab of a tile: this lane's pixel of each 32-pixel half, channels 32 wave + 8 rg + 4 g
  // .. + 3; requested a tile ahead, with the next tile's x
  V4 dac[PB_TP / 32][4], dan[PB_TP / 32][4];
  auto load_d = [&](int64_t t, V4 (&d)[PB_TP / 32][4]) {
    if (!has_unit) return;
#pragma unroll
    for (int s = 0; s < PB_TP / 32; ++s) {
      const int64_t rr = min(t * PB_TP + 32 * s + l32, rows - 1);
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) d[s][rg] = load4((const T*)a.d_ab + rr * a.dab_ld + 32 * wave + 8 * rg + 4 * g);
    }
  };

  auto compute = [&](int64_t t) {
    if (!has_unit) return;
#pragma unroll
    for (int s = 0; s < PB_TP / 32; ++s) {
      const int64_t row = t * PB_TP + 32 * s + l32;
      const bool rok = row < rows;
      const V4 (&da)[4] = dac[s];
      f32x16 accp, accg;
#pragma unroll
      for (int i = 0; i < 16; ++i) accp[i] = accg[i] = 0.f;
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const V8 zf = load8(&zs[(32 * s + l32) * ZR + 16 * k + 8 * g]);
        Mma<T, PREC_NATIVE>::step(accp, wpf[k], zf);
        Mma<T, PREC_NATIVE>::step(accg, wgf[k], zf);
      }
      const float m = mk[32 * s + l32];
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int c0 = 32 * wave + 8 * rg + 4 * g;
        const f32x4 bp = *reinterpret_cast<const f32x4*>(&bias[c0]);
        const f32x4 bg = *reinterpret_cast<const f32x4*>(&bias[256 + c0]);
        const f32x4 d = TypeOps<T>::to_f32(da[rg]);
        f32x4 dp, dg;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // p and g rounded to T, as the linear layers' outputs are
          const float p = TypeOps<T>::to_f32(TypeOps<T>::from_f32(accp[4 * rg + e] + bp[e]));
          const float gg = TypeOps<T>::to_f32(TypeOps<T>::from_f32(accg[4 * rg + e] + bg[e]));
          const float sgm = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gg * -1.4426950408889634f));
          const float gm = d[e] * m;
          dp[e] = gm * sgm;
          dg[e] = gm * p * sgm * (1.0f - sgm);
        }
        const V4 dpr = TypeOps<T>::from_f32(dp), dgr = TypeOps<T>::from_f32(dg);
        if constexpr (ALLU) {
          // ranges from the tile's first row to the end of its last valid one (the row pitch
          // is at least 2 c_hidden), so the lanes of rows past the end fall outside them
          const int64_t r0 = t * PB_TP;
          const int nv = (int)min<int64_t>(PB_TP, rows - r0);
          const int range = (int)(((int64_t)(nv - 1) * a.dl_ld + Ch2) * (int64_t)sizeof(T));
          const uint32_t off = (uint32_t)(((int64_t)(32 * s + l32) * a.dl_ld + c0) * (int64_t)sizeof(T));
          buffer_store(dpr, buffer_rsrc((T*)a.d_p + r0 * a.dl_ld, range), off);
          buffer_store(dgr, buffer_rsrc((T*)a.d_g + r0 * a.dl_ld, range), off);
        }
        if (rok) {
          if constexpr (!ALLU) {
            store4((T*)a.d_p + row * a.dl_ld + c0, dpr);
            store4((T*)a.d_g + row * a.dl_ld + c0, dgr);
          }
          const f32x4 dpf = TypeOps<T>::to_f32(dpr), dgf = TypeOps<T>::to_f32(dgr);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sp[4 * rg + e] += dpf[e];
            sg[4 * rg + e] += dgf[e];
          }
        }
      }
    }
  };

  int64_t t = blockIdx.x;
  if (t < ntiles) {
    load_x(t);
    load_d(t, dac);
    ln_partial();
    __syncthreads();  // partials, LayerNorm parameters and biases published
    ln_finish(t);
    __syncthreads();
    for (; t < ntiles; t += gridDim.x) {
      // ALLU: the last tile is requested (and normalised, and its z stored) again, so that
      // no load or store of the loop sits in a branch
      const int64_t tn = ALLU && t + gridDim.x >= ntiles ? t : t + gridDim.x;
      const bool has_next = ALLU || tn < ntiles;  // uniform over the workgroup
      if (has_next) {
        load_x(tn);
        load_d(tn, dan);
      }
      compute(t);
#pragma unroll
      for (int s = 0; s < PB_TP / 32; ++s)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) dac[s][rg] = dan[s][rg];
      if (has_next) ln_partial();
      __syncthreads();  // z / mask of this tile consumed, partials of the next one published
      if (has_next) ln_finish(tn);
      __syncthreads();
    }
  }
  // ---- the workgroup's column sums: over the 32 lanes of each lane group (their pixels)
  if (has_unit) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) {
        sp[i] += __shfl_xor(sp[i], o);
        sg[i] += __shfl_xor(sg[i], o);
      }
    }
    if (l32 == 0) {
      float* prow = a.partial + (int64_t)blockIdx.x * 2 * Ch2;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int c = 32 * wave + 8 * (i / 4) + 4 * g + (i % 4);
        prow[c] = sp[i];
        prow[Ch2 + c] = sg[i];
      }
    }
  }
}

template <typename T, int CK>
int launch_proj_bwd(const gnn_trimul_proj_bwd_args& a, hipStream_t st) {
  const int64_t grid = trimul_proj_bwd_partials(a.rows);
  // the buffer ranges of one tile: 64 rows of z and of the gradient's row pitch
  if (2 * a.Ch == 32 * PB_W && (int64_t)PB_TP * std::max<int64_t>(a.dl_ld, CK) * 2 < ((int64_t)1 << 31))
    hipLaunchKernelGGL((trimul_proj_bwd_kernel<T, CK, true>), dim3((uint32_t)grid), dim3(PB_NT), 0, st, a);
  else
    hipLaunchKernelGGL((trimul_proj_bwd_kernel<T, CK, false>), dim3((uint32_t)grid), dim3(PB_NT), 0, st, a);
  return (int)hipGetLastError();
}

// ---- the output side of the backward in one pass (16-bit, C = CK in {64, 128}, c_hidden =
// CHK in {32, 64, 128}) -------------------------------------------------------------------
// Per tile of 64 consecutive pixels of one pair-grid row (the forward output stage's tiles):
// the channel-major o tile is staged in LDS and normalised per pixel (LN_out, two-pass fp32
// statistics over a pair of pixels per thread, as the forward), on written once (for the
// p_out weight gradient); y = on p_out_w^T + p_out_b on MFMA as [output channel][pixel]
// blocks (wave: 32 output channels x 32 pixels), so that a lane holds one pixel and 4
// consecutive channels: dout and the saved gate are read, and d_go / dy written, 8 bytes at a
// time straight from the accumulators; dy is also staged in LDS for d(on) = dy p_out_w, again
// [channel][pixel] blocks, whose per-pixel LayerNorm reductions meet in LDS. Weight fragments
// stay in registers for the whole launch; the column sums of dy, d_go, d(on) x^ and d(on) stay
// in registers until the workgroup ends.
constexpr int OB_W = 8;
constexpr int OB_NT = 64 * OB_W;
constexpr int OB_TP = 64;           // pixels per tile
constexpr int OB_MAX_GRID = 512;    // partial rows of the bias / LayerNorm gradients

template <typename T, int CK, int CHK>
struct ObLds {
  static constexpr int OR = OB_TP + (int)(16 / sizeof(T));  // o tile [CHK][OR]
  static constexpr int ZR = CHK + (int)(16 / sizeof(T));    // on tile [OB_TP][ZR]
  static constexpr int DR = CK + (int)(16 / sizeof(T));     // dy tile [OB_TP][DR]
  static constexpr size_t ot = 0;
  static constexpr size_t zs = ot + (size_t)CHK * OR * sizeof(T);
  static constexpr size_t dys = zs + (size_t)OB_TP * ZR * sizeof(T);
  static constexpr size_t red1 = dys + (size_t)OB_TP * DR * sizeof(T);  // [8 parts][32 pairs] f32x2 sums
  static constexpr size_t red2 = red1 + 8 * 32 * 8;                      // ... squared deviations
  static constexpr size_t red3 = red2 + 8 * 32 * 8;                      // [CHK / 32][OB_TP] LN-bwd sums
  static constexpr size_t stat = red3 + (size_t)(CHK / 32) * OB_TP * 8;  // [OB_TP] (mean, rstd)
  static constexpr size_t lnw = stat + OB_TP * 8;
  static constexpr size_t lnb = lnw + CHK * 4;
  static constexpr size_t bpo = lnb + CHK * 4;
  static constexpr size_t fin = bpo + CK * 4;  // [2 halves][4][128] final column sums
  static constexpr size_t total = fin + 2 * 4 * 128 * 4;
};

template <typename T, int CK, int CHK>
__global__ __launch_bounds__(OB_NT, 1) void trimul_out_bwd_kernel(const gnn_trimul_out_bwd_args a) {
  typedef ObLds<T, CK, CHK> S;
  typedef typename TypeOps<T>::V8 V8;
  typedef typename TypeOps<T>::V4 V4;
  constexpr int NUY = CK / 32, NUD = CHK / 32;  // output-channel units of y and of d(on)
  constexpr int NKY = CHK / 16, NKD = CK / 16;   // their k-steps
  constexpr int OR = S::OR, ZR = S::ZR, DR = S::DR;
  __shared__ __align__(16) unsigned char smem[S::total];
  T* ot = reinterpret_cast<T*>(smem + S::ot);
  T* zs = reinterpret_cast<T*>(smem + S::zs);
  T* dys = reinterpret_cast<T*>(smem + S::dys);
  float2* red1 = reinterpret_cast<float2*>(smem + S::red1);
  float2* red2 = reinterpret_cast<float2*>(smem + S::red2);
  float2* red3 = reinterpret_cast<float2*>(smem + S::red3);
  float2* stat = reinterpret_cast<float2*>(smem + S::stat);
  float* lnw = reinterpret_cast<float*>(smem + S::lnw);
  float* lnb = reinterpret_cast<float*>(smem + S::lnb);
  float* bpo = reinterpret_cast<float*>(smem + S::bpo);
  float* fin = reinterpret_cast<float*>(smem + S::fin);
  const int N = (int)a.N;
  const int64_t NP = (a.N + 31) / 32 * 32;
  const int ntj = (N + OB_TP - 1) / OB_TP;
  const int64_t ntiles = a.B * a.N * ntj;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;

  for (int c = tid; c < CHK; c += OB_NT) {
    lnw[c] = a.ln_w ? TypeOps<T>::to_f32(((const T*)a.ln_w)[c]) : 1.f;
    lnb[c] = a.ln_b ? TypeOps<T>::to_f32(((const T*)a.ln_b)[c]) : 0.f;
  }
  for (int c = tid; c < CK; c += OB_NT) bpo[c] = a.p_out_b ? TypeOps<T>::to_f32(((const T*)a.p_out_b)[c]) : 0.f;

  // y: wave = (unit uy, pixel half hy); A fragments row = output channel 32 uy + l32, k = 16 kk + 8 g + e
  const int uy = wave % NUY, hy = wave / NUY;
  const bool has_y = hy < 2;  // uniform over the wave
  // d(on): wave = (unit ud, pixel half hd); A fragments row = channel 32 ud + l32, k = output channel
  const int ud = wave % NUD, hd = wave / NUD;
  const bool has_d = hd < 2;
  const T* wpo = (const T*)a.p_out_w;
  V8 wy[NKY], wd[NKD];
#pragma unroll
  for (int k = 0; k < NKY; ++k) wy[k] = load8(wpo + (int64_t)((has_y ? 32 * uy : 0) + l32) * CHK + 16 * k + 8 * g);
#pragma unroll
  for (int k = 0; k < NKD; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) wd[k][e] = wpo[(int64_t)(16 * k + 8 * g + e) * CHK + (has_d ? 32 * ud : 0) + l32];
  float s_dy[16], s_dgo[16], s_dx[16], s_db[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) s_dy[i] = s_dgo[i] = s_dx[i] = s_db[i] = 0.f;

  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    const int jt = (int)(t % ntj);
    const int64_t rest = t / ntj;
    const int i = (int)(rest % N);
    const int64_t b = rest / N;
    const int j0 = jt * OB_TP;
    const int64_t pb = (b * N + i) * N + j0;  // the tile's first pixel

    // ---- 1. the o tile [CHK][64] (columns past N zero), and this lane's dout / gate
    constexpr int OCH = CHK * (OB_TP / 8) / OB_NT;  // 16-byte chunks per thread (0 when CHK < 64)
#pragma unroll
    for (int k = 0; k < (OCH > 0 ? OCH : 1); ++k) {
      const int c = tid + k * OB_NT;
      if (c < CHK * (OB_TP / 8)) {
        const int ch = c / (OB_TP / 8), jj = (c % (OB_TP / 8)) * 8;
        V8 v = zero8<T>();
        if (j0 + jj < N) {
          v = load8((const T*)a.o + ((b * CHK + ch) * N + i) * NP + j0 + jj);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (j0 + jj + e >= N) v[e] = TypeOps<T>::from_f32(0.f);
        }
        store8(&ot[ch * OR + jj], v);
      }
    }
    const int pxy = 32 * hy + l32;
    const bool vy = has_y && j0 + pxy < N;
    const int64_t piy = pb + (vy ? pxy : 0);  // rows past N read the tile's first pixel
    V4 dout4[4], gate4[4];
    if (has_y) {
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int c0 = 32 * uy + 8 * rg + 4 * g;
        dout4[rg] = load4((const T*)a.dout + piy * CK + c0);
        gate4[rg] = load4((const T*)a.gate + piy * CK + c0);
      }
    }
    __syncthreads();

    // ---- 2. LN_out over the CHK channels of each pixel: thread = (pixel pair pp, part of
    // CHK / 8 channels), threads 0 .. 255
    typedef T T2 __attribute__((ext_vector_type(2)));
    const int pp = tid & 31, part = (tid >> 5) & 7;
    constexpr int KC = CHK / 8;
    const int k0 = part * KC;
    auto pair = [&](int k) -> f32x2 {
      return __builtin_convertvector(*reinterpret_cast<const T2*>(&ot[k * OR + 2 * pp]), f32x2);
    };
    f32x2 mean = {0.f, 0.f};
    if (tid < 256) {
      f32x2 s2 = {0.f, 0.f};
#pragma unroll
      for (int k = k0; k < k0 + KC; ++k) s2 += pair(k);
      red1[part * 32 + pp] = make_float2(s2[0], s2[1]);
    }
    __syncthreads();
    f32x2 rs = {0.f, 0.f};
    if (tid < 256) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float2 v = red1[j * 32 + pp];
        mean += f32x2{v.x, v.y};
      }
      mean *= 1.0f / CHK;
      f32x2 q2 = {0.f, 0.f};
#pragma unroll
      for (int k = k0; k < k0 + KC; ++k) {
        const f32x2 d = pair(k) - mean;
        q2 += d * d;
      }
      red2[part * 32 + pp] = make_float2(q2[0], q2[1]);
    }
    __syncthreads();
    if (tid < 256) {
      f32x2 var = {0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float2 v = red2[j * 32 + pp];
        var += f32x2{v.x, v.y};
      }
      rs[0] = 1.0f / sqrtf(var[0] * (1.0f / CHK) + a.eps);
      rs[1] = 1.0f / sqrtf(var[1] * (1.0f / CHK) + a.eps);
      if (part == 0) {
        stat[2 * pp] = make_float2(mean[0], rs[0]);
        stat[2 * pp + 1] = make_float2(mean[1], rs[1]);
      }
#pragma unroll
      for (int k = k0; k < k0 + KC; ++k) {
        const f32x2 x = pair(k);
        zs[(2 * pp) * ZR + k] = TypeOps<T>::from_f32((x[0] - mean[0]) * rs[0] * lnw[k] + lnb[k]);
        zs[(2 * pp + 1) * ZR + k] = TypeOps<T>::from_f32((x[1] - mean[1]) * rs[1] * lnw[k] + lnb[k]);
      }
    }
    __syncthreads();
    // on to its pixel-major rows (16-byte chunks)
    for (int c = tid; c < OB_TP * (CHK / 8); c += OB_NT) {
      const int px = c / (CHK / 8), k = (c % (CHK / 8)) * 8;
      if (j0 + px < N) store8((T*)a.on + (pb + px) * CHK + k, load8(&zs[px * ZR + k]));
    }

    // ---- 3. y and the output gate's backward
    if (has_y) {
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
      for (int k = 0; k < NKY; ++k)
        Mma<T, PREC_NATIVE>::step(acc, wy[k], load8(&zs[pxy * ZR + 16 * k + 8 * g]));
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int c0 = 32 * uy + 8 * rg + 4 * g;
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bpo[c0]);
        const f32x4 d4 = TypeOps<T>::to_f32(dout4[rg]), s4 = TypeOps<T>::to_f32(gate4[rg]);
        f32x4 dy, dg;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float y = TypeOps<T>::to_f32(TypeOps<T>::from_f32(acc[4 * rg + e] + b4[e]));
          dy[e] = d4[e] * s4[e];
          dg[e] = d4[e] * y * s4[e] * (1.0f - s4[e]);
        }
        const V4 dyr = TypeOps<T>::from_f32(dy), dgr = TypeOps<T>::from_f32(dg);
        store4(&dys[pxy * DR + c0], dyr);
        if (vy) {
          store4((T*)a.dy + piy * CK + c0, dyr);
          store4((T*)a.d_go + piy * a.dgo_ld + c0, dgr);
          const f32x4 dyf = TypeOps<T>::to_f32(dyr), dgf = TypeOps<T>::to_f32(dgr);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s_dy[4 * rg + e] += dyf[e];
            s_dgo[4 * rg + e] += dgf[e];
          }
        }
      }
    }
    __syncthreads();

    // ---- 4. d(on) = dy p_out_w and the LN_out backward
    const int pxd = 32 * hd + l32;
    const bool vd = has_d && j0 + pxd < N;
    f32x4 donv[4];  // d(on) rounded as the linear's output; x^ is read again after the barrier
    float2 st = make_float2(0.f, 1.f);
    if (has_d) {
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
      for (int k = 0; k < NKD; ++k)
        Mma<T, PREC_NATIVE>::step(acc, wd[k], load8(&dys[pxd * DR + 16 * k + 8 * g]));
      st = stat[pxd];
      float sg = 0.f, sgx = 0.f;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int c0 = 32 * ud + 8 * rg + 4 * g;
        const f32x4 w4 = *reinterpret_cast<const f32x4*>(&lnw[c0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float don = TypeOps<T>::to_f32(TypeOps<T>::from_f32(acc[4 * rg + e]));
          const float x = (TypeOps<T>::to_f32(ot[(c0 + e) * OR + pxd]) - st.x) * st.y;
          donv[rg][e] = don;
          const float gc = don * w4[e];
          sg += gc;
          sgx += gc * x;
          if (vd) {
            s_dx[4 * rg + e] += don * x;
            s_db[4 * rg + e] += don;
          }
        }
      }
      // the pixel's two lanes (l, l ^ 32) hold its other channels of this unit
      sg += __shfl_xor(sg, 32);
      sgx += __shfl_xor(sgx, 32);
      if (g == 0) red3[ud * OB_TP + pxd] = make_float2(sg, sgx);
    }
    __syncthreads();
    if (has_d) {
      float mg = 0.f, mgx = 0.f;
#pragma unroll
      for (int u = 0; u < NUD; ++u) {
        const float2 v = red3[u * OB_TP + pxd];
        mg += v.x;
        mgx += v.y;
      }
      mg *= 1.0f / CHK;
      mgx *= 1.0f / CHK;
      if (vd) {
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int c0 = 32 * ud + 8 * rg + 4 * g;
          const f32x4 w4 = *reinterpret_cast<const f32x4*>(&lnw[c0]);
          f32x4 dx;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = (TypeOps<T>::to_f32(ot[(c0 + e) * OR + pxd]) - st.x) * st.y;
            dx[e] = st.y * (donv[rg][e] * w4[e] - mg - x * mgx);
          }
          store4((T*)a.d_o + (pb + pxd) * CHK + c0, TypeOps<T>::from_f32(dx));
        }
      }
    }
    __syncthreads();  // ot / zs / dys / red3 free for the next tile
  }

  // ---- the workgroup's column sums: over the 32 pixels of a lane group, then the two halves
#pragma unroll
  for (int i = 0; i < 16; ++i) {
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
      s_dy[i] += __shfl_xor(s_dy[i], o);
      s_dgo[i] += __shfl_xor(s_dgo[i], o);
      s_dx[i] += __shfl_xor(s_dx[i], o);
      s_db[i] += __shfl_xor(s_db[i], o);
    }
  }
  for (int c = tid; c < 2 * 4 * 128; c += OB_NT) fin[c] = 0.f;
  __syncthreads();
  if (l32 == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int cc = 8 * (i / 4) + 4 * g + (i % 4);
      if (has_y) {
        fin[(hy * 4 + 0) * 128 + 32 * uy + cc] = s_dy[i];
        fin[(hy * 4 + 1) * 128 + 32 * uy + cc] = s_dgo[i];
      }
      if (has_d) {
        fin[(hd * 4 + 2) * 128 + 32 * ud + cc] = s_dx[i];
        fin[(hd * 4 + 3) * 128 + 32 * ud + cc] = s_db[i];
      }
    }
  }
  __syncthreads();
  for (int c = tid; c < 4 * 128; c += OB_NT) a.partial[(int64_t)blockIdx.x * 4 * 128 + c] = fin[c] + fin[4 * 128 + c];
}

template <typename T, int CK, int CHK>
int launch_out_bwd(const gnn_trimul_out_bwd_args& a, hipStream_t st) {
  const int64_t grid = trimul_out_bwd_partials(a.B, a.N);
  hipLaunchKernelGGL((trimul_out_bwd_kernel<T, CK, CHK>), dim3((uint32_t)grid), dim3(OB_NT), 0, st, a);
  return (int)hipGetLastError();
}

template <typename T>
int launch_out_bwd_t(const gnn_trimul_out_bwd_args& a, hipStream_t st) {
  if (a.C == 128) {
    if (a.Ch == 128) return launch_out_bwd<T, 128, 128>(a, st);
    if (a.Ch == 64) return launch_out_bwd<T, 128, 64>(a, st);
    return launch_out_bwd<T, 128, 32>(a, st);
  }
  if (a.Ch == 128) return launch_out_bwd<T, 64, 128>(a, st);
  if (a.Ch == 64) return launch_out_bwd<T, 64, 64>(a, st);
  return launch_out_bwd<T, 64, 32>(a, st);
}

}  // namespace

int64_t gate_bwd_partials(int64_t rows, int64_t K) {
  if (K < 8 || K % 8 != 0 || GB_THREADS % (K / 8) != 0) return 0;
  const int64_t want = (rows * (K / 8) + GB_THREADS - 1) / GB_THREADS;
  return want < 1 ? 1 : (want > GB_MAX_GRID ? GB_MAX_GRID : want);
}

int64_t trimul_proj_bwd_partials(int64_t rows) {
  const int64_t t = (rows + PB_TP - 1) / PB_TP;
  return t < 1 ? 1 : (t > PB_MAX_GRID ? PB_MAX_GRID : t);
}

int trimul_proj_bwd(const gnn_trimul_proj_bwd_args& a, hipStream_t st) {
  if ((a.C != 64 && a.C != 128) || a.Ch < 16 || a.Ch > 128 || (2 * a.Ch) % 32 != 0)
    return set_error(GNN_ERR_UNSUPPORTED, "trimul_proj_bwd: C must be 64 or 128 and 2 * c_hidden a multiple of 32, at most 256");
  switch (a.dtype) {
    case GNN_BF16: return a.C == 128 ? launch_proj_bwd<bf16, 128>(a, st) : launch_proj_bwd<bf16, 64>(a, st);
    case GNN_F16: return a.C == 128 ? launch_proj_bwd<f16, 128>(a, st) : launch_proj_bwd<f16, 64>(a, st);
  }
  return set_error(GNN_ERR_UNSUPPORTED, "trimul_proj_bwd: bf16 / fp16 only");
}

int64_t trimul_out_bwd_partials(int64_t B, int64_t N) {
  const int64_t t = B * N * ((N + OB_TP - 1) / OB_TP);
  return t < 1 ? 1 : (t > OB_MAX_GRID ? OB_MAX_GRID : t);
}

int trimul_out_bwd(const gnn_trimul_out_bwd_args& a, hipStream_t st) {
  if ((a.C != 64 && a.C != 128) || (a.Ch != 32 && a.Ch != 64 && a.Ch != 128))
    return set_error(GNN_ERR_UNSUPPORTED, "trimul_out_bwd: C must be 64 or 128 and c_hidden 32, 64 or 128");
  switch (a.dtype) {
    case GNN_BF16: return launch_out_bwd_t<bf16>(a, st);
    case GNN_F16: return launch_out_bwd_t<f16>(a, st);
  }
  return set_error(GNN_ERR_UNSUPPORTED, "trimul_out_bwd: bf16 / fp16 only");
}

int64_t layernorm_partials(int64_t rows, int64_t K) {
  (void)K;
  const int64_t want = (rows + LN_ROWS * LN_UNROLL - 1) / (LN_ROWS * LN_UNROLL);
  return want < 1 ? 1 : (want > LN_MAX_GRID ? LN_MAX_GRID : want);
}

int layernorm_rows(const gnn_layernorm_args& a, hipStream_t st) {
  const bool bwd = a.dy != nullptr;
  if (a.K % 32 == 0 && a.K > LN_MAX_K && a.K <= LN_WIDE_MAX_K && !bwd) {
    // wide rows: forward only; 16-byte row accesses
    const int64_t e = a.dtype == GNN_F32 ? 4 : 2;
    if (((uintptr_t)a.x | (uintptr_t)a.out) % 16 != 0 || (a.x_stride * e) % 16 != 0 || (a.out_stride * e) % 16 != 0)
      return set_error(GNN_ERR_ARG, "layernorm_rows: rows wider than 512 need 16-byte aligned rows");
    switch (a.dtype) {
      case GNN_BF16: return launch_ln_wide<bf16>(a, st);
      case GNN_F16: return launch_ln_wide<f16>(a, st);
      case GNN_F32: return launch_ln_wide<float>(a, st);
    }
    return set_error(GNN_ERR_ARG, "layernorm_rows: unknown dtype");
  }
  if (a.K % 32 != 0 || a.K > LN_MAX_K)
    return set_error(GNN_ERR_UNSUPPORTED,
                     "layernorm_rows: K must be a multiple of 32, at most 512 (8192 for the forward)");
  switch (a.dtype) {
    case GNN_BF16: return bwd ? launch_ln<bf16, true>(a, st) : launch_ln<bf16, false>(a, st);
    case GNN_F16: return bwd ? launch_ln<f16, true>(a, st) : launch_ln<f16, false>(a, st);
    case GNN_F32: return bwd ? launch_ln<float, true>(a, st) : launch_ln<float, false>(a, st);
  }
  return set_error(GNN_ERR_ARG, "layernorm_rows: unknown dtype");
}

int gate_bwd(const gnn_gate_bwd_args& a, hipStream_t st) {
  if (a.K % 8 != 0) return set_error(GNN_ERR_UNSUPPORTED, "gate_bwd: K must be a multiple of 8");
  switch (a.dtype) {
    case GNN_BF16: return launch_gate<bf16>(a, st);
    case GNN_F16: return launch_gate<f16>(a, st);
    case GNN_F32: return launch_gate<float>(a, st);
  }
  return set_error(GNN_ERR_ARG, "gate_bwd: unknown dtype");
}

}  // namespace gnn
