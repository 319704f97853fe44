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
      // sigmoid with the hardware exp2 and reciprocal, as the forward's gates
      const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gp[e] * -1.4426950408889634f));
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

}  // namespace

int64_t gate_bwd_partials(int64_t rows, int64_t K) {
  if (K < 8 || K % 8 != 0 || GB_THREADS % (K / 8) != 0) return 0;
  const int64_t want = (rows * (K / 8) + GB_THREADS - 1) / GB_THREADS;
  return want < 1 ? 1 : (want > GB_MAX_GRID ? GB_MAX_GRID : want);
}

int64_t layernorm_partials(int64_t rows, int64_t K) {
  (void)K;
  const int64_t want = (rows + LN_ROWS * LN_UNROLL - 1) / (LN_ROWS * LN_UNROLL);
  return want < 1 ? 1 : (want > LN_MAX_GRID ? LN_MAX_GRID : want);
}

int layernorm_rows(const gnn_layernorm_args& a, hipStream_t st) {
  if (a.K % 32 != 0 || a.K > LN_MAX_K)
    return set_error(GNN_ERR_UNSUPPORTED, "layernorm_rows: K must be a multiple of 32, at most 512");
  const bool bwd = a.dy != nullptr;
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
