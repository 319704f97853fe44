// Triangle attention backward for gfx950, row-resident variant of dq and dk / dv: 16-bit
// inputs, head dim 32, N_res <= BWD_ROW_MAX_N.
//
// Same mathematics and the same per-element arithmetic as bwd_dq_kernel and
// bwd_dkdv_kernel (triattn_bwd.hip), so both paths give identical results:
//   dP_ij = dO_i . v_j,  dS_ij = P_ij (dP_ij - Delta_i),  P_ij = exp(S_ij - lse_i),
//   dV_j = sum_i P_ij dO_i,  dK_j = sum_i dS_ij Q'_i,  dQ_i = scale * sum_j dS_ij k_j,
// the gradient of triangle_attention_torch (geometric_nn_ops_torch/triangle/_reference/
// triangle_attention.py:11-44) that the reference's Triton backward computes
// (geometric_nn_ops_torch/triangle/_kernels/triangle_attention.py:548-1087).
//
// What changes is the schedule, as in the forward's row kernel (triattn_row.hip): one
// workgroup of 8 waves per (b, s, h) row stages the operands the row's loops sweep ONCE in
// LDS and its waves then run their loops with no barrier (the tiled kernels re-stage a
// 64-row tile behind two barriers per step, exposing the load latency every step):
//   bwd_dq_row    K and V of the row (global_load_lds, chunks XOR-swizzled by (row / 4) % 4),
//                 the per-key mask term and a per-64-key-tile "no masked key" flag; the waves
//                 take 32-query blocks round robin and sweep every key tile. Also writes
//                 Delta = rowsum(dO * O) for bwd_dkdv_row and bwd_dbias.
//   bwd_dkdv_row  Q' = bf16(q * scale) (through registers: the product is rounded) and dO
//                 (global_load_lds) of the row, with its lse and Delta; the waves take
//                 32-key blocks round robin and sweep every query tile.
// The pair-bias fragments of the next step are requested from global memory (L2: a bias
// plane is shared by every N_seq row) while the current one is computed. The reference's
// correction for rows whose keys are all masked (P of a masked key divided by N_res, which
// only changes such rows: elsewhere a masked key's P is exactly 0) is applied per row, as
// P = exp2((S - lse) log2(e) - log2(N_res)) where the row's lse sits at the mask sentinel.
#include <type_traits>

#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

constexpr float LOG2E_R = 1.4426950408889634f;
constexpr int RW = 8;             // waves per workgroup
constexpr int RNT = 64 * RW;      // threads per workgroup
constexpr int RT = 64;            // rows (keys or queries) per tile
constexpr int RROW = 64;          // bytes per staged row (32 x 16-bit)
constexpr int RTILE = RT * RROW;  // bytes per staged tile
constexpr int BWD_ROW_MAX_N = 1024;
constexpr int RMAX_TILES = BWD_ROW_MAX_N / RT;

// byte offset of (row r, 16-byte chunk c) of a staged [rows][32] tile, chunks XOR-swizzled
// by (r / 4) % 4 (the layout of bwd_dq_kernel / bwd_dkdv_kernel's tiles)
__device__ __forceinline__ int rswz(int r, int c) { return r * RROW + 16 * (c ^ ((r >> 2) & 3)); }

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 rrow8(const unsigned char* base, int r, int c) {
  return *reinterpret_cast<const typename TypeOps<T>::V8*>(base + rswz(r, c));
}

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V4 rtr4(const unsigned char* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(__attribute__((address_space(3))) const unsigned char*)p);
  return __builtin_bit_cast(typename TypeOps<T>::V4, v);
}

// Transposed B fragment of a staged tile: k = rows row0 + 16 kk + 8 (e / 4) + 4 g + e % 4 (the
// 32x32 accumulator's row order), n = column lane % 32.
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 rtr_frag(const unsigned char* tile, int row0, int kk, int lane) {
  const int g = lane >> 5, r16 = lane & 15;
  const int col = 16 * ((lane >> 4) & 1) + 4 * (r16 & 3);
  typename TypeOps<T>::V8 f;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int row = row0 + 16 * kk + 8 * hh + 4 * g + (r16 >> 2);
    const typename TypeOps<T>::V4 x = rtr4<T>(tile + rswz(row, col >> 3) + 2 * (col & 7));
#pragma unroll
    for (int e = 0; e < 4; ++e) f[4 * hh + e] = x[e];
  }
  return f;
}

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 racc_frag(const f32x16& a, int kk) {
  f32x8 x = {a[8 * kk + 0], a[8 * kk + 1], a[8 * kk + 2], a[8 * kk + 3],
             a[8 * kk + 4], a[8 * kk + 5], a[8 * kk + 6], a[8 * kk + 7]};
  return TypeOps<T>::from_f32(x);
}

template <typename T>
__device__ __forceinline__ void ridentity(typename TypeOps<T>::V8 (&idf)[2], int l32, int g) {
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) idf[t][e] = TypeOps<T>::from_f32(l32 == 16 * t + 8 * g + e ? 1.f : 0.f);
}

// Stage rows 0 .. ntiles * 64 - 1 of a [N][32] 16-bit operand (row stride rs elements) into
// a swizzled LDS image with global_load_lds_dwordx4: one instruction moves 16 rows (1 KB),
// lane l filling bytes 16 l .. 16 l + 15 = row l / 4, physical chunk l % 4, which holds
// logical chunk (l % 4) ^ ((l / 16) % 4). Rows past N repeat row N - 1 (finite values whose
// weights are zero).
template <typename T>
__device__ __forceinline__ void stage_rows_dma(unsigned char* dst, const T* src, int64_t rs, int N, int ntiles,
                                               int wave, int lane) {
  const int lrow = lane >> 2, ch = (lane & 3) ^ ((lane >> 4) & 3);
  for (int q = wave; q < ntiles * (RT / 16); q += RW) {
    const int r = min(16 * q + lrow, N - 1);
    __builtin_amdgcn_global_load_lds((const void*)(src + (int64_t)r * rs + 8 * ch),
                                     (__attribute__((address_space(3))) void*)(dst + q * 1024), 16, 0, 0);
  }
}

// Logical workgroup order of the row kernels: the two heads of a pair fastest (they share
// the 128-byte lines of the K / V / Q / dO rows at D = 32), then N_seq, so an XCD keeps the
// bias planes of few heads in its L2; odd H takes rows fastest.
__device__ __forceinline__ void row_coords(uint32_t w, int S, int H, int& b, int& s, int& h) {
  if (H % 2 == 0) {
    const uint32_t hi = w & 1u, rest = w >> 1;
    s = (int)(rest % (uint32_t)S);
    h = 2 * (int)((rest / (uint32_t)S) % (uint32_t)(H / 2)) + (int)hi;
  } else {
    s = (int)(w % (uint32_t)S);
    h = (int)((w / (uint32_t)S) % (uint32_t)H);
  }
  b = (int)(w / ((uint32_t)S * H));
}

// -log2(N_res) for a row whose keys are all masked (its lse then holds the bare mask
// sentinel: log(l) is below the fp32 ulp there), else 0; added to the exp2 argument it
// divides P by N_res. A live row's lse is the logsumexp of real logits, far above half the
// sentinel.
__device__ __forceinline__ float dead_row_log2(const gnn_triattn_bwd_args& a, float lse) {
  return (a.mask && lse <= 0.5f * a.mask_value) ? -__log2f((float)a.N) : 0.f;
}

// ------------------------------------------------------------------------------- dQ
struct DqRowHdr {
  float kterm[BWD_ROW_MAX_N];  // added to the scores of key j: 0, the mask sentinel, or -inf past N
  int plain[RMAX_TILES];       // tile t has no masked key and no key past N
};
constexpr int DQ_HDR = (int)((sizeof(DqRowHdr) + 255) / 256 * 256);

template <typename T, bool HAS_BIAS>
__global__ __launch_bounds__(RNT, 4) void bwd_dq_row_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(256) unsigned char smem_raw[];
  DqRowHdr& hdr = *reinterpret_cast<DqRowHdr*>(smem_raw);
  const int N = (int)a.N, H = (int)a.H, S = (int)a.S;
  const int ntiles = (N + RT - 1) / RT;
  unsigned char* ks = smem_raw + DQ_HDR;
  unsigned char* vs = ks + ntiles * RTILE;
  int b, s, h;
  row_coords(xcd_remap(blockIdx.x, gridDim.x), S, H, b, s, h);
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const T* kp = (const T*)a.k + b * a.k_stride[0] + s * a.k_stride[1] + h * a.k_stride[3];
  const T* vp = (const T*)a.v + b * a.v_stride[0] + s * a.v_stride[1] + h * a.v_stride[3];
  stage_rows_dma<T>(ks, kp, a.k_stride[2], N, ntiles, wave, lane);
  stage_rows_dma<T>(vs, vp, a.v_stride[2], N, ntiles, wave, lane);
  if (wave == 0) {
    for (int t = 0; t < ntiles; ++t) {
      const int key = t * RT + lane;
      float kt = 0.f;
      if (key >= N)
        kt = -INFINITY;
      else if (a.mask && a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)key * a.mask_stride[2]] == 0)
        kt = a.mask_value;
      hdr.kterm[key] = kt;
      const bool plain = __ballot(kt != 0.f) == 0;
      if (lane == 0) hdr.plain[t] = plain;
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): this wave's LDS DMA has landed
  __syncthreads();

  V8 idf[2];
  ridentity<T>(idf, l32, g);
  const int64_t lrow = (((int64_t)b * S + s) * H + h) * N;
  const int nqb = (N + 31) / 32;
  for (int qblk = wave; qblk < nqb; qblk += RW) {
    int Nq = N;  // opaque: keeps the tail compares of the bias loads inside the loop
    asm volatile("" : "+s"(Nq));
    const int qi = qblk * 32 + l32;
    const bool qok = qi < Nq;
    // this lane's query: Q' and dO as B operands (lane = query, 8 consecutive d)
    V8 qf[2], dof[2];
    float delta;
    {
      const T* qr = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3] +
                    (int64_t)(qok ? qi : 0) * a.q_stride[2];
      const T* dr = (const T*)a.dout + b * a.do_stride[0] + s * a.do_stride[1] + h * a.do_stride[3] +
                    (int64_t)(qok ? qi : 0) * a.do_stride[2];
      const T* orow = (const T*)a.o + b * a.o_stride[0] + s * a.o_stride[1] + h * a.o_stride[3] +
                      (int64_t)(qok ? qi : 0) * a.o_stride[2];
      float part = 0.f;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int d0 = 16 * kk + 8 * g;
        qf[kk] = qok ? TypeOps<T>::from_f32(TypeOps<T>::to_f32(load8(qr + d0)) * a.scale) : zero8<T>();
        dof[kk] = qok ? load8(dr + d0) : zero8<T>();
        const f32x8 x = TypeOps<T>::to_f32(qok ? load8(orow + d0) : zero8<T>());
        const f32x8 y = TypeOps<T>::to_f32(dof[kk]);
#pragma unroll
        for (int e = 0; e < 8; ++e) part = __builtin_fmaf(x[e], y[e], part);
      }
      // Delta = dO . O: the lane pair (g = 0, 1) holds the 32 columns between them
      delta = part + __shfl_xor(part, 32);
      if (qok && g == 0) a.delta[lrow + qi] = delta;
    }
    const float lse = qok ? a.lse[lrow + qi] : INFINITY;  // absent queries: p = 0
    const float pl2 = dead_row_log2(a, lse);
    // Unless a query of the wave sits in a fully masked row, P = exp2(S log2 e - lse log2 e)
    // takes one fma per element (lse is this lane's query's, constant along the accumulator);
    // a fully masked row keeps S - lse formed first (both sit near the sentinel).
    const bool dead = __any(pl2 != 0.f);
    const float nl2 = -lse * LOG2E_R;
    const T* brow = HAS_BIAS ? (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] +
                                   (int64_t)(qok ? qi : 0) * a.bias_stride[2]
                             : nullptr;
    // bias fragments of one 32-key step: keys 32 st + 16 t + 8 g + 0..7 of the lane's query
    V8 bb[2];
    auto load_bias = [&](int st) {
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) bb[t2] = load8_bias_tail<T>(brow, 32 * st + 16 * t2 + 8 * g, Nq);
    };
    if constexpr (HAS_BIAS) load_bias(0);
    f32x16 dq;
#pragma unroll
    for (int i = 0; i < 16; ++i) dq[i] = 0.f;

    // 32-key steps: S^T[key][q] = K Q'^T (+ bias) and dP^T[key][q] = V dO^T, rows = keys
    // 32 st + 8 (i / 4) + 4 g + i % 4, column = query
    const int nst = 2 * ntiles;
    for (int st = 0; st < nst; ++st) {
      const unsigned char* kt = ks + st * (RTILE / 2);
      const unsigned char* vt = vs + st * (RTILE / 2);
      const bool plain = hdr.plain[st >> 1] != 0;
      f32x16 sc, dp;
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] = dp[i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        Mma<T, PREC_NATIVE>::step(sc, rrow8<T>(kt, l32, 2 * kk + g), qf[kk]);
        Mma<T, PREC_NATIVE>::step(dp, rrow8<T>(vt, l32, 2 * kk + g), dof[kk]);
      }
      if constexpr (HAS_BIAS) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) Mma<T, PREC_NATIVE>::step(sc, idf[t2], bb[t2]);
        if (st + 1 < nst) load_bias(st + 1);
      }
      // P = exp(S - lse), subtracting first: in a row whose keys are all masked both sit
      // near the sentinel, and only their difference is exact
      f32x16 ds;
      if (plain && !dead) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ds[i] = fast_exp2(__builtin_fmaf(sc[i], LOG2E_R, nl2)) * (dp[i] - delta);
      } else if (!dead) {
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const f32x4 k4 = *reinterpret_cast<const f32x4*>(&hdr.kterm[32 * st + 8 * rg + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * rg + e;
            ds[i] = fast_exp2(__builtin_fmaf(sc[i] + k4[e], LOG2E_R, nl2)) * (dp[i] - delta);
          }
        }
      } else {
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const f32x4 k4 = *reinterpret_cast<const f32x4*>(&hdr.kterm[32 * st + 8 * rg + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * rg + e;
            ds[i] = fast_exp2(__builtin_fmaf(sc[i] + k4[e] - lse, LOG2E_R, pl2)) * (dp[i] - delta);
          }
        }
      }
      // dQ += dS K: A = the dS^T accumulator (lane = query, k = keys), B = K read transposed
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        Mma<T, PREC_NATIVE>::step(dq, racc_frag<T>(ds, kk), rtr_frag<T>(kt, 0, kk, lane));
    }
    // dq[m = query][n = d]: lane = d, rows = queries 32 qblk + 8 (i / 4) + 4 g + i % 4
    T* dqp = (T*)a.dq + b * a.dq_stride[0] + s * a.dq_stride[1] + h * a.dq_stride[3] + l32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int qq = qblk * 32 + 8 * (i / 4) + 4 * g + (i % 4);
      if (qq < Nq) dqp[(int64_t)qq * a.dq_stride[2]] = TypeOps<T>::from_f32(dq[i] * a.scale);
    }
  }
}

// --------------------------------------------------------------------------- dK, dV
struct DkdvRowHdr {
  float lse[BWD_ROW_MAX_N];    // +inf for absent queries (p = 0)
  float ndelta[BWD_ROW_MAX_N];  // -Delta (0 for absent queries): the dP accumulators' start
};
constexpr int DKDV_HDR = (int)((sizeof(DkdvRowHdr) + 255) / 256 * 256);

template <typename T>
struct BiasRows {
  typename TypeOps<T>::V8 f[2];  // [t]: keys kbase + 16 t + 8 g + 0..7 of query row r0 + l32
};

template <typename T, bool HAS_BIAS>
__global__ __launch_bounds__(RNT, 4) void bwd_dkdv_row_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(256) unsigned char smem_raw[];
  DkdvRowHdr& hdr = *reinterpret_cast<DkdvRowHdr*>(smem_raw);
  const int N = (int)a.N, H = (int)a.H, S = (int)a.S;
  const int ntiles = (N + RT - 1) / RT;
  const int nrows = ntiles * RT;
  unsigned char* qs = smem_raw + DKDV_HDR;
  unsigned char* ds_ = qs + ntiles * RTILE;
  int b, s, h;
  row_coords(xcd_remap(blockIdx.x, gridDim.x), S, H, b, s, h);
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // dO by DMA; Q' = bf16(q * scale) through registers (rows past N are zero)
  const T* dop = (const T*)a.dout + b * a.do_stride[0] + s * a.do_stride[1] + h * a.do_stride[3];
  stage_rows_dma<T>(ds_, dop, a.do_stride[2], N, ntiles, wave, lane);
  {
    const T* qp = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3];
    constexpr int U = 4;
    for (int base = 0; base < nrows * 4; base += RNT * U) {
      V8 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = base + u * RNT + tid, r = c >> 2;
        x[u] = (c < nrows * 4 && r < N) ? load8(qp + (int64_t)r * a.q_stride[2] + 8 * (c & 3)) : zero8<T>();
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = base + u * RNT + tid, r = c >> 2;
        if (c < nrows * 4)
          *reinterpret_cast<V8*>(qs + rswz(r, c & 3)) = TypeOps<T>::from_f32(TypeOps<T>::to_f32(x[u]) * a.scale);
      }
    }
    const int64_t lrow = (((int64_t)b * S + s) * H + h) * N;
    for (int r = tid; r < nrows; r += RNT) {
      hdr.lse[r] = r < N ? a.lse[lrow + r] : INFINITY;
      hdr.ndelta[r] = r < N ? -a.delta[lrow + r] : 0.f;
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): this wave's LDS DMA has landed
  __syncthreads();

  V8 idf[2];
  ridentity<T>(idf, l32, g);
  const float pl2 = dead_row_log2(a, hdr.lse[0]);  // query 0 exists (N >= 1)
  const T* bias_plane = HAS_BIAS ? (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] : nullptr;
  const int nkb = (N + 31) / 32;
  const int nsub = 2 * ntiles;  // 32-query steps
  for (int kblk = wave; kblk < nkb; kblk += RW) {
    int Nk = N;  // opaque, as in the dq kernel
    asm volatile("" : "+s"(Nk));
    const int key = kblk * 32 + l32;
    const bool kok = key < Nk;
    // this lane's key: K and V as B operands (lane = key, 8 consecutive d)
    V8 kf[2], vf[2];
    {
      const T* kr = (const T*)a.k + b * a.k_stride[0] + s * a.k_stride[1] + h * a.k_stride[3] +
                    (int64_t)(kok ? key : 0) * a.k_stride[2];
      const T* vr = (const T*)a.v + b * a.v_stride[0] + s * a.v_stride[1] + h * a.v_stride[3] +
                    (int64_t)(kok ? key : 0) * a.v_stride[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        kf[kk] = kok ? load8(kr + 16 * kk + 8 * g) : zero8<T>();
        vf[kk] = kok ? load8(vr + 16 * kk + 8 * g) : zero8<T>();
      }
    }
    // key-side mask term: the sentinel for masked keys, -inf for keys past N (p = 0)
    float kbias = 0.f;
    if (!kok)
      kbias = -INFINITY;
    else if (a.mask && a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)key * a.mask_stride[2]] == 0)
      kbias = a.mask_value;
    // bias rows of the 32 queries of a step: A = bias[query][key] (lane = query, 8 keys)
    auto load_bias = [&](BiasRows<T>& br, int st) {
      const int qq = 32 * st + l32;
      const T* brow = bias_plane + (int64_t)(qq < Nk ? qq : 0) * a.bias_stride[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int k0 = kblk * 32 + 16 * t + 8 * g;
        br.f[t] = qq < Nk ? load8_bias_tail<T>(brow, k0, Nk) : zero8<T>();
      }
    };
    BiasRows<T> bb;
    if constexpr (HAS_BIAS) load_bias(bb, 0);
    f32x16 dk, dv;
#pragma unroll
    for (int i = 0; i < 16; ++i) dk[i] = dv[i] = 0.f;

    for (int st = 0; st < nsub; ++st) {
      const int r0 = 32 * st;
      // S[q][key] = Q' K^T (+ bias) and dP[q][key] - Delta_q = dO V^T - Delta (the accumulator
      // starts at -Delta): rows = queries r0 + 8 (i / 4) + 4 g + i % 4, column = key
      f32x16 sc, dp;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const f32x4 nd4 = *reinterpret_cast<const f32x4*>(&hdr.ndelta[r0 + 8 * rg + 4 * g]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc[4 * rg + e] = 0.f;
          dp[4 * rg + e] = nd4[e];
        }
      }
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        Mma<T, PREC_NATIVE>::step(sc, rrow8<T>(qs, r0 + l32, 2 * kk + g), kf[kk]);
        Mma<T, PREC_NATIVE>::step(dp, rrow8<T>(ds_, r0 + l32, 2 * kk + g), vf[kk]);
      }
      if constexpr (HAS_BIAS) {
#pragma unroll
        for (int t = 0; t < 2; ++t) Mma<T, PREC_NATIVE>::step(sc, bb.f[t], idf[t]);
        if (st + 1 < nsub) load_bias(bb, st + 1);
      }
      // P and dS for this lane's key and its 16 queries, 8 at a time (k-step kk of the
      // products): dV += P^T dO and dK += dS^T Q' with A = P / dS (lane = key, k = queries)
      // and B = the staged rows read transposed (k = queries, n = d)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        f32x8 pv, dv8;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int rg = 2 * kk + hh;
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(&hdr.lse[r0 + 8 * rg + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * rg + e;
            const float x = fast_exp2(__builtin_fmaf(sc[i] + kbias - l4[e], LOG2E_R, pl2));
            pv[4 * hh + e] = x;
            dv8[4 * hh + e] = x * dp[i];
          }
        }
        Mma<T, PREC_NATIVE>::step(dv, TypeOps<T>::from_f32(pv), rtr_frag<T>(ds_, r0, kk, lane));
        Mma<T, PREC_NATIVE>::step(dk, TypeOps<T>::from_f32(dv8), rtr_frag<T>(qs, r0, kk, lane));
      }
    }
    // dk / dv[m = key][n = d]: lane = d (l32), rows = keys 32 kblk + 8 (i / 4) + 4 g + i % 4
    T* dkp = (T*)a.dk + b * a.dk_stride[0] + s * a.dk_stride[1] + h * a.dk_stride[3] + l32;
    T* dvp = (T*)a.dv + b * a.dv_stride[0] + s * a.dv_stride[1] + h * a.dv_stride[3] + l32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kj = kblk * 32 + 8 * (i / 4) + 4 * g + (i % 4);
      if (kj < Nk) {
        dkp[(int64_t)kj * a.dk_stride[2]] = TypeOps<T>::from_f32(dk[i]);
        dvp[(int64_t)kj * a.dv_stride[2]] = TypeOps<T>::from_f32(dv[i]);
      }
    }
  }
}

template <typename T, bool HAS_BIAS>
int launch_bwd_row(const gnn_triattn_bwd_args& a, hipStream_t stream) {
  const int64_t ntiles = (a.N + RT - 1) / RT;
  const dim3 grid((uint32_t)(a.B * a.S * a.H));
  const size_t smem_dq = DQ_HDR + 2 * (size_t)ntiles * RTILE;
  const size_t smem_dkdv = DKDV_HDR + 2 * (size_t)ntiles * RTILE;
  const void* fdq = (const void*)bwd_dq_row_kernel<T, HAS_BIAS>;
  const void* fdkdv = (const void*)bwd_dkdv_row_kernel<T, HAS_BIAS>;
  if (smem_dq > 64 * 1024) (void)hipFuncSetAttribute(fdq, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem_dq);
  if (smem_dkdv > 64 * 1024)
    (void)hipFuncSetAttribute(fdkdv, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem_dkdv);
  // dq first: it also writes Delta, which dk / dv reads
  hipLaunchKernelGGL((bwd_dq_row_kernel<T, HAS_BIAS>), grid, dim3(RNT), smem_dq, stream, a);
  hipLaunchKernelGGL((bwd_dkdv_row_kernel<T, HAS_BIAS>), grid, dim3(RNT), smem_dkdv, stream, a);
  return (int)hipGetLastError();
}

}  // namespace

bool triattn_bwd_row_applicable(const gnn_triattn_bwd_args& a) {
  return (a.dtype == GNN_BF16 || a.dtype == GNN_F16) && a.D == 32 && a.N >= 1 && a.N <= BWD_ROW_MAX_N &&
         a.B * a.S * a.H < ((int64_t)1 << 31);
}

int triattn_bwd_row_dq_dkdv(const gnn_triattn_bwd_args& a, hipStream_t stream) {
  if (a.dtype == GNN_BF16) return a.bias ? launch_bwd_row<bf16, true>(a, stream) : launch_bwd_row<bf16, false>(a, stream);
  return a.bias ? launch_bwd_row<f16, true>(a, stream) : launch_bwd_row<f16, false>(a, stream);
}

}  // namespace gnn
