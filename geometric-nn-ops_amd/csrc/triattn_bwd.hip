// Triangle attention backward for gfx950: dq, dk, dv and the pair-bias gradient.
//
// The forward (triattn_fwd.hip, triattn_row.hip) saves the natural-log lse of every query;
// with P = exp(S - lse), S = bf16(q * scale) . k + bias + mask_bias:
//   dV_j    = sum_i P_ij dO_i                 dP_ij = dO_i . v_j
//   Delta_i = dO_i . O_i                      dS_ij = P_ij (dP_ij - Delta_i)
//   dK_j    = sum_i dS_ij Q'_i                (Q' = bf16(q * scale), so dK carries the scale)
//   dQ_i    = scale * sum_j dS_ij k_j
//   dbias_ij (per b, h) = sum_s dS_ij         (the bias is shared by every N_seq row)
// which is the gradient of triangle_attention_torch (geometric_nn_ops_torch/triangle/
// _reference/triangle_attention.py:11-44) and what the reference's Triton backward computes
// (geometric_nn_ops_torch/triangle/_kernels/triangle_attention.py:548-1087, launched at
// :1278-1442).
//
// Four kernels, every sum owned by one workgroup (no atomics, deterministic):
//   bwd_delta  Delta = rowsum(dO * O) in fp32.
//   bwd_dkdv   one wave per 32 keys of a (b, s, h) row, looping over 64-query tiles staged
//              in LDS. Scores are computed as S = Q' K^T with the KEYS on the lanes, so the
//              P and dS accumulators already are the A operands of dV += P^T dO and
//              dK += dS^T Q'; the B operands (dO and Q' with queries as k) come from the
//              LDS tiles through ds_read_b64_tr_b16, in the accumulator's row order.
//   bwd_dq     the forward's layout (queries on the lanes, K / V tiles in LDS): the dS^T
//              accumulator is the A operand of dQ += dS K, with K read transposed from LDS.
//   bwd_dbias  one wave per 32 queries x 64 keys of a (b, h) bias plane, looping over the
//              N_seq rows and accumulating sum_s dS in fp32 registers; the bias tile is
//              loaded once into the score accumulator's initial value.
// The bias is added to the scores in fp32 exactly as in the forward (bf16 values, fp32
// sums), and the mask sentinel after it, so P matches the forward's normaliser.
// 16-bit inputs, head dim <= 32 (padded to a multiple of 8 by the host).
#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

constexpr float LOG2E_B = 1.4426950408889634f;
constexpr int BT = 64;      // queries per LDS tile (dkdv) / keys per LDS tile (dq)
constexpr int BNT = 256;    // threads per workgroup (4 waves)
constexpr int ROWB = 64;    // bytes per staged row (32 x 16-bit)

// byte offset of (row r, 16-byte chunk c) in a [rows][32] 16-bit tile whose chunks are
// XOR-swizzled by (r / 4) % 4: row-major fragment reads of 32 consecutive rows and the
// transposed reads of 4-row groups both hit distinct bank groups.
__device__ __forceinline__ int swz(int r, int c) { return r * ROWB + 16 * (c ^ ((r >> 2) & 3)); }

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V4 tr4(const unsigned char* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(__attribute__((address_space(3))) const unsigned char*)p);
  return __builtin_bit_cast(typename TypeOps<T>::V4, v);
}

// Transposed B fragment from a swizzled [row][32] tile: k = rows (in the 32x32 accumulator's
// row order: element e of k-step kk is row 16 kk + 8 (e / 4) + 4 g + e % 4 of the 32-row
// block at row0), n = column l % 32.
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 tr_frag(const unsigned char* tile, int row0, int kk, int lane) {
  const int g = lane >> 5, r16 = lane & 15;
  const int col = 16 * ((lane >> 4) & 1) + 4 * (r16 & 3);  // element column of this lane's 4
  typename TypeOps<T>::V8 f;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int row = row0 + 16 * kk + 8 * hh + 4 * g + (r16 >> 2);
    const unsigned char* p = tile + swz(row, col >> 3) + 2 * (col & 7);
    const typename TypeOps<T>::V4 x = tr4<T>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) f[4 * hh + e] = x[e];
  }
  return f;
}

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 lds_row8(const unsigned char* tile, int row, int chunk) {
  return *reinterpret_cast<const typename TypeOps<T>::V8*>(tile + swz(row, chunk));
}

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 acc_to_frag(const f32x16& a, int kk) {
  f32x8 x = {a[8 * kk + 0], a[8 * kk + 1], a[8 * kk + 2], a[8 * kk + 3],
             a[8 * kk + 4], a[8 * kk + 5], a[8 * kk + 6], a[8 * kk + 7]};
  return TypeOps<T>::from_f32(x);
}

// identity A / B fragments: element e of lane group g in k-step t is index 16 t + 8 g + e;
// the lane's row / column l32 holds a 1 there iff it equals that index.
template <typename T>
__device__ __forceinline__ void identity_frags(typename TypeOps<T>::V8 (&idf)[2], int l32, int g) {
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) idf[t][e] = TypeOps<T>::from_f32(l32 == 16 * t + 8 * g + e ? 1.f : 0.f);
}

// 8 elements of a [*, D] row starting at column d0 (zeros past D or for an absent row)
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 row8(const T* row, int d0, int D, bool ok) {
  return (ok && d0 < D) ? load8(row + d0) : zero8<T>();
}

// ------------------------------------------------------------------------- Delta
template <typename T>
__global__ __launch_bounds__(BNT) void bwd_delta_kernel(const gnn_triattn_bwd_args a) {
  const int64_t rows = a.B * a.S * a.N * a.H;
  const int64_t r = (int64_t)blockIdx.x * BNT + threadIdx.x;
  if (r >= rows) return;
  // r enumerates [B, S, H, N] (the lse / Delta layout)
  const int64_t n = r % a.N, h = (r / a.N) % a.H, s = (r / (a.N * a.H)) % a.S, b = r / (a.N * a.H * a.S);
  const T* o = (const T*)a.o + b * a.o_stride[0] + s * a.o_stride[1] + n * a.o_stride[2] + h * a.o_stride[3];
  const T* d = (const T*)a.dout + b * a.do_stride[0] + s * a.do_stride[1] + n * a.do_stride[2] + h * a.do_stride[3];
  float acc = 0.f;
  for (int c = 0; c < a.D; c += 8) {
    const f32x8 x = TypeOps<T>::to_f32(load8(o + c)), y = TypeOps<T>::to_f32(load8(d + c));
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(x[e], y[e], acc);
  }
  a.delta[r] = acc;
}

// ------------------------------------------------------------------------- dK, dV
// LDS: Q' tile and dO tile [64][32] (swizzled), lse and Delta of the tile's queries.
struct DkdvLds {
  unsigned char q[BT * ROWB];
  unsigned char d[BT * ROWB];
  float lse[BT];
  float delta[BT];
};

template <typename T, bool HAS_BIAS>
__global__ __launch_bounds__(BNT, 2) void bwd_dkdv_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  __shared__ __align__(16) DkdvLds sm;
  const int N = (int)a.N, H = (int)a.H, D = (int)a.D;
  const int nkb = (N + 127) / 128;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int kb = w % nkb;
  const int h = (w / nkb) % H;
  const int64_t bs = w / ((uint32_t)nkb * H);
  const int s = (int)(bs % a.S), b = (int)(bs / a.S);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int key = kb * 128 + wave * 32 + l32;
  const bool kok = key < N;

  const int64_t rowoff[4] = {(int64_t)b * a.q_stride[0] + (int64_t)s * a.q_stride[1] + (int64_t)h * a.q_stride[3],
                             (int64_t)b * a.k_stride[0] + (int64_t)s * a.k_stride[1] + (int64_t)h * a.k_stride[3],
                             (int64_t)b * a.v_stride[0] + (int64_t)s * a.v_stride[1] + (int64_t)h * a.v_stride[3],
                             (int64_t)b * a.do_stride[0] + (int64_t)s * a.do_stride[1] + (int64_t)h * a.do_stride[3]};
  const T* qp = (const T*)a.q + rowoff[0];
  const T* dop = (const T*)a.dout + rowoff[3];
  // this lane's key: K and V as B operands (lane = key, 8 consecutive d per lane group)
  V8 kf[2], vf[2];
  {
    const T* kr = (const T*)a.k + rowoff[1] + (int64_t)(kok ? key : 0) * a.k_stride[2];
    const T* vr = (const T*)a.v + rowoff[2] + (int64_t)(kok ? key : 0) * a.v_stride[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      kf[kk] = row8(kr, 16 * kk + 8 * g, D, kok);
      vf[kk] = row8(vr, 16 * kk + 8 * g, D, kok);
    }
  }
  // key-side mask term: the sentinel for masked keys, -inf for keys past N (p = 0)
  float kbias = 0.f;
  if (!kok) {
    kbias = -INFINITY;
  } else if (a.mask && a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)key * a.mask_stride[2]] == 0) {
    kbias = a.mask_value;
  }
  V8 idf[2];
  identity_frags<T>(idf, l32, g);
  const T* bias_plane = HAS_BIAS ? (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] : nullptr;
  const float* lse_row = a.lse + (((int64_t)b * a.S + s) * H + h) * N;
  const float* delta_row = a.delta + (((int64_t)b * a.S + s) * H + h) * N;

  f32x16 dk, dv;
#pragma unroll
  for (int i = 0; i < 16; ++i) dk[i] = dv[i] = 0.f;

  const int ntq = (N + BT - 1) / BT;
  for (int tq = 0; tq < ntq; ++tq) {
    const int q0 = tq * BT;
    __syncthreads();  // the previous tile's reads are done
    // stage Q' = bf16(q * scale) and dO of 64 queries (256 threads: 64 rows x 4 chunks)
    {
      const int r = tid >> 2, c = tid & 3;
      const int qi = q0 + r;
      const bool ok = qi < N;
      V8 x = row8(qp + (int64_t)(ok ? qi : 0) * a.q_stride[2], 8 * c, D, ok);
      const f32x8 xf = TypeOps<T>::to_f32(x) * a.scale;
      *reinterpret_cast<V8*>(sm.q + swz(r, c)) = TypeOps<T>::from_f32(xf);
      *reinterpret_cast<V8*>(sm.d + swz(r, c)) = row8(dop + (int64_t)(ok ? qi : 0) * a.do_stride[2], 8 * c, D, ok);
      if (tid < BT) {
        const int qq = q0 + tid;
        // absent queries: lse = +inf makes their P exactly 0 (their dO is 0 too)
        sm.lse[tid] = qq < N ? lse_row[qq] : INFINITY;
        sm.delta[tid] = qq < N ? delta_row[qq] : 0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int r0 = sub * 32;
      // S[q][key] = Q' K^T (+ bias): rows = queries r0 + 8 (i / 4) + 4 g + i % 4, column = key
      f32x16 sc, dp;
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] = dp[i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        Mma<T, PREC_NATIVE>::step(sc, lds_row8<T>(sm.q, r0 + l32, 2 * kk + g), kf[kk]);
        Mma<T, PREC_NATIVE>::step(dp, lds_row8<T>(sm.d, r0 + l32, 2 * kk + g), vf[kk]);
      }
      if constexpr (HAS_BIAS) {
        // A = bias rows (lane = query, 8 consecutive keys of the wave's 32), B = identity
        const int qi = q0 + r0 + l32;
        const T* brow = bias_plane + (int64_t)(qi < N ? qi : 0) * a.bias_stride[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int k0 = kb * 128 + wave * 32 + 16 * t + 8 * g;
          const V8 bfr = qi < N ? load8_bias_tail<T>(brow, k0, N) : zero8<T>();
          Mma<T, PREC_NATIVE>::step(sc, bfr, idf[t]);
        }
      }
      // P and dS for this lane's key and its 16 queries
      f32x16 p, ds;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(&sm.lse[r0 + 8 * rg + 4 * g]);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sm.delta[r0 + 8 * rg + 4 * g]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * rg + e;
          const float x = sc[i] + kbias;
          const float pv = fast_exp2((x - l4[e]) * LOG2E_B);
          p[i] = pv;
          ds[i] = pv * (dp[i] - d4[e]);
        }
      }
      // dV += P^T dO and dK += dS^T Q': A = the accumulators (lane = key, k = queries),
      // B = the staged tiles read transposed (k = queries, n = d)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        Mma<T, PREC_NATIVE>::step(dv, acc_to_frag<T>(p, kk), tr_frag<T>(sm.d, r0, kk, lane));
        Mma<T, PREC_NATIVE>::step(dk, acc_to_frag<T>(ds, kk), tr_frag<T>(sm.q, r0, kk, lane));
      }
    }
  }
  // dk / dv[m = key][n = d]: lane = d (l32), rows = keys wave*32 + 8 (i / 4) + 4 g + i % 4
  const int d = l32;
  if (d < D) {
    T* dkp = (T*)a.dk + b * a.dk_stride[0] + s * a.dk_stride[1] + h * a.dk_stride[3] + d;
    T* dvp = (T*)a.dv + b * a.dv_stride[0] + s * a.dv_stride[1] + h * a.dv_stride[3] + d;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kj = kb * 128 + wave * 32 + 8 * (i / 4) + 4 * g + (i % 4);
      if (kj < N) {
        dkp[(int64_t)kj * a.dk_stride[2]] = TypeOps<T>::from_f32(dk[i]);
        dvp[(int64_t)kj * a.dv_stride[2]] = TypeOps<T>::from_f32(dv[i]);
      }
    }
  }
}

// ------------------------------------------------------------------------- dQ
struct DqLds {
  unsigned char k[BT * ROWB];
  unsigned char v[BT * ROWB];
};

template <typename T, bool HAS_BIAS>
__global__ __launch_bounds__(BNT, 2) void bwd_dq_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  __shared__ __align__(16) DqLds sm;
  const int N = (int)a.N, H = (int)a.H, D = (int)a.D;
  const int nqb = (N + 127) / 128;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int qb = w % nqb;
  const int h = (w / nqb) % H;
  const int64_t bs = w / ((uint32_t)nqb * H);
  const int s = (int)(bs % a.S), b = (int)(bs / a.S);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int qi = qb * 128 + wave * 32 + l32;
  const bool qok = qi < N;

  const T* kp = (const T*)a.k + b * a.k_stride[0] + s * a.k_stride[1] + h * a.k_stride[3];
  const T* vp = (const T*)a.v + b * a.v_stride[0] + s * a.v_stride[1] + h * a.v_stride[3];
  // this lane's query: Q' and dO as B operands (lane = query, 8 consecutive d)
  V8 qf[2], dof[2];
  {
    const T* qr = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3] +
                  (int64_t)(qok ? qi : 0) * a.q_stride[2];
    const T* dr = (const T*)a.dout + b * a.do_stride[0] + s * a.do_stride[1] + h * a.do_stride[3] +
                  (int64_t)(qok ? qi : 0) * a.do_stride[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      qf[kk] = TypeOps<T>::from_f32(TypeOps<T>::to_f32(row8(qr, 16 * kk + 8 * g, D, qok)) * a.scale);
      dof[kk] = row8(dr, 16 * kk + 8 * g, D, qok);
    }
  }
  const int64_t lrow = (((int64_t)b * a.S + s) * H + h) * N;
  const float lse = qok ? a.lse[lrow + qi] : INFINITY;  // absent queries: p = 0
  const float delta = qok ? a.delta[lrow + qi] : 0.f;
  const float nl = -lse * LOG2E_B;
  V8 idf[2];
  identity_frags<T>(idf, l32, g);
  const T* brow = HAS_BIAS ? (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] +
                                 (int64_t)(qok ? qi : 0) * a.bias_stride[2]
                           : nullptr;
  f32x16 dq;
#pragma unroll
  for (int i = 0; i < 16; ++i) dq[i] = 0.f;

  const int ntk = (N + BT - 1) / BT;
  for (int tk = 0; tk < ntk; ++tk) {
    const int k0 = tk * BT;
    __syncthreads();
    {
      const int r = tid >> 2, c = tid & 3;
      const int kj = k0 + r;
      const bool ok = kj < N;
      *reinterpret_cast<V8*>(sm.k + swz(r, c)) = row8(kp + (int64_t)(ok ? kj : 0) * a.k_stride[2], 8 * c, D, ok);
      *reinterpret_cast<V8*>(sm.v + swz(r, c)) = row8(vp + (int64_t)(ok ? kj : 0) * a.v_stride[2], 8 * c, D, ok);
    }
    __syncthreads();
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int r0 = sub * 32;
      // S^T[key][q] = K Q'^T (+ bias), dP^T[key][q] = V dO^T: rows = keys r0 + 8 (i / 4) + 4 g + i % 4
      f32x16 sc, dp;
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] = dp[i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        Mma<T, PREC_NATIVE>::step(sc, lds_row8<T>(sm.k, r0 + l32, 2 * kk + g), qf[kk]);
        Mma<T, PREC_NATIVE>::step(dp, lds_row8<T>(sm.v, r0 + l32, 2 * kk + g), dof[kk]);
      }
      if constexpr (HAS_BIAS) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const V8 bfr = qok ? load8_bias_tail<T>(brow, k0 + r0 + 16 * t + 8 * g, N) : zero8<T>();
          Mma<T, PREC_NATIVE>::step(sc, idf[t], bfr);
        }
      }
      f32x16 ds;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kj = k0 + r0 + 8 * (i / 4) + 4 * g + (i % 4);
        float x = sc[i];
        if (kj >= N) {
          x = -INFINITY;
        } else if (a.mask && a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)kj * a.mask_stride[2]] == 0) {
          x += a.mask_value;
        }
        const float pv = fast_exp2(__builtin_fmaf(x, LOG2E_B, nl));
        ds[i] = pv * (dp[i] - delta);
      }
      // dQ += dS K: A = dS^T accumulator (lane = query, k = keys), B = K read transposed
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        Mma<T, PREC_NATIVE>::step(dq, acc_to_frag<T>(ds, kk), tr_frag<T>(sm.k, r0, kk, lane));
    }
  }
  // dq[m = query][n = d]: lane = d, rows = queries wave*32 + 8 (i / 4) + 4 g + i % 4
  const int d = l32;
  if (d < D) {
    T* dqp = (T*)a.dq + b * a.dq_stride[0] + s * a.dq_stride[1] + h * a.dq_stride[3] + d;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int qq = qb * 128 + wave * 32 + 8 * (i / 4) + 4 * g + (i % 4);
      if (qq < N) dqp[(int64_t)qq * a.dq_stride[2]] = TypeOps<T>::from_f32(dq[i] * a.scale);
    }
  }
}

// ------------------------------------------------------------------------- dbias
// One wave per (b, h, 32 queries, 64 keys); S and dP as [query][key] (lane = key).
template <typename T>
__global__ __launch_bounds__(BNT, 2) void bwd_dbias_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  const int N = (int)a.N, H = (int)a.H, D = (int)a.D;
  const int nqt = (N + 31) / 32, nkt = (N + 63) / 64;
  const int64_t tiles = (int64_t)a.B * H * nqt * nkt;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int64_t t = (int64_t)xcd_remap(blockIdx.x, gridDim.x) * 4 + wave;
  if (t >= tiles) return;  // whole wave
  const int kt = (int)(t % nkt);
  const int qt = (int)((t / nkt) % nqt);
  const int h = (int)((t / ((int64_t)nkt * nqt)) % H);
  const int b = (int)(t / ((int64_t)nkt * nqt * H));
  const int q0 = qt * 32;
  // this lane's keys: kcol[sub] = k0 + 32 sub + l32
  int kcol[2];
  bool kok[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    kcol[sub] = kt * 64 + 32 * sub + l32;
    kok[sub] = kcol[sub] < N;
  }
  // the bias tile as the scores' initial value: element i = query q0 + 8 (i / 4) + 4 g + i % 4
  f32x16 binit[2];
  const T* bias_plane = (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int qq = q0 + 8 * (i / 4) + 4 * g + (i % 4);
      binit[sub][i] = (qq < N && kok[sub]) ? TypeOps<T>::to_f32(bias_plane[(int64_t)qq * a.bias_stride[2] + kcol[sub]]) : 0.f;
    }
  f32x16 acc[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[sub][i] = 0.f;

  const int qa = q0 + l32;  // this lane's query row for the A operands
  const bool qaok = qa < N;
  for (int s = 0; s < a.S; ++s) {
    const T* qr = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3] + (int64_t)(qaok ? qa : 0) * a.q_stride[2];
    const T* dr = (const T*)a.dout + b * a.do_stride[0] + s * a.do_stride[1] + h * a.do_stride[3] + (int64_t)(qaok ? qa : 0) * a.do_stride[2];
    V8 qf[2], dof[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      qf[kk] = TypeOps<T>::from_f32(TypeOps<T>::to_f32(row8(qr, 16 * kk + 8 * g, D, qaok)) * a.scale);
      dof[kk] = row8(dr, 16 * kk + 8 * g, D, qaok);
    }
    const int64_t lrow = (((int64_t)b * a.S + s) * H + h) * N;
    f32x4 l4[4], d4[4];
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int qq = q0 + 8 * rg + 4 * g;
      if (qq + 4 <= N) {
        l4[rg] = *reinterpret_cast<const f32x4*>(a.lse + lrow + qq);
        d4[rg] = *reinterpret_cast<const f32x4*>(a.delta + lrow + qq);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          l4[rg][e] = qq + e < N ? a.lse[lrow + qq + e] : INFINITY;
          d4[rg][e] = qq + e < N ? a.delta[lrow + qq + e] : 0.f;
        }
      }
    }
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const T* kr = (const T*)a.k + b * a.k_stride[0] + s * a.k_stride[1] + h * a.k_stride[3] + (int64_t)(kok[sub] ? kcol[sub] : 0) * a.k_stride[2];
      const T* vr = (const T*)a.v + b * a.v_stride[0] + s * a.v_stride[1] + h * a.v_stride[3] + (int64_t)(kok[sub] ? kcol[sub] : 0) * a.v_stride[2];
      f32x16 sc = binit[sub], dp;
#pragma unroll
      for (int i = 0; i < 16; ++i) dp[i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        Mma<T, PREC_NATIVE>::step(sc, qf[kk], row8(kr, 16 * kk + 8 * g, D, kok[sub]));
        Mma<T, PREC_NATIVE>::step(dp, dof[kk], row8(vr, 16 * kk + 8 * g, D, kok[sub]));
      }
      float kb = 0.f;
      if (!kok[sub]) {
        kb = -INFINITY;
      } else if (a.mask && a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)kcol[sub] * a.mask_stride[2]] == 0) {
        kb = a.mask_value;
      }
#pragma unroll
      for (int rg = 0; rg < 4; ++rg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * rg + e;
          const float pv = fast_exp2((sc[i] + kb - l4[rg][e]) * LOG2E_B);
          acc[sub][i] += pv * (dp[i] - d4[rg][e]);
        }
    }
  }
  // dbias[b, h, q, k] fp32 [B, H, N, N] contiguous
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    if (!kok[sub]) continue;
    float* out = a.dbias + ((int64_t)b * H + h) * N * N + kcol[sub];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int qq = q0 + 8 * (i / 4) + 4 * g + (i % 4);
      if (qq < N) out[(int64_t)qq * N] = acc[sub][i];
    }
  }
}

template <typename T>
int launch_bwd(const gnn_triattn_bwd_args& a, hipStream_t stream) {
  const int64_t rows = a.B * a.S * a.N * a.H;
  hipLaunchKernelGGL(bwd_delta_kernel<T>, dim3((uint32_t)((rows + BNT - 1) / BNT)), dim3(BNT), 0, stream, a);
  const int64_t nb128 = (a.N + 127) / 128;
  const dim3 grid((uint32_t)(nb128 * a.H * a.S * a.B));
  if (a.bias) {
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, true>), grid, dim3(BNT), 0, stream, a);
    hipLaunchKernelGGL((bwd_dq_kernel<T, true>), grid, dim3(BNT), 0, stream, a);
  } else {
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, false>), grid, dim3(BNT), 0, stream, a);
    hipLaunchKernelGGL((bwd_dq_kernel<T, false>), grid, dim3(BNT), 0, stream, a);
  }
  if (a.bias && a.dbias) {
    const int64_t tiles = a.B * a.H * ((a.N + 31) / 32) * ((a.N + 63) / 64);
    hipLaunchKernelGGL(bwd_dbias_kernel<T>, dim3((uint32_t)((tiles + 3) / 4)), dim3(BNT), 0, stream, a);
  }
  return (int)hipGetLastError();
}

}  // namespace

int triattn_bwd(const gnn_triattn_bwd_args& a, hipStream_t stream) {
  if (a.D > 32)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention backward: head dim > 32 is not supported");
  if (a.B * a.S * a.H * ((a.N + 127) / 128) >= ((int64_t)1 << 31))
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention backward: grid too large");
  switch (a.dtype) {
    case GNN_BF16: return launch_bwd<bf16>(a, stream);
    case GNN_F16: return launch_bwd<f16>(a, stream);
  }
  return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention backward: bf16 / fp16 only");
}

}  // namespace gnn
