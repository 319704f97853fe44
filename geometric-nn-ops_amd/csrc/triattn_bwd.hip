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
// Three kernels (plus an ordered reduction of the dbias splits), every sum owned by one
// workgroup (no atomics, deterministic):
//   bwd_dkdv   one wave per 32 keys of a (b, s, h) row, looping over 64-query tiles staged
//              in LDS. Scores are computed as S = Q' K^T with the KEYS on the lanes, so the
//              P and dS accumulators already are the A operands of dV += P^T dO and
//              dK += dS^T Q'; the B operands (dO and Q' with queries as k) come from the
//              LDS tiles through ds_read_b64_tr_b16, in the accumulator's row order.
//   bwd_dq     the forward's layout (queries on the lanes, K / V tiles in LDS): the dS^T
//              accumulator is the A operand of dQ += dS K, with K read transposed from LDS.
//              It runs first and also writes Delta = rowsum(dO * O) (fp32) for the others.
//   bwd_dbias  a 128 x 128 tile of a (b, h) bias plane per workgroup, sweeping a range of
//              N_seq rows with the row's operands staged in LDS and sum_s dS accumulating in
//              fp32 registers; the bias tile is loaded once as the scores' initial value.
// The bias is added to the scores in fp32 exactly as in the forward (bf16 values, fp32
// sums), and the mask sentinel after it, so P matches the forward's normaliser. P of a
// masked key is divided by N_res, as the reference's backward does
// (triangle_attention.py:753-766, :1033-1038): in a row whose keys are all masked the
// forward's lse holds the bare sentinel (its log(l) term is below the fp32 ulp there), so
// exp(S - lse) is 1 for every key where softmax gives 1 / N_res; in any other row a masked
// key's P is 0 either way. dq and dk / dv divide per masked key; bwd_dbias, which sees a
// row's keys one tile at a time, per row (its lse at the sentinel): -log2(N_res) joins the
// exp2 argument.
// 16-bit inputs, head dim <= 128 (a multiple of 8, ensured by the host). Every kernel is
// templated on DC, the number of 32-column chunks of the head dim (1, 2 or 4): the staged
// tiles are DC swizzled [rows][32] tiles, the score and dP products sum over the chunks, and
// dQ / dK / dV keep one 32 x 32 accumulator per chunk (columns past D are zeros on input and
// not stored).
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

// ------------------------------------------------------------------------- dK, dV
// LDS: Q' tile and dO tile [64][32] (swizzled), lse and Delta of the tile's queries.
template <int DC>
struct DkdvLds {
  unsigned char q[DC][BT * ROWB];
  unsigned char d[DC][BT * ROWB];
  float lse[BT];
  float delta[BT];
};

template <typename T, bool HAS_BIAS, int DC>
__global__ __launch_bounds__(BNT, DC > 2 ? 1 : 2) void bwd_dkdv_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  __shared__ __align__(16) DkdvLds<DC> sm;
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
  V8 kf[DC][2], vf[DC][2];
  {
    const T* kr = (const T*)a.k + rowoff[1] + (int64_t)(kok ? key : 0) * a.k_stride[2];
    const T* vr = (const T*)a.v + rowoff[2] + (int64_t)(kok ? key : 0) * a.v_stride[2];
#pragma unroll
    for (int dc = 0; dc < DC; ++dc)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        kf[dc][kk] = row8(kr, 32 * dc + 16 * kk + 8 * g, D, kok);
        vf[dc][kk] = row8(vr, 32 * dc + 16 * kk + 8 * g, D, kok);
      }
  }
  // key-side mask term: the sentinel for masked keys, -inf for keys past N (p = 0)
  float kbias = 0.f, kmul = 1.f;
  if (!kok) {
    kbias = -INFINITY;
  } else if (a.mask && a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)key * a.mask_stride[2]] == 0) {
    kbias = a.mask_value;
    kmul = 1.0f / (float)N;  // masked key: P / N_res
  }
  const bool any_masked = __any(kmul != 1.f);
  V8 idf[2];
  identity_frags<T>(idf, l32, g);
  const T* bias_plane = HAS_BIAS ? (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] : nullptr;
  const float* lse_row = a.lse + (((int64_t)b * a.S + s) * H + h) * N;
  const float* delta_row = a.delta + (((int64_t)b * a.S + s) * H + h) * N;

  f32x16 dk[DC], dv[DC];
#pragma unroll
  for (int dc = 0; dc < DC; ++dc)
#pragma unroll
    for (int i = 0; i < 16; ++i) dk[dc][i] = dv[dc][i] = 0.f;

  const int ntq = (N + BT - 1) / BT;
  for (int tq = 0; tq < ntq; ++tq) {
    const int q0 = tq * BT;
    __syncthreads();  // the previous tile's reads are done
    // stage Q' = bf16(q * scale) and dO of 64 queries (256 threads: 64 rows x 4 chunks)
    {
      const int r = tid >> 2, c = tid & 3;
      const int qi = q0 + r;
      const bool ok = qi < N;
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        V8 x = row8(qp + (int64_t)(ok ? qi : 0) * a.q_stride[2], 32 * dc + 8 * c, D, ok);
        const f32x8 xf = TypeOps<T>::to_f32(x) * a.scale;
        *reinterpret_cast<V8*>(sm.q[dc] + swz(r, c)) = TypeOps<T>::from_f32(xf);
        *reinterpret_cast<V8*>(sm.d[dc] + swz(r, c)) =
            row8(dop + (int64_t)(ok ? qi : 0) * a.do_stride[2], 32 * dc + 8 * c, D, ok);
      }
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
      for (int dc = 0; dc < DC; ++dc)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          Mma<T, PREC_NATIVE>::step(sc, lds_row8<T>(sm.q[dc], r0 + l32, 2 * kk + g), kf[dc][kk]);
          Mma<T, PREC_NATIVE>::step(dp, lds_row8<T>(sm.d[dc], r0 + l32, 2 * kk + g), vf[dc][kk]);
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
          float pv = fast_exp2((x - l4[e]) * LOG2E_B);
          if (any_masked) pv *= kmul;
          p[i] = pv;
          ds[i] = pv * (dp[i] - d4[e]);
        }
      }
      // dV += P^T dO and dK += dS^T Q': A = the accumulators (lane = key, k = queries),
      // B = the staged tiles read transposed (k = queries, n = d)
#pragma unroll
      for (int dc = 0; dc < DC; ++dc)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          Mma<T, PREC_NATIVE>::step(dv[dc], acc_to_frag<T>(p, kk), tr_frag<T>(sm.d[dc], r0, kk, lane));
          Mma<T, PREC_NATIVE>::step(dk[dc], acc_to_frag<T>(ds, kk), tr_frag<T>(sm.q[dc], r0, kk, lane));
        }
    }
  }
  // dk / dv[m = key][n = d]: lane = d (32 dc + l32), rows = keys wave*32 + 8 (i / 4) + 4 g + i % 4
#pragma unroll
  for (int dc = 0; dc < DC; ++dc) {
    const int d = 32 * dc + l32;
    if (d < D) {
      T* dkp = (T*)a.dk + b * a.dk_stride[0] + s * a.dk_stride[1] + h * a.dk_stride[3] + d;
      T* dvp = (T*)a.dv + b * a.dv_stride[0] + s * a.dv_stride[1] + h * a.dv_stride[3] + d;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kj = kb * 128 + wave * 32 + 8 * (i / 4) + 4 * g + (i % 4);
        if (kj < N) {
          dkp[(int64_t)kj * a.dk_stride[2]] = TypeOps<T>::from_f32(dk[dc][i]);
          dvp[(int64_t)kj * a.dv_stride[2]] = TypeOps<T>::from_f32(dv[dc][i]);
        }
      }
    }
  }
}

// ------------------------------------------------------------------------- dQ
template <int DC>
struct DqLds {
  unsigned char k[DC][BT * ROWB];
  unsigned char v[DC][BT * ROWB];
};

template <typename T, bool HAS_BIAS, int DC>
__global__ __launch_bounds__(BNT, DC > 2 ? 1 : 2) void bwd_dq_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  __shared__ __align__(16) DqLds<DC> sm;
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
  V8 qf[DC][2], dof[DC][2];
  {
    const T* qr = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3] +
                  (int64_t)(qok ? qi : 0) * a.q_stride[2];
    const T* dr = (const T*)a.dout + b * a.do_stride[0] + s * a.do_stride[1] + h * a.do_stride[3] +
                  (int64_t)(qok ? qi : 0) * a.do_stride[2];
#pragma unroll
    for (int dc = 0; dc < DC; ++dc)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int d0 = 32 * dc + 16 * kk + 8 * g;
        qf[dc][kk] = TypeOps<T>::from_f32(TypeOps<T>::to_f32(row8(qr, d0, D, qok)) * a.scale);
        dof[dc][kk] = row8(dr, d0, D, qok);
      }
  }
  const int64_t lrow = (((int64_t)b * a.S + s) * H + h) * N;
  const float lse = qok ? a.lse[lrow + qi] : INFINITY;  // absent queries: p = 0
  // Delta = dO . O of this query: the lane pair (g = 0, 1) holds the 32 columns between them
  float delta;
  {
    const T* orow = (const T*)a.o + b * a.o_stride[0] + s * a.o_stride[1] + h * a.o_stride[3] +
                    (int64_t)(qok ? qi : 0) * a.o_stride[2];
    float part = 0.f;
#pragma unroll
    for (int dc = 0; dc < DC; ++dc)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const f32x8 x = TypeOps<T>::to_f32(row8(orow, 32 * dc + 16 * kk + 8 * g, D, qok));
        const f32x8 y = TypeOps<T>::to_f32(dof[dc][kk]);
#pragma unroll
        for (int e = 0; e < 8; ++e) part = __builtin_fmaf(x[e], y[e], part);
      }
    delta = part + __shfl_xor(part, 32);
    if (qok && g == 0) a.delta[lrow + qi] = delta;
  }
  V8 idf[2];
  identity_frags<T>(idf, l32, g);
  const T* brow = HAS_BIAS ? (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] +
                                 (int64_t)(qok ? qi : 0) * a.bias_stride[2]
                           : nullptr;
  f32x16 dq[DC];
#pragma unroll
  for (int dc = 0; dc < DC; ++dc)
#pragma unroll
    for (int i = 0; i < 16; ++i) dq[dc][i] = 0.f;

  const int ntk = (N + BT - 1) / BT;
  for (int tk = 0; tk < ntk; ++tk) {
    const int k0 = tk * BT;
    __syncthreads();
    {
      const int r = tid >> 2, c = tid & 3;
      const int kj = k0 + r;
      const bool ok = kj < N;
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        *reinterpret_cast<V8*>(sm.k[dc] + swz(r, c)) =
            row8(kp + (int64_t)(ok ? kj : 0) * a.k_stride[2], 32 * dc + 8 * c, D, ok);
        *reinterpret_cast<V8*>(sm.v[dc] + swz(r, c)) =
            row8(vp + (int64_t)(ok ? kj : 0) * a.v_stride[2], 32 * dc + 8 * c, D, ok);
      }
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
      for (int dc = 0; dc < DC; ++dc)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          Mma<T, PREC_NATIVE>::step(sc, lds_row8<T>(sm.k[dc], r0 + l32, 2 * kk + g), qf[dc][kk]);
          Mma<T, PREC_NATIVE>::step(dp, lds_row8<T>(sm.v[dc], r0 + l32, 2 * kk + g), dof[dc][kk]);
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
        float x = sc[i], pm = 1.f;
        if (kj >= N) {
          x = -INFINITY;
        } else if (a.mask && a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)kj * a.mask_stride[2]] == 0) {
          x += a.mask_value;
          pm = 1.0f / (float)N;  // masked key: P / N_res
        }
        // subtract first: in a row whose keys are all masked both x and lse sit near the
        // sentinel, and only their difference is exact
        const float pv = fast_exp2((x - lse) * LOG2E_B) * pm;
        ds[i] = pv * (dp[i] - delta);
      }
      // dQ += dS K: A = dS^T accumulator (lane = query, k = keys), B = K read transposed
#pragma unroll
      for (int dc = 0; dc < DC; ++dc)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          Mma<T, PREC_NATIVE>::step(dq[dc], acc_to_frag<T>(ds, kk), tr_frag<T>(sm.k[dc], r0, kk, lane));
    }
  }
  // dq[m = query][n = d]: lane = d (32 dc + l32), rows = queries wave*32 + 8 (i / 4) + 4 g + i % 4
#pragma unroll
  for (int dc = 0; dc < DC; ++dc) {
    const int d = 32 * dc + l32;
    if (d < D) {
      T* dqp = (T*)a.dq + b * a.dq_stride[0] + s * a.dq_stride[1] + h * a.dq_stride[3] + d;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qq = qb * 128 + wave * 32 + 8 * (i / 4) + 4 * g + (i % 4);
        if (qq < N) dqp[(int64_t)qq * a.dq_stride[2]] = TypeOps<T>::from_f32(dq[dc][i] * a.scale);
      }
    }
  }
}

// ------------------------------------------------------------------------- dbias
// Eight waves per workgroup own a 128-query x 128-key tile of one (b, h) bias plane; wave w
// takes queries 32 (w % 4) .. + 31 and keys 64 (w / 4) .. + 63 (two 32-key halves), scores
// laid out [query][key] with the keys on the lanes. The workgroup sweeps N_seq rows
// [s_begin, s_end): per row, Q' / dO / K / V of the tile, lse / Delta of its queries and the
// key-mask term of its keys are staged in LDS (the next row's loads are in flight while the
// current one is computed), and sum_s dS accumulates in fp32 registers. With more than one
// N_seq split the partial sums go to the workspace and bwd_dbias_reduce adds them in order.
// Measured without gain at N = 512 (350 us): sixteen waves of 32 x 32 (128 VGPRs, the bias
// tile in LDS; 405 us) and a 128 x 64 tile with two workgroups per CU (384 us).
constexpr int DB_T = 128;
constexpr int DB_NT = 512;
template <int DC>
struct DbLds {  // DC > 1 exceeds 64 KB: dynamic LDS
  unsigned char q[DC][DB_T * ROWB];
  unsigned char d[DC][DB_T * ROWB];
  unsigned char k[DC][DB_T * ROWB];
  unsigned char v[DC][DB_T * ROWB];
  float lse[DB_T];
  float delta[DB_T];
  float kb[DB_T];
  float pl2;  // -log2(N_res) when the row's keys are all masked, else 0
};

template <typename T, int DC>
__global__ __launch_bounds__(DB_NT, 1) void bwd_dbias_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(16) unsigned char db_smem[];
  DbLds<DC>& sm = *reinterpret_cast<DbLds<DC>*>(db_smem);
  const int N = (int)a.N, H = (int)a.H, D = (int)a.D, S = (int)a.S;
  const int nt = (N + DB_T - 1) / DB_T;
  const int splits = a.dbias_splits > 1 ? a.dbias_splits : 1;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  // tiles of a plane fastest, then the N_seq split: the workgroups an XCD runs together are
  // the tiles of one or two splits, which read the same N_seq rows (each Q' / dO tile is
  // shared by a tile row, each K / V tile by a tile column) from its L2
  const int kt = w % nt;
  const int qt = (w / nt) % nt;
  const int split = (w / (nt * nt)) % splits;
  const int64_t bh = w / ((uint32_t)splits * nt * nt);
  const int h = (int)(bh % H), b = (int)(bh / H);
  const int per = (S + splits - 1) / splits;
  const int s_begin = split * per, s_end = min(S, s_begin + per);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int qw = 32 * (wave & 3), kw = 64 * (wave >> 2);  // wave's rows within the tile
  const int q0 = qt * DB_T, k0 = kt * DB_T;

  // the bias tile as the scores' initial value: element i of half sub is query
  // q0 + qw + 8 (i / 4) + 4 g + i % 4, key k0 + kw + 32 sub + l32
  f32x16 binit[2], acc[2];
  {
    const T* plane = (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int kj = k0 + kw + 32 * sub + l32;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qq = q0 + qw + 8 * (i / 4) + 4 * g + (i % 4);
        binit[sub][i] = (qq < N && kj < N) ? TypeOps<T>::to_f32(plane[(int64_t)qq * a.bias_stride[2] + kj]) : 0.f;
        acc[sub][i] = 0.f;
      }
    }
  }

  // staging: thread = (row r = tid / 4, chunk c = tid % 4) of each of the four tiles
  const int sr = tid >> 2, sc4 = tid & 3;
  V8 pq[DC], pd[DC], pk[DC], pv[DC];
  float plse = 0.f, pdel = 0.f, pkb = 0.f;
  auto load_stage = [&](int s) {
    const int qi = q0 + sr, kj = k0 + sr;
    const bool qok = qi < N, kok = kj < N;
    const int64_t qo = (int64_t)b * a.q_stride[0] + (int64_t)s * a.q_stride[1] + (int64_t)h * a.q_stride[3];
    const int64_t doo = (int64_t)b * a.do_stride[0] + (int64_t)s * a.do_stride[1] + (int64_t)h * a.do_stride[3];
    const int64_t ko = (int64_t)b * a.k_stride[0] + (int64_t)s * a.k_stride[1] + (int64_t)h * a.k_stride[3];
    const int64_t vo = (int64_t)b * a.v_stride[0] + (int64_t)s * a.v_stride[1] + (int64_t)h * a.v_stride[3];
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      const int c0 = 32 * dc + 8 * sc4;
      pq[dc] = row8((const T*)a.q + qo + (int64_t)(qok ? qi : 0) * a.q_stride[2], c0, D, qok);
      pd[dc] = row8((const T*)a.dout + doo + (int64_t)(qok ? qi : 0) * a.do_stride[2], c0, D, qok);
      pk[dc] = row8((const T*)a.k + ko + (int64_t)(kok ? kj : 0) * a.k_stride[2], c0, D, kok);
      pv[dc] = row8((const T*)a.v + vo + (int64_t)(kok ? kj : 0) * a.v_stride[2], c0, D, kok);
    }
    if (sc4 == 0) {
      const int64_t lrow = (((int64_t)b * S + s) * H + h) * N;
      plse = qok ? a.lse[lrow + qi] : INFINITY;  // absent queries: p = 0
      pdel = qok ? a.delta[lrow + qi] : 0.f;
      pkb = !kok ? -INFINITY
                 : ((a.mask && a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)kj * a.mask_stride[2]] == 0)
                        ? a.mask_value
                        : 0.f);
    }
  };
  auto store_stage = [&]() {
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      *reinterpret_cast<V8*>(sm.q[dc] + swz(sr, sc4)) = TypeOps<T>::from_f32(TypeOps<T>::to_f32(pq[dc]) * a.scale);
      *reinterpret_cast<V8*>(sm.d[dc] + swz(sr, sc4)) = pd[dc];
      *reinterpret_cast<V8*>(sm.k[dc] + swz(sr, sc4)) = pk[dc];
      *reinterpret_cast<V8*>(sm.v[dc] + swz(sr, sc4)) = pv[dc];
    }
    if (sc4 == 0) {
      sm.lse[sr] = plse;
      sm.delta[sr] = pdel;
      sm.kb[sr] = pkb;
      // every query of the row shares its keys' mask: the tile's first query (< N) decides
      if (sr == 0) sm.pl2 = (a.mask && plse <= 0.5f * a.mask_value) ? -__log2f((float)N) : 0.f;
    }
  };

  if (s_begin < s_end) {
    load_stage(s_begin);
    store_stage();
  }
  __syncthreads();
  for (int s = s_begin; s < s_end; ++s) {
    const bool has_next = s + 1 < s_end;
    if (has_next) load_stage(s + 1);
    V8 qf[DC][2], dof[DC][2];
#pragma unroll
    for (int dc = 0; dc < DC; ++dc)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        qf[dc][kk] = lds_row8<T>(sm.q[dc], qw + l32, 2 * kk + g);
        dof[dc][kk] = lds_row8<T>(sm.d[dc], qw + l32, 2 * kk + g);
      }
    f32x4 l4[4], d4[4];
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      l4[rg] = *reinterpret_cast<const f32x4*>(&sm.lse[qw + 8 * rg + 4 * g]);
      d4[rg] = *reinterpret_cast<const f32x4*>(&sm.delta[qw + 8 * rg + 4 * g]);
    }
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int kr = kw + 32 * sub + l32;
      f32x16 scv = binit[sub], dp;
#pragma unroll
      for (int i = 0; i < 16; ++i) dp[i] = 0.f;
#pragma unroll
      for (int dc = 0; dc < DC; ++dc)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          Mma<T, PREC_NATIVE>::step(scv, qf[dc][kk], lds_row8<T>(sm.k[dc], kr, 2 * kk + g));
          Mma<T, PREC_NATIVE>::step(dp, dof[dc][kk], lds_row8<T>(sm.v[dc], kr, 2 * kk + g));
        }
      const float kb = sm.kb[kr], pl2 = sm.pl2;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * rg + e;
          const float pv = fast_exp2(__builtin_fmaf(scv[i] + kb - l4[rg][e], LOG2E_B, pl2));
          acc[sub][i] += pv * (dp[i] - d4[rg][e]);
        }
    }
    __syncthreads();
    if (has_next) store_stage();
    __syncthreads();
  }
  // [B, H, N, N] fp32: the final gradient, or this split's slice of the workspace
  float* out = (splits > 1 ? a.dbias_ws + (int64_t)split * a.B * H * N * N : a.dbias) + ((int64_t)b * H + h) * N * N;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int kj = k0 + kw + 32 * sub + l32;
    if (kj >= N) continue;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int qq = q0 + qw + 8 * (i / 4) + 4 * g + (i % 4);
      if (qq < N) out[(int64_t)qq * N + kj] = acc[sub][i];
    }
  }
}

// dbias = sum over the splits of the workspace slices, in split order (deterministic)
__global__ __launch_bounds__(BNT) void bwd_dbias_reduce_kernel(const gnn_triattn_bwd_args a) {
  const int64_t n = a.B * a.H * a.N * a.N;
  for (int64_t i = (int64_t)blockIdx.x * BNT + threadIdx.x; i < n; i += (int64_t)gridDim.x * BNT) {
    float x = 0.f;
    for (int c = 0; c < a.dbias_splits; ++c) x += a.dbias_ws[c * n + i];
    a.dbias[i] = x;
  }
}

template <typename T, int DC>
int launch_bwd(const gnn_triattn_bwd_args& a, hipStream_t stream) {
  const int64_t nb128 = (a.N + 127) / 128;
  const dim3 grid((uint32_t)(nb128 * a.H * a.S * a.B));
  // dq first: it also writes Delta, which dk / dv and dbias read
  if (DC == 1 && triattn_bwd_row_applicable(a)) {
    const int rc = triattn_bwd_row_dq_dkdv(a, stream);
    if (rc != 0) return rc;
  } else if (a.bias) {
    hipLaunchKernelGGL((bwd_dq_kernel<T, true, DC>), grid, dim3(BNT), 0, stream, a);
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, true, DC>), grid, dim3(BNT), 0, stream, a);
  } else {
    hipLaunchKernelGGL((bwd_dq_kernel<T, false, DC>), grid, dim3(BNT), 0, stream, a);
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, false, DC>), grid, dim3(BNT), 0, stream, a);
  }
  if (a.bias && a.dbias) {
    const int64_t nt = (a.N + DB_T - 1) / DB_T;
    const int splits = a.dbias_splits > 1 ? a.dbias_splits : 1;
    const size_t smem = sizeof(DbLds<DC>);
    const void* fn = (const void*)bwd_dbias_kernel<T, DC>;
    if (smem > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    hipLaunchKernelGGL((bwd_dbias_kernel<T, DC>), dim3((uint32_t)(a.B * a.H * nt * nt * splits)), dim3(DB_NT), smem,
                       stream, a);
    if (splits > 1) {
      const int64_t n = a.B * a.H * a.N * a.N;
      const int64_t blocks = std::min<int64_t>((n + BNT - 1) / BNT, 4096);
      hipLaunchKernelGGL(bwd_dbias_reduce_kernel, dim3((uint32_t)blocks), dim3(BNT), 0, stream, a);
    }
  }
  return (int)hipGetLastError();
}

}  // namespace

int triattn_bwd(const gnn_triattn_bwd_args& a, hipStream_t stream) {
  if (a.bias && a.dbias && a.dbias_splits > 1 && !a.dbias_ws)
    return set_error(GNN_ERR_ARG, "triangle_attention backward: dbias_splits > 1 needs dbias_ws");
  if (a.bias && a.dbias && (a.dbias_splits > a.S || a.dbias_splits > 64))
    return set_error(GNN_ERR_ARG, "triangle_attention backward: dbias_splits must be at most N_seq and 64");
  if (a.D > 128 || a.D % 8 != 0)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention backward: head dim must be a multiple of 8 and at most 128");
  if (a.B * a.S * a.H * ((a.N + 127) / 128) >= ((int64_t)1 << 31))
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention backward: grid too large");
  const int dc = a.D <= 32 ? 1 : a.D <= 64 ? 2 : 4;  // 32-column chunks of the head dim
  switch (a.dtype) {
    case GNN_BF16: return dc == 1 ? launch_bwd<bf16, 1>(a, stream) : dc == 2 ? launch_bwd<bf16, 2>(a, stream)
                                                                             : launch_bwd<bf16, 4>(a, stream);
    case GNN_F16: return dc == 1 ? launch_bwd<f16, 1>(a, stream) : dc == 2 ? launch_bwd<f16, 2>(a, stream)
                                                                           : launch_bwd<f16, 4>(a, stream);
  }
  return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention backward: bf16 / fp16 only");
}

}  // namespace gnn
