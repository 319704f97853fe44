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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// byte offset of (row r, 16-byte chunk c) in a [rows][32] 16-bit tile whose chunks are
// XOR-swizzled by (r / 4) % 4: row-major fragment reads of 32 consecutive rows and the
// transposed reads of 4-row groups both hit distinct bank groups.
__device__ __forceinline__ int swz(int r, int c) { return r * ROWB + 16 * (c ^ ((r >> 2) & 3)); }
// The same for a [row][32] tile of T: rows of 32 elements, chunks of 8 elements (16 bytes for
// 16-bit types, as swz; 32 bytes for fp32) XOR-swizzled by (r / 4) % 4.
template <typename T> __host__ __device__ constexpr int rowb() { return 32 * (int)sizeof(T); }
template <typename T>
__device__ __forceinline__ int swzt(int r, int c) { return r * rowb<T>() + 8 * (int)sizeof(T) * (c ^ ((r >> 2) & 3)); }

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

// fp32: the transposed fragment from scalar LDS reads, same element order
template <>
__device__ __forceinline__ f32x8 tr_frag<float>(const unsigned char* tile, int row0, int kk, int lane) {
  const int g = lane >> 5, col = lane & 31;
  f32x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int row = row0 + 16 * kk + 8 * (e >> 2) + 4 * g + (e & 3);
    f[e] = *reinterpret_cast<const float*>(tile + swzt<float>(row, col >> 3) + 4 * (col & 7));
  }
  return f;
}

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 lds_row8(const unsigned char* tile, int row, int chunk) {
  return *reinterpret_cast<const typename TypeOps<T>::V8*>(tile + swzt<T>(row, chunk));
}

// -x of a fragment (a sign flip per element)
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 neg8(const typename TypeOps<T>::V8& x) {
  if constexpr (sizeof(T) == 2) {
    u32x4 u = __builtin_bit_cast(u32x4, x);
    u ^= 0x80008000u;
    return __builtin_bit_cast(typename TypeOps<T>::V8, u);
  } else {
    return -x;
  }
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
template <typename T, int DC>
struct DkdvLds {
  unsigned char q[DC][BT * rowb<T>()];
  unsigned char d[DC][BT * rowb<T>()];
  float lse[BT];
  float delta[BT];
};

template <typename T, bool HAS_BIAS, int DC, int PREC>
__global__ __launch_bounds__(BNT, DC > 2 ? 1 : 2) void bwd_dkdv_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  __shared__ __align__(16) DkdvLds<T, DC> sm;
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
        *reinterpret_cast<V8*>(sm.q[dc] + swzt<T>(r, c)) = TypeOps<T>::from_f32(xf);
        *reinterpret_cast<V8*>(sm.d[dc] + swzt<T>(r, c)) =
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
          Mma<T, PREC>::step(sc, lds_row8<T>(sm.q[dc], r0 + l32, 2 * kk + g), kf[dc][kk]);
          Mma<T, PREC>::step(dp, lds_row8<T>(sm.d[dc], r0 + l32, 2 * kk + g), vf[dc][kk]);
        }
      if constexpr (HAS_BIAS) {
        // A = bias rows (lane = query, 8 consecutive keys of the wave's 32), B = identity
        const int qi = q0 + r0 + l32;
        const T* brow = bias_plane + (int64_t)(qi < N ? qi : 0) * a.bias_stride[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int k0 = kb * 128 + wave * 32 + 16 * t + 8 * g;
          const V8 bfr = qi < N ? load8_bias_tail<T>(brow, k0, N) : zero8<T>();
          Mma<T, PREC>::step(sc, bfr, idf[t]);
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
          Mma<T, PREC>::step(dv[dc], acc_to_frag<T>(p, kk), tr_frag<T>(sm.d[dc], r0, kk, lane));
          Mma<T, PREC>::step(dk[dc], acc_to_frag<T>(ds, kk), tr_frag<T>(sm.q[dc], r0, kk, lane));
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
template <typename T, int DC>
struct DqLds {
  unsigned char k[DC][BT * rowb<T>()];
  unsigned char v[DC][BT * rowb<T>()];
};

template <typename T, bool HAS_BIAS, int DC, int PREC>
__global__ __launch_bounds__(BNT, DC > 2 ? 1 : 2) void bwd_dq_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  __shared__ __align__(16) DqLds<T, DC> sm;
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
        *reinterpret_cast<V8*>(sm.k[dc] + swzt<T>(r, c)) =
            row8(kp + (int64_t)(ok ? kj : 0) * a.k_stride[2], 32 * dc + 8 * c, D, ok);
        *reinterpret_cast<V8*>(sm.v[dc] + swzt<T>(r, c)) =
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
          Mma<T, PREC>::step(sc, lds_row8<T>(sm.k[dc], r0 + l32, 2 * kk + g), qf[dc][kk]);
          Mma<T, PREC>::step(dp, lds_row8<T>(sm.v[dc], r0 + l32, 2 * kk + g), dof[dc][kk]);
        }
      if constexpr (HAS_BIAS) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const V8 bfr = qok ? load8_bias_tail<T>(brow, k0 + r0 + 16 * t + 8 * g, N) : zero8<T>();
          Mma<T, PREC>::step(sc, idf[t], bfr);
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
          Mma<T, PREC>::step(dq[dc], acc_to_frag<T>(ds, kk), tr_frag<T>(sm.k[dc], r0, kk, lane));
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
template <typename T, int DC>
struct DbLds {  // beyond 64 KB (16-bit DC > 1, fp32): dynamic LDS
  unsigned char q[DC][DB_T * rowb<T>()];
  unsigned char d[DC][DB_T * rowb<T>()];
  unsigned char k[DC][DB_T * rowb<T>()];
  unsigned char v[DC][DB_T * rowb<T>()];
  float lse[DB_T];
  float delta[DB_T];
  float kb[DB_T];
  float pl2;  // -log2(N_res) when the row's keys are all masked, else 0
};

template <typename T, int DC, int PREC>
__global__ __launch_bounds__(DB_NT, 1) void bwd_dbias_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(16) unsigned char db_smem[];
  DbLds<T, DC>& sm = *reinterpret_cast<DbLds<T, DC>*>(db_smem);
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
    // indices clamped into the plane (elements past N are never stored), so the 32 loads
    // issue back to back instead of one at a time behind a branch each
    const T* plane = (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int kj = min(k0 + kw + 32 * sub + l32, N - 1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qq = min(q0 + qw + 8 * (i / 4) + 4 * g + (i % 4), N - 1);
        binit[sub][i] = TypeOps<T>::to_f32(plane[(int64_t)qq * a.bias_stride[2] + kj]);
        acc[sub][i] = 0.f;
      }
    }
  }

  // staging: thread = (row r = tid / 4, chunk c = tid % 4) of each of the four tiles. PF
  // register sets hold the next PF N_seq rows, so each row's loads have PF rows of compute to
  // arrive (two for D <= 32; wider heads have no registers to spare); the loads past the range
  // repeat its last row (in bounds, never used).
  constexpr int PF = 1;
  const int sr = tid >> 2, sc4 = tid & 3;
  V8 pq[PF][DC], pd[PF][DC], pk[PF][DC], pv[PF][DC];
  float plse[PF], pdel[PF];
  int pmk[PF];  // the key's raw mask byte (1 without a mask), compared only when staged
  auto load_stage = [&](int set, int s) {
    const int qi = q0 + sr, kj = k0 + sr;
    const bool qok = qi < N, kok = kj < N;
    const int64_t qo = (int64_t)b * a.q_stride[0] + (int64_t)s * a.q_stride[1] + (int64_t)h * a.q_stride[3];
    const int64_t doo = (int64_t)b * a.do_stride[0] + (int64_t)s * a.do_stride[1] + (int64_t)h * a.do_stride[3];
    const int64_t ko = (int64_t)b * a.k_stride[0] + (int64_t)s * a.k_stride[1] + (int64_t)h * a.k_stride[3];
    const int64_t vo = (int64_t)b * a.v_stride[0] + (int64_t)s * a.v_stride[1] + (int64_t)h * a.v_stride[3];
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      const int c0 = 32 * dc + 8 * sc4;
      pq[set][dc] = row8((const T*)a.q + qo + (int64_t)(qok ? qi : 0) * a.q_stride[2], c0, D, qok);
      pd[set][dc] = row8((const T*)a.dout + doo + (int64_t)(qok ? qi : 0) * a.do_stride[2], c0, D, qok);
      pk[set][dc] = row8((const T*)a.k + ko + (int64_t)(kok ? kj : 0) * a.k_stride[2], c0, D, kok);
      pv[set][dc] = row8((const T*)a.v + vo + (int64_t)(kok ? kj : 0) * a.v_stride[2], c0, D, kok);
    }
    if (sc4 == 0) {
      const int64_t lrow = (((int64_t)b * S + s) * H + h) * N;
      plse[set] = qok ? a.lse[lrow + qi] : INFINITY;  // absent queries: p = 0
      pdel[set] = qok ? a.delta[lrow + qi] : 0.f;
      pmk[set] = (a.mask && kok) ? (int)a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)kj * a.mask_stride[2]] : 1;
    }
  };
  auto store_stage = [&](int set) {
    // the staged values are first touched here, so the wait for their loads stays here (the
    // scaling of q would otherwise be scheduled at the top of the row's compute)
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) asm volatile("" : "+v"(pq[set][dc]), "+v"(pd[set][dc]), "+v"(pk[set][dc]), "+v"(pv[set][dc]));
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      *reinterpret_cast<V8*>(sm.q[dc] + swzt<T>(sr, sc4)) = TypeOps<T>::from_f32(TypeOps<T>::to_f32(pq[set][dc]) * a.scale);
      *reinterpret_cast<V8*>(sm.d[dc] + swzt<T>(sr, sc4)) = pd[set][dc];
      *reinterpret_cast<V8*>(sm.k[dc] + swzt<T>(sr, sc4)) = pk[set][dc];
      *reinterpret_cast<V8*>(sm.v[dc] + swzt<T>(sr, sc4)) = pv[set][dc];
    }
    if (sc4 == 0) {
      asm volatile("" : "+v"(plse[set]), "+v"(pdel[set]), "+v"(pmk[set]));
      sm.lse[sr] = plse[set];
      sm.delta[sr] = pdel[set];
      sm.kb[sr] = k0 + sr >= N ? -INFINITY : pmk[set] == 0 ? a.mask_value : 0.f;
      // every query of the row shares its keys' mask: the tile's first query (< N) decides
      if (sr == 0) sm.pl2 = (a.mask && plse[set] <= 0.5f * a.mask_value) ? -__log2f((float)N) : 0.f;
    }
  };
  // one N_seq row of the tile from LDS: sum_s dS += P (dP - Delta)
  auto compute_row = [&]() {
    // dO fragments negated and the dP accumulator started at Delta: the MFMA yields Delta - dP
    V8 qf[DC][2], ndof[DC][2];
#pragma unroll
    for (int dc = 0; dc < DC; ++dc)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        qf[dc][kk] = lds_row8<T>(sm.q[dc], qw + l32, 2 * kk + g);
        ndof[dc][kk] = neg8<T>(lds_row8<T>(sm.d[dc], qw + l32, 2 * kk + g));
      }
    f32x4 l4[4];
    f32x16 dinit;
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      l4[rg] = *reinterpret_cast<const f32x4*>(&sm.lse[qw + 8 * rg + 4 * g]);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sm.delta[qw + 8 * rg + 4 * g]);
#pragma unroll
      for (int e = 0; e < 4; ++e) dinit[4 * rg + e] = d4[e];
    }
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int kr = kw + 32 * sub + l32;
      f32x16 scv = binit[sub], ndp = dinit;
#pragma unroll
      for (int dc = 0; dc < DC; ++dc)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          Mma<T, PREC>::step(scv, qf[dc][kk], lds_row8<T>(sm.k[dc], kr, 2 * kk + g));
          Mma<T, PREC>::step(ndp, ndof[dc][kk], lds_row8<T>(sm.v[dc], kr, 2 * kk + g));
        }
      const float kb = sm.kb[kr], pl2 = sm.pl2;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * rg + e;
          const float pv = fast_exp2(__builtin_fmaf(scv[i] + kb - l4[rg][e], LOG2E_B, pl2));
          acc[sub][i] -= pv * ndp[i];
        }
    }
  };

  if (s_begin < s_end) {
    const int last = s_end - 1;
    load_stage(0, s_begin);
    store_stage(0);
#pragma unroll
    for (int j = 0; j < PF; ++j) load_stage(j, min(s_begin + 1 + j, last));
    __syncthreads();
    // whole groups of PF rows, with no branch between a set's loads and its use (the wait
    // before staging a set then leaves the other set's loads in flight)
    int s = s_begin;
    for (; s + PF <= s_end; s += PF) {
#pragma unroll
      for (int ph = 0; ph < PF; ++ph) {
        compute_row();
        __syncthreads();
        store_stage(ph);  // row s + ph + 1
        __syncthreads();
        load_stage(ph, min(s + ph + 1 + PF, last));
      }
    }
    if (s < s_end) compute_row();  // PF = 2 and an odd number of rows: the last one is in LDS
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

// The D = 32 (16-bit) form of bwd_dbias_kernel: the four tiles of each N_seq row arrive by
// global_load_lds (no staging registers) into a ring of DBD_NS stages, so the loads of the
// next DBD_NS - 1 rows are in flight while a row is computed, with one barrier per row. q is
// staged raw and scaled (Q' = T(q * scale), the same rounding) as its fragments are read. lse
// and Delta ride in the same ring (dword DMA); the key-mask bytes of 64 rows at a time are
// staged once per 64 rows.
constexpr int DBD_NS = 3;
constexpr int DBD_MROWS = 64;
struct DbdStage {
  unsigned char q[DB_T * ROWB];
  unsigned char d[DB_T * ROWB];
  unsigned char k[DB_T * ROWB];
  unsigned char v[DB_T * ROWB];
  float lse[DB_T];
  float delta[DB_T];
};
struct DbdLds {
  DbdStage st[DBD_NS];
  unsigned char mask[DBD_MROWS][DB_T];
};

template <typename T, bool MASK>
__global__ __launch_bounds__(DB_NT, 1) void bwd_dbias_dma_kernel(const gnn_triattn_bwd_args a) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(16) unsigned char db_smem[];
  DbdLds& sm = *reinterpret_cast<DbdLds*>(db_smem);
  const int N = (int)a.N, H = (int)a.H, S = (int)a.S;
  const int nt = (N + DB_T - 1) / DB_T;
  const int splits = a.dbias_splits > 1 ? a.dbias_splits : 1;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int kt = w % nt;
  const int qt = (w / nt) % nt;
  const int split = (w / (nt * nt)) % splits;
  const int64_t bh = w / ((uint32_t)splits * nt * nt);
  const int h = (int)(bh % H), b = (int)(bh / H);
  const int per = (S + splits - 1) / splits;
  const int s_begin = split * per, s_end = min(S, s_begin + per);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int qw = 32 * (wave & 3), kw = 64 * (wave >> 2);
  const int q0 = qt * DB_T, k0 = kt * DB_T;

  f32x16 binit[2], acc[2];
  {
    // indices clamped into the plane (elements past N are never stored), so the 32 loads
    // issue back to back instead of one at a time behind a branch each
    const T* plane = (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int kj = min(k0 + kw + 32 * sub + l32, N - 1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qq = min(q0 + qw + 8 * (i / 4) + 4 * g + (i % 4), N - 1);
        binit[sub][i] = TypeOps<T>::to_f32(plane[(int64_t)qq * a.bias_stride[2] + kj]);
        acc[sub][i] = 0.f;
      }
    }
  }

  // DMA work of a wave per row: tile wave / 2 (q, dO, k, v), its 16-row groups 4 (wave % 2) ..
  // 4 (wave % 2) + 3 (lane l: row l / 4 of the group, physical chunk l % 4 = logical chunk
  // (l % 4) ^ ((l / 16) % 4), the tiles' XOR swizzle), and one 64-float piece of lse / Delta
  // (waves 4..7 write the same bytes as waves 0..3). Rows past N repeat row N - 1: finite
  // values whose results are never stored.
  const int tile = wave >> 1, grp0 = 4 * (wave & 1);
  const int lrow = lane >> 2, ch = (lane & 3) ^ ((lane >> 4) & 3);
  const T* tsrc = tile == 0 ? (const T*)a.q + b * a.q_stride[0] + h * a.q_stride[3]
                : tile == 1 ? (const T*)a.dout + b * a.do_stride[0] + h * a.do_stride[3]
                : tile == 2 ? (const T*)a.k + b * a.k_stride[0] + h * a.k_stride[3]
                            : (const T*)a.v + b * a.v_stride[0] + h * a.v_stride[3];
  const int64_t trs = tile == 0 ? a.q_stride[2] : tile == 1 ? a.do_stride[2] : tile == 2 ? a.k_stride[2] : a.v_stride[2];
  const int64_t tss = tile == 0 ? a.q_stride[1] : tile == 1 ? a.do_stride[1] : tile == 2 ? a.k_stride[1] : a.v_stride[1];
  const int trow0 = tile < 2 ? q0 : k0;
  const int tbyte = tile * (DB_T * ROWB);  // offset of the tile within a stage
  const int piece = wave & 3;
  const float* ssrc = (piece < 2 ? a.lse : a.delta) + ((int64_t)b * S * H + h) * N + min(q0 + 64 * (piece & 1) + lane, N - 1);
  const int sbyte = 4 * DB_T * ROWB + (piece >> 1) * (DB_T * 4) + (piece & 1) * 256;
  auto issue = [&](int s, int stage) {
    unsigned char* base = reinterpret_cast<unsigned char*>(&sm.st[stage]);
    const T* src = tsrc + (int64_t)s * tss;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int grp = grp0 + j;
      const int r = min(trow0 + 16 * grp + lrow, N - 1);
      __builtin_amdgcn_global_load_lds((const void*)(src + (int64_t)r * trs + 8 * ch),
                                       (__attribute__((address_space(3))) void*)(base + tbyte + grp * 1024), 16, 0, 0);
    }
    __builtin_amdgcn_global_load_lds((const void*)(ssrc + (int64_t)s * H * N),
                                     (__attribute__((address_space(3))) void*)(base + sbyte), 4, 0, 0);
  };
  // the key-mask bytes of rows s0 .. s0 + 63 (clamped to the range) of the tile's keys
  auto stage_mask = [&](int s0) {
    const int kk = tid & (DB_T - 1), r0 = tid >> 7;
    const unsigned char* mrow = a.mask + b * a.mask_stride[0] + (int64_t)min(k0 + kk, N - 1) * a.mask_stride[2];
    unsigned char mv[DBD_MROWS / 4];
#pragma unroll
    for (int j = 0; j < DBD_MROWS / 4; ++j)
      mv[j] = mrow[(int64_t)min(s0 + r0 + 4 * j, s_end - 1) * a.mask_stride[1]];
#pragma unroll
    for (int j = 0; j < DBD_MROWS / 4; ++j) sm.mask[r0 + 4 * j][kk] = mv[j];
  };

  const float scale = a.scale;
  constexpr bool has_mask = MASK;
  const float pl2_masked = -__log2f((float)N);
  auto compute_row = [&](int stage, int mrow) {
    const DbdStage& st = sm.st[stage];
    // dO fragments negated (a sign flip, exact) and the dP accumulator started at Delta: the
    // MFMA yields Delta - dP, so dS = P (dP - Delta) needs no subtraction per element
    V8 qf[2], ndof[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      qf[kk] = TypeOps<T>::from_f32(TypeOps<T>::to_f32(lds_row8<T>(st.q, qw + l32, 2 * kk + g)) * scale);
      u32x4 u = __builtin_bit_cast(u32x4, lds_row8<T>(st.d, qw + l32, 2 * kk + g));
      u ^= 0x80008000u;
      ndof[kk] = __builtin_bit_cast(V8, u);
    }
    f32x4 l4[4];
    f32x16 dinit;
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      l4[rg] = *reinterpret_cast<const f32x4*>(&st.lse[qw + 8 * rg + 4 * g]);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(&st.delta[qw + 8 * rg + 4 * g]);
#pragma unroll
      for (int e = 0; e < 4; ++e) dinit[4 * rg + e] = d4[e];
    }
    // every query of the row shares its keys' mask: the tile's first query decides
    const float pl2 = (has_mask && st.lse[0] <= 0.5f * a.mask_value) ? pl2_masked : 0.f;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int kr = kw + 32 * sub + l32;
      f32x16 scv = binit[sub], ndp = dinit;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        Mma<T, PREC_NATIVE>::step(scv, qf[kk], lds_row8<T>(st.k, kr, 2 * kk + g));
        Mma<T, PREC_NATIVE>::step(ndp, ndof[kk], lds_row8<T>(st.v, kr, 2 * kk + g));
      }
      const float kb = (has_mask && sm.mask[mrow][kr] == 0) ? a.mask_value : 0.f;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * rg + e;
          // the logit minus lse first (in a fully masked row both sit near the sentinel)
          const float x = has_mask ? scv[i] + kb - l4[rg][e] : scv[i] - l4[rg][e];
          const float pv = fast_exp2(has_mask ? __builtin_fmaf(x, LOG2E_B, pl2) : x * LOG2E_B);
          acc[sub][i] -= pv * ndp[i];
        }
    }
  };

  if (s_begin < s_end) {
    const int last = s_end - 1;
    // rows s_begin .. s_begin + NS - 2 in flight before the loop; row s's stage is
    // (s - s_begin) % NS, and the row NS - 1 ahead goes into the stage computed last
#pragma unroll
    for (int j = 0; j < DBD_NS - 1; ++j) issue(min(s_begin + j, last), j);
    int stage = 0;
    for (int s = s_begin; s < s_end; ++s) {
      const int rr = s - s_begin;
      if (has_mask && rr % DBD_MROWS == 0) {
        __syncthreads();  // every wave is done with the previous 64 rows' mask bytes
        stage_mask(s);
      }
      // this wave's DMA of row s has landed once only the younger row's five remain (the
      // DMA per wave and row: four tile groups and one lse / Delta piece); after the barrier
      // every wave's has, and every wave is done with row s - 1's stage. (__syncthreads would
      // wait for every load in flight.)
      static_assert(DBD_NS == 3, "the wait below counts one younger row");
      asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      int nstage = stage + DBD_NS - 1;
      nstage -= nstage >= DBD_NS ? DBD_NS : 0;
      issue(min(s + DBD_NS - 1, last), nstage);
      compute_row(stage, rr % DBD_MROWS);
      stage = stage + 1 == DBD_NS ? 0 : stage + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outlives the workgroup
  }
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

// the DMA form of the dbias kernel moves 16-byte pieces of the q / dO / k / v rows: D = 32
// and every row start 16-byte aligned
bool dbias_dma_ok(const gnn_triattn_bwd_args& a) {
  if (a.D != 32) return false;
  const void* ptrs[4] = {a.q, a.dout, a.k, a.v};
  const int64_t* strides[4] = {a.q_stride, a.do_stride, a.k_stride, a.v_stride};
  for (int t = 0; t < 4; ++t) {
    if (reinterpret_cast<uintptr_t>(ptrs[t]) % 16 != 0) return false;
    for (int d = 0; d < 4; ++d)
      if (strides[t][d] % 8 != 0) return false;
  }
  return true;
}

template <typename T, int DC, int PREC>
int launch_bwd(const gnn_triattn_bwd_args& a, hipStream_t stream) {
  const int64_t nb128 = (a.N + 127) / 128;
  const dim3 grid((uint32_t)(nb128 * a.H * a.S * a.B));
  constexpr bool B16 = sizeof(T) == 2;
  // dq first: it also writes Delta, which dk / dv and dbias read. 16-bit D <= 32 rows take
  // the row-resident kernels and the DMA-ring pair-bias gradient.
  bool row_done = false, dma_ok = false;
  if constexpr (B16) {
    if (DC == 1 && triattn_bwd_row_applicable(a)) {
      const int rc = triattn_bwd_row_dq_dkdv(a, stream);
      if (rc != 0) return rc;
      row_done = true;
    }
    dma_ok = DC == 1 && dbias_dma_ok(a);
  }
  if (!row_done) {
    if (a.bias) {
      hipLaunchKernelGGL((bwd_dq_kernel<T, true, DC, PREC>), grid, dim3(BNT), 0, stream, a);
      hipLaunchKernelGGL((bwd_dkdv_kernel<T, true, DC, PREC>), grid, dim3(BNT), 0, stream, a);
    } else {
      hipLaunchKernelGGL((bwd_dq_kernel<T, false, DC, PREC>), grid, dim3(BNT), 0, stream, a);
      hipLaunchKernelGGL((bwd_dkdv_kernel<T, false, DC, PREC>), grid, dim3(BNT), 0, stream, a);
    }
  }
  if (a.bias && a.dbias) {
    const int64_t nt = (a.N + DB_T - 1) / DB_T;
    const int splits = a.dbias_splits > 1 ? a.dbias_splits : 1;
    const dim3 dgrid((uint32_t)(a.B * a.H * nt * nt * splits));
    if constexpr (B16) {
      if (dma_ok) {
        const size_t smem = sizeof(DbdLds);
        if (a.mask) {
          (void)hipFuncSetAttribute((const void*)bwd_dbias_dma_kernel<T, true>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
          hipLaunchKernelGGL((bwd_dbias_dma_kernel<T, true>), dgrid, dim3(DB_NT), smem, stream, a);
        } else {
          (void)hipFuncSetAttribute((const void*)bwd_dbias_dma_kernel<T, false>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
          hipLaunchKernelGGL((bwd_dbias_dma_kernel<T, false>), dgrid, dim3(DB_NT), smem, stream, a);
        }
      }
    }
    if (!dma_ok) {
      const size_t smem = sizeof(DbLds<T, DC>);
      const void* fn = (const void*)bwd_dbias_kernel<T, DC, PREC>;
      if (smem > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      hipLaunchKernelGGL((bwd_dbias_kernel<T, DC, PREC>), dgrid, dim3(DB_NT), smem, stream, a);
    }
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
    case GNN_BF16:
      return dc == 1 ? launch_bwd<bf16, 1, PREC_NATIVE>(a, stream)
                     : dc == 2 ? launch_bwd<bf16, 2, PREC_NATIVE>(a, stream) : launch_bwd<bf16, 4, PREC_NATIVE>(a, stream);
    case GNN_F16:
      return dc == 1 ? launch_bwd<f16, 1, PREC_NATIVE>(a, stream)
                     : dc == 2 ? launch_bwd<f16, 2, PREC_NATIVE>(a, stream) : launch_bwd<f16, 4, PREC_NATIVE>(a, stream);
    case GNN_F32:
      // fp32 tiles are twice the bytes: head dims up to 64 (the pair-bias gradient's four
      // [128][64] fp32 tiles take 128 KB of LDS)
      if (dc > 2)
        return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention backward: fp32 head dim must be at most 64");
      if (a.precision == GNN_PREC_BF16X3)
        return dc == 1 ? launch_bwd<float, 1, PREC_BF16X3>(a, stream) : launch_bwd<float, 2, PREC_BF16X3>(a, stream);
      return dc == 1 ? launch_bwd<float, 1, PREC_IEEE>(a, stream) : launch_bwd<float, 2, PREC_IEEE>(a, stream);
  }
  return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention backward: bf16 / fp16 / fp32 only");
}

}  // namespace gnn
