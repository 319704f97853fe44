// Triangle attention forward for gfx950 (MI355X).
//
// Computes, for every (b, s, h) row of the pair stack and every query i,
//   o[b,s,i,h,:] = sum_j softmax_j(l_ij) v[b,s,j,h,:],
//   l_ij = scale * q[b,s,i,h,:].k[b,s,j,h,:] + bias[b,h,i,j] + mask_bias[b,s,j]
// which is triangle_attention_torch (geometric_nn_ops_torch/triangle/_reference/
// triangle_attention.py:11-44) and the Triton forward it stands in for
// (geometric_nn_ops_torch/triangle/_kernels/triangle_attention.py:48-365).
//
// Design (one workgroup = 4 waves = 128 queries of one (b, s, h); one wave = 32 queries):
//   * The score tile is computed transposed, S^T = K Q'^T, on 32x32x16 MFMA so that each
//     lane ends up owning ONE query (l % 32) and 16 of the 32 keys of a sub-tile. The
//     softmax statistics are then per-lane scalars, the row max needs a single
//     permlane32 swap per 64 keys, and the row sum needs none until the end.
//   * O^T = V^T P^T: the probabilities feed the second MFMA straight from the score
//     registers (P^T is the B operand), and the running-max rescale of O is a per-lane
//     scalar multiply.
//   * K (row-major), V^T and the [128 query x 64 key] pair-bias tile are staged per key
//     tile in LDS (16-byte coalesced global loads), shared by the 4 waves; Q' =
//     bf16(q * scale), rounded like the reference's Q * softmax_scale, lives in registers.
//   * For 16-bit inputs the pair bias is added by the MFMA unit: one extra 32x32x16 step
//     per 16 keys multiplies an identity fragment (rows = keys) by the bias fragment read
//     from LDS (cols = queries), so no VALU work is spent on the bias. fp32 inputs add it
//     on the VALU.
//   * p = exp2(s * log2 e - m * log2 e) is one FMA and one v_exp_f32 per score (rows with
//     no live key use the exact (s - m) * log2 e, since m is then the -1e9 sentinel); the
//     row sum is taken on the rounded probabilities with v_dot2 (16-bit inputs), so the
//     normaliser matches what the PV product consumes.
//   * The running max is only moved when a tile raises it by more than 8 ln 2, so most
//     tiles skip the O / l rescale; p then stays below 2^8.
//   * Key tiles whose keys are all masked are skipped when the row has at least one
//     live key (their probabilities are exactly 0 either way). Rows with no live key
//     are computed in full, reproducing the finite-sentinel result of the reference.
//   * Keys past N get -inf; masked keys get the caller's mask_value (the reference's
//     bf16/fp16/fp32-rounded sentinel) added in fp32.
//   * Workgroup ids are remapped so the workgroups on one XCD walk consecutive
//     (b, s, h, q-block) items: the 4 q-blocks sharing K/V, and the heads sharing one
//     bias plane, then hit that XCD's L2.
#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

constexpr int QB = 128;  // queries per workgroup
constexpr int KT = 64;   // keys per LDS tile
constexpr int NTHREADS = 256;
constexpr int MAX_TILES = 512;  // N <= 32768
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_THRESHOLD = 8.0f / LOG2E;  // natural-log units: p <= 2^8

template <typename T, int DP>
struct Smem {
  static constexpr int KPAD = (sizeof(T) == 2) ? 8 : 4;  // 16 B per K row
  static constexpr int VPAD = 4;
  static constexpr int KROW = DP + KPAD;
  static constexpr int VROW = KT + VPAD;
  static constexpr int BROW = KT + KPAD;  // bias tile row pitch (16 B of padding)
  static constexpr int STAGE_BYTES = (KT * KROW + DP * VROW + QB * BROW) * (int)sizeof(T);
  // two stages (one barrier per key tile) when they fit in 80 KB, else one
  static constexpr int NBUF = 2 * STAGE_BYTES <= 80 * 1024 ? 2 : 1;
  T k[NBUF][KT * KROW];
  T vt[NBUF][DP * VROW];
  T bias[NBUF][QB * BROW];
  uint64_t tile_live[MAX_TILES];  // bit j: key tile*64+j is < N and unmasked
  uint16_t tile_list[MAX_TILES];
  int ntiles_run;
  int row_dead;
};

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 frag_from_acc(const f32x16& p, int t) {
  f32x8 x = {p[8 * t + 0], p[8 * t + 1], p[8 * t + 2], p[8 * t + 3],
             p[8 * t + 4], p[8 * t + 5], p[8 * t + 6], p[8 * t + 7]};
  return TypeOps<T>::from_f32(x);
}

// Adds the 8 probabilities of a fragment (as rounded for the MFMA, so the normaliser
// matches the numerator) to acc: two-element dot products with 1 for 16-bit types.
__device__ __forceinline__ float rowsum_add(const bf16x8& v, float acc) {
  const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
#pragma unroll
  for (int e = 0; e < 8; e += 2) acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[e], v[e + 1]}, one, acc, false);
  return acc;
}
__device__ __forceinline__ float rowsum_add(const f16x8& v, float acc) {
  const f16x2 one = {(f16)1.0f, (f16)1.0f};
#pragma unroll
  for (int e = 0; e < 8; e += 2) acc = __builtin_amdgcn_fdot2(f16x2{v[e], v[e + 1]}, one, acc, false);
  return acc;
}
__device__ __forceinline__ float rowsum_add(const f32x8& v, float acc) {
  return acc + (((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7])));
}

template <typename T, int PREC, int DP>
__global__ __launch_bounds__(NTHREADS, 2) void triattn_fwd_kernel(const gnn_triattn_args a) {
  typedef typename TypeOps<T>::V8 V8;
  typedef Smem<T, DP> S;
  constexpr int MP = (PREC == PREC_NATIVE) ? PREC_NATIVE : PREC;
  __shared__ S sm;

  const int N = (int)a.N;
  const int H = (int)a.H;
  const int D = (int)a.D;
  const int nqb = (N + QB - 1) / QB;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int qb = w % nqb;
  const int h = (w / nqb) % H;
  const int64_t bs = w / ((uint32_t)nqb * H);
  const int s = (int)(bs % a.S);
  const int b = (int)(bs / a.S);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int ntiles = (N + KT - 1) / KT;

  const T* __restrict__ qp = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3];
  const T* __restrict__ kp = (const T*)a.k + b * a.k_stride[0] + s * a.k_stride[1] + h * a.k_stride[3];
  const T* __restrict__ vp = (const T*)a.v + b * a.v_stride[0] + s * a.v_stride[1] + h * a.v_stride[3];
  T* __restrict__ op = (T*)a.o + b * a.o_stride[0] + s * a.o_stride[1] + h * a.o_stride[3];
  const int64_t qsn = a.q_stride[2], ksn = a.k_stride[2], vsn = a.v_stride[2], osn = a.o_stride[2];
  const bool has_bias = a.bias != nullptr;
  const T* __restrict__ biasp =
      has_bias ? (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] : nullptr;
  const int64_t bsi = a.bias_stride[2];
  const float mask_add = a.mask_value;

  // ---- per-row key liveness: one 64-bit word per key tile, and the list of tiles to run.
  if (wave == 0) {
    const uint8_t* mrow =
        a.mask ? a.mask + b * a.mask_stride[0] + s * a.mask_stride[1] : nullptr;
    int n = 0;  // tiles holding at least one live key, listed as they are found
    for (int t = 0; t < ntiles; ++t) {
      const int key = t * KT + lane;
      bool live = key < N;
      if (live && mrow) live = mrow[(int64_t)key * a.mask_stride[2]] != 0;
      const uint64_t bits = __ballot(live);
      if (lane == 0) {
        sm.tile_live[t] = bits;
        if (bits != 0) sm.tile_list[n] = (uint16_t)t;
      }
      n += bits != 0;
    }
    const int dead = n == 0;
    if (dead) {  // no live key anywhere in the row: every tile runs
      for (int t = lane; t < ntiles; t += 64) sm.tile_list[t] = (uint16_t)t;
      n = ntiles;
    }
    if (lane == 0) {
      sm.row_dead = dead;
      sm.ntiles_run = n;
    }
  }

  // ---- this wave's queries: Q' fragments (B operand of S^T = K Q'^T).
  const int q0 = qb * QB + wave * 32;
  const int myq = q0 + l32;
  const bool qvalid = myq < N;
  const float qscale = a.scale;
  V8 qf[DP / 16];
#pragma unroll
  for (int t = 0; t < DP / 16; ++t) {
    const int d0 = 16 * t + 8 * g;
    if (qvalid && d0 < D) {
      f32x8 x = TypeOps<T>::to_f32(load8(qp + myq * qsn + d0));
      qf[t] = TypeOps<T>::from_f32(x * qscale);
    } else {
      qf[t] = zero8<T>();
    }
  }

  f32x16 o[DP / 32];
#pragma unroll
  for (int c = 0; c < DP / 32; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[c][r] = 0.f;
  float m = -INFINITY;
  float lsum = 0.f;

  // identity A-fragments for the bias MFMA: element e of lane group g in step t is key
  // 16t + 8g + e; row l32 of the identity holds a 1 there iff l32 is that key.
  V8 idf[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) idf[t][e] = TypeOps<T>::from_f32(l32 == 16 * t + 8 * g + e ? 1.f : 0.f);

  __syncthreads();
  const int nrun = sm.ntiles_run;
  const bool row_dead = sm.row_dead != 0;

  // ---- K / V^T tile staging: each thread moves CH chunks of 8 elements of K and of V.
  constexpr int CPK = DP / 8;                  // chunks per key
  constexpr int CH = KT * CPK / NTHREADS;      // chunks per thread
  constexpr int BCH = QB * KT / 8 / NTHREADS;  // bias chunks per thread
  V8 kreg[CH], vreg[CH], breg[BCH];
  auto load_tile = [&](int t) {
    if (has_bias) {
#pragma unroll
      for (int i = 0; i < BCH; ++i) {
        const int c = tid + i * NTHREADS;
        const int q = qb * QB + c / (KT / 8);
        const int key = t * KT + (c % (KT / 8)) * 8;
        // keys up to the next multiple of 8 stay inside the row pitch (host guarantees it)
        breg[i] = (q < N && key < N) ? load8(biasp + (int64_t)q * bsi + key) : zero8<T>();
      }
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NTHREADS;
      const int key = t * KT + c / CPK;
      const int d0 = (c % CPK) * 8;
      if (key < N && d0 < D) {
        kreg[i] = load8(kp + key * ksn + d0);
        vreg[i] = load8(vp + key * vsn + d0);
      } else {
        kreg[i] = zero8<T>();
        vreg[i] = zero8<T>();
      }
    }
  };
  auto store_tile = [&](int buf) {
    if (has_bias) {
#pragma unroll
      for (int i = 0; i < BCH; ++i) {
        const int c = tid + i * NTHREADS;
        store8(&sm.bias[buf][(c / (KT / 8)) * S::BROW + (c % (KT / 8)) * 8], breg[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NTHREADS;
      const int kl = c / CPK;
      const int d0 = (c % CPK) * 8;
      store8(&sm.k[buf][kl * S::KROW + d0], kreg[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.vt[buf][(d0 + e) * S::VROW + kl] = vreg[i][e];
    }
  };

  if (nrun > 0) {
    load_tile(sm.tile_list[0]);
    store_tile(0);
  }
  __syncthreads();

  for (int it = 0; it < nrun; ++it) {
    const int cur = S::NBUF == 2 ? (it & 1) : 0;
    const int t = sm.tile_list[it];
    const bool has_next = it + 1 < nrun;
    if (has_next) load_tile(sm.tile_list[it + 1]);

    const uint64_t live = sm.tile_live[t];
    const int kbase = t * KT;
    const int nvalid = min(KT, N - kbase);
    const uint64_t valid = nvalid >= 64 ? ~0ull : ((1ull << nvalid) - 1ull);
    const bool all_live = live == ~0ull;  // every one of the 64 keys exists and is kept

    // S^T tile (+ bias): sc[sub][r] is key kbase + sub*32 + 8*(r/4) + 4g + r%4, query myq.
    f32x16 sc[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[sub][r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < DP / 16; ++kk) {
        const V8 kf = *reinterpret_cast<const V8*>(&sm.k[cur][(sub * 32 + l32) * S::KROW + 16 * kk + 8 * g]);
        Mma<T, MP>::step(sc[sub], kf, qf[kk]);
      }
      if (has_bias) {
        const T* brow = &sm.bias[cur][(wave * 32 + l32) * S::BROW + sub * 32];
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2)
            Mma<T, MP>::step(sc[sub], idf[t2], *reinterpret_cast<const V8*>(brow + 16 * t2 + 8 * g));
        } else {
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const f32x4 bv = TypeOps<T>::to_f32(load4(brow + 8 * rg + 4 * g));
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[sub][4 * rg + e] += bv[e];
          }
        }
      }
    }

    if (!all_live) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kl = sub * 32 + 8 * (r / 4) + 4 * g + (r % 4);
          if (!((valid >> kl) & 1ull))
            sc[sub][r] = -INFINITY;
          else if (!((live >> kl) & 1ull))
            sc[sub][r] += mask_add;
        }
    }

    // online softmax (log2 units), lazily rescaled
    float mt = sc[0][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, sc[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[1][r]);
    mt = pair_max(mt);
    if (__any(mt > m + RESCALE_THRESHOLD)) {
      const float mnew = fmaxf(m, mt);
      const float alpha = fast_exp2((m - mnew) * LOG2E);  // 0 on the first tile (m = -inf)
      m = mnew;
      lsum *= alpha;
#pragma unroll
      for (int c = 0; c < DP / 32; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[c][r] *= alpha;
    }
    V8 pf[2][2];
    const float nm = -m * LOG2E;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      if (sizeof(T) == 2 && !row_dead) {
        // residual of the folded FMA is below half an ulp of s * log2 e; after the 16-bit
        // rounding of p the row maximum still maps to exactly 1
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[sub][r] = fast_exp2(__builtin_fmaf(sc[sub][r], LOG2E, nm));
      } else {  // fp32, or m is the collapsed sentinel: subtract first so s - m is exact
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[sub][r] = fast_exp2((sc[sub][r] - m) * LOG2E);
      }
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        pf[sub][kk] = frag_from_acc<T>(sc[sub], kk);
        lsum = rowsum_add(pf[sub][kk], lsum);
      }
    }

    // O^T += V^T P^T. Fragment element e of k-step kk of sub-tile sub is key
    // sub*32 + 16*kk + 8*(e/4) + 4g + e%4 in both operands.
#pragma unroll
    for (int c = 0; c < DP / 32; ++c)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const T* vrow = &sm.vt[cur][(32 * c + l32) * S::VROW + sub * 32 + 16 * kk + 4 * g];
          const typename TypeOps<T>::V4 lo = load4(vrow);
          const typename TypeOps<T>::V4 hi = load4(vrow + 8);
          V8 vf;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vf[e] = lo[e];
            vf[e + 4] = hi[e];
          }
          Mma<T, MP>::step(o[c], vf, pf[sub][kk]);
        }

    if constexpr (S::NBUF == 2) {
      // the other stage was last read in the previous iteration, before its barrier
      if (has_next) store_tile(cur ^ 1);
      __syncthreads();
    } else {
      __syncthreads();
      if (has_next) store_tile(0);
      __syncthreads();
    }
  }

  // ---- normalise and store. o[c][r] is O[myq][32c + 8*(r/4) + 4g + r%4].
  const float ltot = pair_sum(lsum);
  const float inv = 1.0f / ltot;
  if (qvalid) {
    T* orow = op + (int64_t)myq * osn;
#pragma unroll
    for (int c = 0; c < DP / 32; ++c)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int d0 = 32 * c + 8 * rg + 4 * g;
        if (d0 < D) {
          f32x4 x = {o[c][4 * rg] * inv, o[c][4 * rg + 1] * inv, o[c][4 * rg + 2] * inv,
                     o[c][4 * rg + 3] * inv};
          store4(orow + d0, TypeOps<T>::from_f32(x));
        }
      }
    if (a.lse && g == 0) {
      // natural-log lse of the logits
      a.lse[((bs * H + h) * (int64_t)N) + myq] = m + __log2f(ltot) * (1.0f / LOG2E);
    }
  }
}

template <typename T, int PREC>
int launch_dp(const gnn_triattn_args& a, hipStream_t stream) {
  const int64_t nqb = (a.N + QB - 1) / QB;
  const int64_t nblk = nqb * a.H * a.S * a.B;
  dim3 grid((uint32_t)nblk), block(NTHREADS);
  if (a.D <= 32)
    hipLaunchKernelGGL((triattn_fwd_kernel<T, PREC, 32>), grid, block, 0, stream, a);
  else if (a.D <= 64)
    hipLaunchKernelGGL((triattn_fwd_kernel<T, PREC, 64>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((triattn_fwd_kernel<T, PREC, 128>), grid, block, 0, stream, a);
  return (int)hipGetLastError();
}

}  // namespace

int triattn_fwd(const gnn_triattn_args& a, hipStream_t stream) {
  if (a.N > (int64_t)MAX_TILES * KT)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention: N_res > 32768 is not supported");
  if (a.D > 128)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention: head dim > 128 is not supported");
  const int64_t nqb = (a.N + QB - 1) / QB;
  if (nqb * a.H * a.S * a.B >= (int64_t)1 << 31)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention: grid too large");
  switch (a.dtype) {
    case GNN_BF16: return launch_dp<bf16, PREC_NATIVE>(a, stream);
    case GNN_F16: return launch_dp<f16, PREC_NATIVE>(a, stream);
    case GNN_F32:
      return a.precision == GNN_PREC_BF16X3 ? launch_dp<float, PREC_BF16X3>(a, stream)
                                            : launch_dp<float, PREC_IEEE>(a, stream);
  }
  return set_error(GNN_ERR_ARG, "triangle_attention: unknown dtype");
}

}  // namespace gnn
