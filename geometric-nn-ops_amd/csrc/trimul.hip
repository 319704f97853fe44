// Triangle multiplicative update forward for gfx950 (MI355X), three kernels.
//
// Reference math: trimul_torch (geometric_nn_ops_torch/triangle/_reference/trimul.py:57-97);
// reference kernels: trimul_triton (geometric_nn_ops_torch/triangle/_kernels/trimul.py:404-448).
//
//   proj     (stage 1)  z = LN_in(x) (fp32 statistics, biased variance, 1/sqrt(var+eps) as
//                       F.layer_norm), then ONE pass over z for all 4*Ch + C output columns:
//                       p = (z Wp^T + bp) * sigmoid(z Wg^T + bg) * mask, split into a / b and
//                       written channel-major; g = sigmoid(z Wgo^T + bgo) written pixel-major.
//                       z never leaves LDS. For 'incoming' the pixel tile walks a column of
//                       the pair grid instead of a row, so a and b land transposed per
//                       channel and stage 2 is the same N x N x N product for both directions.
//   contract (stage 2)  o_c = A_c B_c^T per (batch, channel): a 128x128-tile MFMA GEMM with
//                       both operands k-contiguous, staged through LDS.
//   out      (stage 3)  LN_out over the Ch channels of each pixel (the channel-major o tile
//                       is read down its columns in LDS), then out = (LN(o) Wpo^T + bpo) * g.
//
// Workspace (element type = input dtype): a, b, o are [B, Ch, N, NP] with a row pitch
// NP = round_up(N, 32) so every row is 16-byte aligned; g is [B, N, N, C].
#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

constexpr int NT = 256;  // threads per workgroup (4 waves)
constexpr int PT = 128;  // pixels per workgroup in the projection stage
constexpr int LDB = 8;   // tile loads kept in flight per thread (issued before their LDS stores)

__host__ __device__ inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

template <typename T>
__device__ __forceinline__ float ld_or(const void* p, int64_t i, float dflt) {
  return p ? TypeOps<T>::to_f32(((const T*)p)[i]) : dflt;
}

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal (about 1 ulp
// each), instead of an IEEE division sequence per element. x -> -inf gives rcp(inf) = 0,
// x -> +inf gives rcp(1) = 1.
__device__ __forceinline__ float sigmoid_acc(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// Row pitch (elements) of the LDS pixel tiles: 16 B of padding keeps the fragment reads
// of consecutive rows on distinct banks.
template <typename T>
__host__ __device__ constexpr int lds_pad() {
  return (int)(16 / sizeof(T));
}

// Orders LDS accesses of the lanes of one wave (a wave executes its LDS operations in
// order; this keeps the compiler from moving them across the exchange).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-wave epilogue staging tile of the projection stage: max(32 x (64 + pad), 64 x (32 + pad)).
template <typename T>
__host__ __device__ constexpr int proj_ebuf_elems() {
  return (32 * (64 + lds_pad<T>()) > 64 * (32 + lds_pad<T>())) ? 32 * (64 + lds_pad<T>())
                                                                 : 64 * (32 + lds_pad<T>());
}
// LDS of the projection stage: z tile [PT][C + pad] (T), LN gamma / beta [C] and the mask
// of the tile [PT] (fp32), then 4 staging tiles (T), each region 16-byte aligned.
template <typename T>
__host__ __device__ inline size_t proj_ebuf_offset(int C) {
  const size_t head = (size_t)PT * (C + lds_pad<T>()) * sizeof(T) + (2 * (size_t)C + PT) * sizeof(float);
  return (head + 15) / 16 * 16;
}
template <typename T>
__device__ __forceinline__ T* proj_ebuf(unsigned char* smem, int C) {
  return reinterpret_cast<T*>(smem + proj_ebuf_offset<T>(C));
}

// ============================== stage 1: LN-in + projections ==============================
// One workgroup = PT pixels along one row ('outgoing') or column ('incoming') of the pair
// grid. LDS holds the x tile (normalised in place to z), the LayerNorm parameters and the
// tile's mask values. Work units per wave: 32 channels of the 2*Ch gated projection (p and
// its gate g_in share the unit so the epilogue can combine them), or 32 channels of the
// output gate. Weight fragments are read once per pair of 32-pixel sub-tiles.
template <typename T, int PREC>
#ifndef GNN_PROJ_MINBLOCKS
#define GNN_PROJ_MINBLOCKS 2
#endif
__global__ __launch_bounds__(NT, GNN_PROJ_MINBLOCKS) void trimul_proj_kernel(const gnn_trimul_args a, int64_t NP,
                                                            size_t off_a, size_t off_b,
                                                            size_t off_g) {
  typedef typename TypeOps<T>::V8 V8;
  typedef typename TypeOps<T>::V4 V4;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int C = (int)a.C, Ch = (int)a.Ch, N = (int)a.N;
  const int ZR = C + lds_pad<T>();
  T* zs = reinterpret_cast<T*>(smem_raw);                                   // [PT][ZR]
  float* lnw = reinterpret_cast<float*>(smem_raw + (size_t)PT * ZR * sizeof(T));  // [C]
  float* lnb = lnw + C;                                                      // [C]
  float* mk = lnb + C;                                                       // [PT]

  const int ntile = (N + PT - 1) / PT;
  const int ct = blockIdx.x % ntile;
  const int row = (blockIdx.x / ntile) % N;
  const int b = blockIdx.x / (ntile * N);
  const int c0 = ct * PT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const bool outgoing = a.outgoing != 0;

  // pixel (pp, qq) of local pixel index pl: outgoing walks row `row`, incoming column `row`
  auto pix_index = [&](int pl) -> int64_t {
    const int cpos = c0 + pl;
    const int pp = outgoing ? row : cpos;
    const int qq = outgoing ? cpos : row;
    return ((int64_t)b * N + pp) * N + qq;
  };

  for (int c = tid; c < C; c += NT) {
    lnw[c] = ld_or<T>(a.ln_in_w, c, 1.f);
    lnb[c] = ld_or<T>(a.ln_in_b, c, 0.f);
  }
  for (int pl = tid; pl < PT; pl += NT) {
    float mval = 1.f;
    if (a.mask && c0 + pl < N) {
      const int cpos = c0 + pl;
      const int pp = outgoing ? row : cpos;
      const int qq = outgoing ? cpos : row;
      mval = TypeOps<T>::to_f32(
          ((const T*)a.mask)[b * a.mask_stride[0] + pp * a.mask_stride[1] + qq * a.mask_stride[2]]);
    }
    mk[pl] = mval;
  }

  // ---- x tile (PT pixels x C channels) into LDS, LDB 16-byte loads in flight per thread
  const T* __restrict__ x = (const T*)a.x;
  const int cpp = C / 8;
  for (int cb = 0; cb < PT * cpp; cb += LDB * NT) {
    V8 v[LDB];
#pragma unroll
    for (int i = 0; i < LDB; ++i) {
      const int c = cb + tid + i * NT, pl = c / cpp, k0 = (c % cpp) * 8;
      v[i] = zero8<T>();
      if (c < PT * cpp && c0 + pl < N) v[i] = load8(x + pix_index(pl) * C + k0);
    }
#pragma unroll
    for (int i = 0; i < LDB; ++i) {
      const int c = cb + tid + i * NT, pl = c / cpp, k0 = (c % cpp) * 8;
      if (c < PT * cpp) store8(&zs[pl * ZR + k0], v[i]);
    }
  }
  __syncthreads();

  // ---- LayerNorm in place (fp32 statistics, biased variance). Thread = (pixel tid % 128,
  // channel half tid / 128), so the lanes of a wave read 64 different rows at one column
  // (conflict-free); the two halves' partial sums meet in LDS (the staging area, idle now).
  {
    const int pl = tid & (PT - 1), half = tid / PT;
    const int k0 = half * (C / 2);
    T* zrow = &zs[pl * ZR];
    float* red = reinterpret_cast<float*>(proj_ebuf<T>(smem_raw, C));  // [2 stats][2 halves][PT]
    float sum = 0.f;
    for (int k = k0; k < k0 + C / 2; k += 8) {
      const f32x8 v = TypeOps<T>::to_f32(load8(zrow + k));
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += v[e];
    }
    red[half * PT + pl] = sum;
    __syncthreads();
    const float mean = (red[pl] + red[PT + pl]) / (float)C;
    float sq = 0.f;
    for (int k = k0; k < k0 + C / 2; k += 8) {
      const f32x8 v = TypeOps<T>::to_f32(load8(zrow + k));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[e] - mean;
        sq += d * d;
      }
    }
    red[2 * PT + half * PT + pl] = sq;
    __syncthreads();
    const float rstd = 1.0f / sqrtf((red[2 * PT + pl] + red[3 * PT + pl]) / (float)C + a.eps);
    for (int k = k0; k < k0 + C / 2; k += 8) {
      f32x8 v = TypeOps<T>::to_f32(load8(zrow + k));
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(lnw + k);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(lnw + k + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(lnb + k);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(lnb + k + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = (v[e] - mean) * rstd * w0[e] + b0[e];
        v[e + 4] = (v[e + 4] - mean) * rstd * w1[e] + b1[e];
      }
      store8(zrow + k, TypeOps<T>::from_f32(v));
    }
  }
  __syncthreads();

  const int npg = 2 * Ch / 32;
  const int nunits = npg + C / 32;
  const int nk = C / 16;
  T* __restrict__ a_cm = (T*)((unsigned char*)a.workspace + off_a);
  T* __restrict__ b_cm = (T*)((unsigned char*)a.workspace + off_b);
  T* __restrict__ gout = (T*)((unsigned char*)a.workspace + off_g);
  const T* __restrict__ wp = (const T*)a.p_in_w;
  const T* __restrict__ wg = (const T*)a.g_in_w;
  const T* __restrict__ wgo = (const T*)a.g_out_w;
  // wave-private staging tile for the epilogues (32 channels x 64 pixels, or 64 x 32)
  T* ebuf = proj_ebuf<T>(smem_raw, C) + wave * proj_ebuf_elems<T>();
  constexpr int ER = 64 + lds_pad<T>();  // [32 channel rows][64 pixels] (a / b)
  constexpr int EG = 32 + lds_pad<T>();  // [64 pixel rows][32 channels] (g)

  for (int u = wave; u < nunits; u += 4) {
    if (u < npg) {
      // acc[s] = [pixel][channel] tiles: row = pixel 32*s + 8*(r/4) + 4g + r%4, col = channel
      const int ch = 32 * u + l32;  // channel of the 2*Ch projection held by this lane
      const float bp = ld_or<T>(a.p_in_b, ch, 0.f);
      const float bg = ld_or<T>(a.g_in_b, ch, 0.f);
      const T* wprow = wp + (int64_t)ch * C + 8 * g;
      const T* wgrow = wg + (int64_t)ch * C + 8 * g;
      // weight fragments of up to KCH k-steps stay in registers across the pixel sub-tiles
      constexpr int KCH = sizeof(T) == 2 ? 8 : 4;
      V8 wpf[KCH], wgf[KCH];
      auto load_w = [&](int kc) {
#pragma unroll
        for (int j = 0; j < KCH; ++j)
          if (kc + j < nk) {
            wpf[j] = load8(wprow + 16 * (kc + j));
            wgf[j] = load8(wgrow + 16 * (kc + j));
          }
      };
      if (nk <= KCH) load_w(0);
      for (int sp = 0; sp < PT / 32; sp += 2) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          f32x16 accp, accg;
#pragma unroll
          for (int r = 0; r < 16; ++r) accp[r] = accg[r] = 0.f;
          for (int kc = 0; kc < nk; kc += KCH) {
            if (nk > KCH) load_w(kc);
#pragma unroll
            for (int j = 0; j < KCH; ++j) {
              if (kc + j >= nk) break;
              const V8 zf = load8(&zs[(32 * (sp + s2) + l32) * ZR + 16 * (kc + j) + 8 * g]);
              Mma<T, PREC>::step(accp, zf, wpf[j]);
              Mma<T, PREC>::step(accg, zf, wgf[j]);
            }
          }
          // gated, masked values -> staging tile [channel l32][pixel]
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int pt = 32 * s2 + 8 * rg + 4 * g;  // pixel within the sub-tile pair
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              v[e] = (accp[4 * rg + e] + bp) * sigmoid_acc(accg[4 * rg + e] + bg) * mk[32 * sp + pt + e];
            store4(&ebuf[l32 * ER + pt], TypeOps<T>::from_f32(v));
          }
        }
        wave_lds_sync();
        // 16-byte stores, 8 lanes per 128-byte channel row segment
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = lane + 64 * i;
          const int crow = c / 8, p0 = (c % 8) * 8;
          const int chg = 32 * u + crow;
          T* dst = chg < Ch ? a_cm : b_cm;
          const int chh = chg < Ch ? chg : chg - Ch;
          const int pl = 32 * sp + p0;
          T* drow = dst + (((int64_t)b * Ch + chh) * N + row) * NP + c0 + pl;
          const V8 val = load8(&ebuf[crow * ER + p0]);
          if (c0 + pl + 8 <= N) {
            store8(drow, val);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (c0 + pl + e < N) drow[e] = val[e];
          }
        }
        wave_lds_sync();
      }
    } else {
      // acc[s] = [channel][pixel]: row = channel c00 + 8*(r/4) + 4g + r%4, col = pixel
      const int c00 = 32 * (u - npg);
      float bgo[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) bgo[r] = ld_or<T>(a.g_out_b, c00 + 8 * (r / 4) + 4 * g + (r % 4), 0.f);
      const T* wrow = wgo + (int64_t)(c00 + l32) * C + 8 * g;
      constexpr int KCH = sizeof(T) == 2 ? 8 : 4;
      V8 wf[KCH];
      auto load_w = [&](int kc) {
#pragma unroll
        for (int j = 0; j < KCH; ++j)
          if (kc + j < nk) wf[j] = load8(wrow + 16 * (kc + j));
      };
      if (nk <= KCH) load_w(0);
      for (int sp = 0; sp < PT / 32; sp += 2) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          f32x16 acc;
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r] = 0.f;
          for (int kc = 0; kc < nk; kc += KCH) {
            if (nk > KCH) load_w(kc);
#pragma unroll
            for (int j = 0; j < KCH; ++j) {
              if (kc + j >= nk) break;
              const V8 zf = load8(&zs[(32 * (sp + s2) + l32) * ZR + 16 * (kc + j) + 8 * g]);
              Mma<T, PREC>::step(acc, wf[j], zf);
            }
          }
          // sigmoid -> staging tile [pixel][channel]
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = sigmoid_acc(acc[4 * rg + e] + bgo[4 * rg + e]);
            store4(&ebuf[(32 * s2 + l32) * EG + 8 * rg + 4 * g], TypeOps<T>::from_f32(v));
          }
        }
        wave_lds_sync();
        // 16-byte stores, 4 lanes per 64-byte pixel row segment
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = lane + 64 * i;
          const int px = c / 4, k0 = (c % 4) * 8;
          const int pl = 32 * sp + px;
          if (c0 + pl < N) store8(gout + pix_index(pl) * C + c00 + k0, load8(&ebuf[px * EG + k0]));
        }
        wave_lds_sync();
      }
    }
  }
}

// ============================== stage 2: per-channel contraction ==========================
template <typename T>
struct ContractCfg {
  static constexpr int BM = 128, BN = 128;
  static constexpr int BK = sizeof(T) == 2 ? 64 : 32;  // 128 B of k per row per stage
  static constexpr int ROW = BK + lds_pad<T>();
};

template <typename T, int PREC>
__global__ __launch_bounds__(NT, 2) void trimul_contract_kernel(const T* __restrict__ A,
                                                                const T* __restrict__ Bm,
                                                                T* __restrict__ O, int N,
                                                                int64_t NP) {
  typedef typename TypeOps<T>::V8 V8;
  typedef ContractCfg<T> Cfg;
  __shared__ __align__(16) T as[Cfg::BM * Cfg::ROW];
  __shared__ __align__(16) T bs[Cfg::BN * Cfg::ROW];

  const int nti = (N + Cfg::BM - 1) / Cfg::BM;
  const int ntj = (N + Cfg::BN - 1) / Cfg::BN;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int tj = w % ntj;
  const int ti = (w / ntj) % nti;
  const int64_t plane = w / ((uint32_t)ntj * nti);
  const int64_t poff = plane * N * NP;
  const T* Ap = A + poff;
  const T* Bp = Bm + poff;
  T* Op = O + poff;
  const int i0 = ti * Cfg::BM, j0 = tj * Cfg::BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  constexpr int CPR = Cfg::BK / 8;                 // chunks per row per stage
  constexpr int CH = Cfg::BM * CPR / NT;           // chunks per thread per operand
  V8 ra[CH], rb[CH];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NT;
      const int r = c / CPR, kc = k0 + (c % CPR) * 8;
      ra[i] = zero8<T>();
      rb[i] = zero8<T>();
      if (kc < N) {
        if (kc + 8 <= N) {
          if (i0 + r < N) ra[i] = load8(Ap + (int64_t)(i0 + r) * NP + kc);
          if (j0 + r < N) rb[i] = load8(Bp + (int64_t)(j0 + r) * NP + kc);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (kc + e < N) {
              if (i0 + r < N) ra[i][e] = Ap[(int64_t)(i0 + r) * NP + kc + e];
              if (j0 + r < N) rb[i][e] = Bp[(int64_t)(j0 + r) * NP + kc + e];
            }
        }
      }
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NT;
      const int r = c / CPR, kl = (c % CPR) * 8;
      store8(&as[r * Cfg::ROW + kl], ra[i]);
      store8(&bs[r * Cfg::ROW + kl], rb[i]);
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[x][y][r] = 0.f;

  const int nkt = (N + Cfg::BK - 1) / Cfg::BK;
  load(0);
  store();
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const bool has_next = kt + 1 < nkt;
    if (has_next) load((kt + 1) * Cfg::BK);
#pragma unroll
    for (int kk = 0; kk < Cfg::BK / 16; ++kk) {
      V8 af[2], bf[2];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        af[x] = load8(&as[(64 * wm + 32 * x + l32) * Cfg::ROW + 16 * kk + 8 * g]);
#pragma unroll
      for (int y = 0; y < 2; ++y)
        bf[y] = load8(&bs[(64 * wn + 32 * y + l32) * Cfg::ROW + 16 * kk + 8 * g]);
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) Mma<T, PREC>::step(acc[x][y], af[x], bf[y]);
    }
    __syncthreads();
    if (has_next) store();
    __syncthreads();
  }

  // acc[x][y][r] = o[i0 + 64wm + 32x + 8(r/4) + 4g + r%4][j0 + 64wn + 32y + l32]
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int j = j0 + 64 * wn + 32 * y + l32;
      if (j >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + 64 * wm + 32 * x + 8 * (r / 4) + 4 * g + (r % 4);
        if (i < N) Op[(int64_t)i * NP + j] = TypeOps<T>::from_f32(acc[x][y][r]);
      }
    }
}

// ============================== stage 3: LN-out + p_out + gate ============================
// One workgroup = PTO consecutive pixels of one row of the pair grid; their g and out rows
// form one contiguous block of PTO * C elements (pixel-major). The channel-major o tile is
// loaded with 16-byte rows and normalised per pixel (lanes walk consecutive pixels of one
// channel row), then p_out runs on MFMA in passes of OPC output channels, one 32-channel
// tile per wave. A pass writes the linear output, rounded to T as the reference's linear
// layer does, into an LDS tile; the workgroup then streams the tile out with 16-byte g loads
// and 16-byte out stores over the contiguous block, multiplying in fp32 and rounding once.
// The g chunk of a pass is loaded into registers one pass ahead (the first before the o
// tile), so its latency hides behind the LayerNorm / the previous pass.
constexpr int PTO = 64;
constexpr int OPC = 128;                  // output channels per pass (4 waves x 32)
constexpr int OCH = PTO * OPC / 8 / NT;  // 8-element chunks per thread per pass

// LDS of the output stage: region 1 = the raw o tile [Ch][PTO + pad], reused after the
// LayerNorm as the pass tile [PTO][OPC + pad]; then the normalised tile [PTO][Ch + pad] (T),
// LN gamma / beta [Ch] and the LayerNorm partial sums [2][4][PTO] (fp32).
__host__ __device__ inline size_t out_region1_elems(int64_t Ch, int pad) {
  const int64_t o = Ch * (PTO + pad), y = (int64_t)PTO * (OPC + pad);
  return (size_t)(o > y ? o : y);
}
__host__ __device__ inline size_t out_lds_bytes(int64_t Ch, size_t elem) {
  const int pad = (int)(16 / elem);
  return (out_region1_elems(Ch, pad) + (size_t)PTO * (Ch + pad)) * elem + (2 * (size_t)Ch + 8 * PTO) * 4;
}

// Chunk i of a thread = 8 output channels (c8) of one pixel (px) of the pass's
// [PTO][W] sub-block, W = 8 * W8 channels; consecutive threads take consecutive chunks.
template <typename T>
__device__ __forceinline__ void out_load_g(typename TypeOps<T>::V8 (&gr)[OCH], const T* __restrict__ gblk,
                                           int C, int c0, int W8, int npix, int tid) {
#pragma unroll
  for (int i = 0; i < OCH; ++i) {
    const int idx = tid + i * NT, px = idx / W8, c8 = idx - px * W8;
    gr[i] = zero8<T>();
    if (idx < PTO * W8 && px < npix) gr[i] = load8(gblk + (int64_t)px * C + c0 + 8 * c8);
  }
}

template <typename T, int PREC>
__global__ __launch_bounds__(NT, 2) void trimul_out_kernel(const gnn_trimul_args a, int64_t NP,
                                                           size_t off_g, size_t off_o) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int C = (int)a.C, Ch = (int)a.Ch, N = (int)a.N;
  const int OR = PTO + lds_pad<T>();  // raw o tile [Ch][OR]
  const int ZR = Ch + lds_pad<T>();   // normalised tile [PTO][ZR]
  const int YR = OPC + lds_pad<T>();  // pass tile [PTO][YR]
  T* ot = reinterpret_cast<T*>(smem_raw);
  T* ys = ot;  // the o tile is dead once the LayerNorm has written zs
  T* zs = ot + out_region1_elems(Ch, lds_pad<T>());
  float* lnw = reinterpret_cast<float*>(zs + (size_t)PTO * ZR);
  float* lnb = lnw + Ch;
  float* red = lnb + Ch;  // [2 stats][4 quarters][PTO] partial sums

  const int ntile = (N + PTO - 1) / PTO;
  const int ct = blockIdx.x % ntile;
  const int p = (blockIdx.x / ntile) % N;
  const int b = blockIdx.x / (ntile * N);
  const int q0 = ct * PTO;
  const int npix = N - q0 < PTO ? N - q0 : PTO;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;

  const T* __restrict__ ocm = (const T*)((const unsigned char*)a.workspace + off_o);
  const int64_t blk = (((int64_t)b * N + p) * N + q0) * C;
  const T* __restrict__ gblk = (const T*)((const unsigned char*)a.workspace + off_g) + blk;
  T* __restrict__ oblk = (T*)a.out + blk;

  V8 gr[OCH];
  out_load_g<T>(gr, gblk, C, 0, (C < OPC ? C : OPC) / 8, npix, tid);

  for (int c = tid; c < Ch; c += NT) {
    lnw[c] = ld_or<T>(a.ln_out_w, c, 1.f);
    lnb[c] = ld_or<T>(a.ln_out_b, c, 0.f);
  }
  for (int cb = 0; cb < Ch * (PTO / 8); cb += LDB * NT) {
    V8 v[LDB];
#pragma unroll
    for (int i = 0; i < LDB; ++i) {
      const int c = cb + tid + i * NT, ch = c / (PTO / 8), k0 = (c % (PTO / 8)) * 8;
      v[i] = zero8<T>();
      if (c < Ch * (PTO / 8) && q0 + k0 < N) v[i] = load8(ocm + (((int64_t)b * Ch + ch) * N + p) * NP + q0 + k0);
    }
#pragma unroll
    for (int i = 0; i < LDB; ++i) {
      const int c = cb + tid + i * NT, ch = c / (PTO / 8), k0 = (c % (PTO / 8)) * 8;
      if (c < Ch * (PTO / 8)) store8(&ot[ch * OR + k0], v[i]);
    }
  }
  __syncthreads();

  // ---- LayerNorm over channels. Thread = (pixel tid % 64, channel quarter tid / 64): the
  // lanes of a wave read 64 consecutive pixels of one channel row (conflict-free); the
  // quarters' partial sums meet in LDS.
  {
    const int pl = tid & (PTO - 1), qtr = tid / PTO;
    const int k0 = qtr * (Ch / 4), k1 = k0 + Ch / 4;
    float sum = 0.f;
    for (int k = k0; k < k1; ++k) sum += TypeOps<T>::to_f32(ot[k * OR + pl]);
    red[qtr * PTO + pl] = sum;
    __syncthreads();
    const float mean = ((red[pl] + red[PTO + pl]) + (red[2 * PTO + pl] + red[3 * PTO + pl])) / (float)Ch;
    float sq = 0.f;
    for (int k = k0; k < k1; ++k) {
      const float d = TypeOps<T>::to_f32(ot[k * OR + pl]) - mean;
      sq += d * d;
    }
    float* red2 = red + 4 * PTO;
    red2[qtr * PTO + pl] = sq;
    __syncthreads();
    const float var = ((red2[pl] + red2[PTO + pl]) + (red2[2 * PTO + pl] + red2[3 * PTO + pl])) / (float)Ch;
    const float rstd = 1.0f / sqrtf(var + a.eps);
    for (int k = k0; k < k1; k += 8) {
      f32x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        v[e] = (TypeOps<T>::to_f32(ot[(k + e) * OR + pl]) - mean) * rstd * lnw[k + e] + lnb[k + e];
      store8(&zs[pl * ZR + k], TypeOps<T>::from_f32(v));
    }
  }
  __syncthreads();

  // ---- out = (z Wpo^T + bpo) * g, in passes of OPC output channels.
  // acc[s] = [cout][pixel]: cout = c0 + 32 wave + 8(r/4) + 4g + r%4, pixel = 32s + l32.
  const T* __restrict__ wpo = (const T*)a.p_out_w;
  const int nk = Ch / 16;
  for (int c0 = 0; c0 < C; c0 += OPC) {
    const int W = C - c0 < OPC ? C - c0 : OPC;
    if (32 * wave < W) {
      const int cw = c0 + 32 * wave;
      float bpo[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) bpo[r] = ld_or<T>(a.p_out_b, cw + 4 * g + 8 * (r / 4) + (r % 4), 0.f);
      const T* wrow = wpo + (int64_t)(cw + l32) * Ch + 8 * g;
      f32x16 acc[PTO / 32];
#pragma unroll
      for (int s = 0; s < PTO / 32; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][r] = 0.f;
      for (int k = 0; k < nk; ++k) {
        const V8 wf = load8(wrow + 16 * k);
#pragma unroll
        for (int s = 0; s < PTO / 32; ++s) {
          const V8 zf = load8(&zs[(32 * s + l32) * ZR + 16 * k + 8 * g]);
          Mma<T, PREC>::step(acc[s], wf, zf);
        }
      }
#pragma unroll
      for (int s = 0; s < PTO / 32; ++s)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[s][4 * rg + e] + bpo[4 * rg + e];
          store4(&ys[(32 * s + l32) * YR + 32 * wave + 8 * rg + 4 * g], TypeOps<T>::from_f32(v));
        }
    }
    __syncthreads();
    const int W8 = W / 8;
#pragma unroll
    for (int i = 0; i < OCH; ++i) {
      const int idx = tid + i * NT, px = idx / W8, c8 = idx - px * W8;
      if (idx < PTO * W8 && px < npix) {
        const f32x8 y = TypeOps<T>::to_f32(load8(&ys[px * YR + 8 * c8]));
        store8(oblk + (int64_t)px * C + c0 + 8 * c8, TypeOps<T>::from_f32(y * TypeOps<T>::to_f32(gr[i])));
      }
    }
    if (c0 + OPC < C) {
      __syncthreads();  // the next pass rewrites ys
      const int Wn = C - c0 - OPC < OPC ? C - c0 - OPC : OPC;
      out_load_g<T>(gr, gblk, C, c0 + OPC, Wn / 8, npix, tid);
    }
  }
}

template <typename T>
size_t proj_smem(const gnn_trimul_args& a) {
  return proj_ebuf_offset<T>((int)a.C) + 4 * (size_t)proj_ebuf_elems<T>() * sizeof(T);
}

template <typename T>
size_t out_smem(const gnn_trimul_args& a) {
  return out_lds_bytes(a.Ch, sizeof(T));
}

template <typename T, int PREC>
int launch_proj(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  const int64_t ntile = (a.N + PT - 1) / PT;
  const size_t smem = proj_smem<T>(a);
  if (smem > 64 * 1024)
    (void)hipFuncSetAttribute((const void*)trimul_proj_kernel<T, PREC>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  hipLaunchKernelGGL((trimul_proj_kernel<T, PREC>), dim3((uint32_t)(a.B * a.N * ntile)), dim3(NT),
                     smem, st, a, NP, L.off_a, L.off_b, L.off_g);
  return (int)hipGetLastError();
}

template <typename T, int PREC>
int launch_contract(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  typedef ContractCfg<T> Cfg;
  const int64_t nblk = a.B * a.Ch * ((a.N + Cfg::BM - 1) / Cfg::BM) * ((a.N + Cfg::BN - 1) / Cfg::BN);
  unsigned char* ws = (unsigned char*)a.workspace;
  hipLaunchKernelGGL((trimul_contract_kernel<T, PREC>), dim3((uint32_t)nblk), dim3(NT), 0, st,
                     (const T*)(ws + L.off_a), (const T*)(ws + L.off_b), (T*)(ws + L.off_o), (int)a.N,
                     NP);
  return (int)hipGetLastError();
}

template <typename T, int PREC>
int launch_out(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  const int64_t ntile = (a.N + PTO - 1) / PTO;
  const size_t smem = out_smem<T>(a);
  if (smem > 64 * 1024)
    (void)hipFuncSetAttribute((const void*)trimul_out_kernel<T, PREC>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  hipLaunchKernelGGL((trimul_out_kernel<T, PREC>), dim3((uint32_t)(a.B * a.N * ntile)), dim3(NT),
                     smem, st, a, NP, L.off_g, L.off_o);
  return (int)hipGetLastError();
}

int check_args(const gnn_trimul_args& a, const char* who) {
  (void)who;
  if (!a.x || !a.out || !a.p_in_w || !a.g_in_w || !a.p_out_w || !a.g_out_w)
    return set_error(GNN_ERR_ARG, "trimul: x, out and the four projection weights are required");
  if (a.B < 1 || a.N < 1 || a.C < 1 || a.Ch < 1)
    return set_error(GNN_ERR_ARG, "trimul: B, N, C and Ch must be positive");
  if (a.C % 32 != 0 || a.Ch % 32 != 0)
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: c_z and c_hidden must be multiples of 32");
  if (a.C > 512 || a.Ch > 512)
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: c_z and c_hidden above 512 are not supported");
  if (a.dtype != GNN_BF16 && a.dtype != GNN_F16 && a.dtype != GNN_F32)
    return set_error(GNN_ERR_ARG, "trimul: unknown dtype");
  const void* vec[] = {a.x, a.out, a.p_in_w, a.g_in_w, a.p_out_w, a.g_out_w, a.workspace};
  for (const void* ptr : vec)
    if (((uintptr_t)ptr) % 16 != 0)
      return set_error(GNN_ERR_ARG, "trimul: x, out, weights and workspace must be 16-byte aligned");
  const size_t e = a.dtype == GNN_F32 ? 4 : 2;
  const size_t proj_lds = (size_t)PT * (a.C + 16 / e) * e + (2 * (size_t)a.C + PT) * 4 + 16 +
                          4 * (size_t)(e == 2 ? proj_ebuf_elems<bf16>() : proj_ebuf_elems<float>()) * e;
  const size_t out_lds = out_lds_bytes(a.Ch, e);
  if (proj_lds > 160 * 1024 || out_lds > 160 * 1024)
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: channel count too large for the LDS tiles");
  if (a.B * a.N * ((a.N + PT - 1) / PT) >= ((int64_t)1 << 31))
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: grid too large");
  const TrimulLayout L = trimul_layout(a.B, a.N, a.C, a.Ch, a.dtype);
  if (!a.workspace || a.workspace_bytes < L.total)
    return set_error(GNN_ERR_WORKSPACE, "trimul: workspace missing or smaller than gnn_trimul_workspace_bytes()");
  return GNN_OK;
}

}  // namespace

TrimulLayout trimul_layout(int64_t B, int64_t N, int64_t C, int64_t Ch, int32_t dtype) {
  const size_t e = dtype == GNN_F32 ? 4 : 2;
  const int64_t NP = round_up(N, 32);
  const size_t cm = (size_t)round_up((int64_t)(B * Ch * N * NP * e), 256);
  const size_t pm = (size_t)round_up((int64_t)(B * N * N * C * e), 256);
  TrimulLayout L;
  L.off_a = 0;
  L.off_b = cm;
  L.off_g = 2 * cm;
  L.off_o = 2 * cm + pm;
  L.total = 3 * cm + pm;
  return L;
}

#define GNN_TRIMUL_DISPATCH(FN)                                                         \
  switch (a.dtype) {                                                                    \
    case GNN_BF16: return FN<bf16, PREC_NATIVE>(a, L, st);                              \
    case GNN_F16: return FN<f16, PREC_NATIVE>(a, L, st);                                \
    default:                                                                            \
      return a.precision == GNN_PREC_BF16X3 ? FN<float, PREC_BF16X3>(a, L, st)          \
                                            : FN<float, PREC_IEEE>(a, L, st);           \
  }

int trimul_proj(const gnn_trimul_args& a, hipStream_t st) {
  if (int rc = check_args(a, "proj")) return rc;
  const TrimulLayout L = trimul_layout(a.B, a.N, a.C, a.Ch, a.dtype);
  GNN_TRIMUL_DISPATCH(launch_proj)
}

int trimul_contract(const gnn_trimul_args& a, hipStream_t st) {
  if (int rc = check_args(a, "contract")) return rc;
  const TrimulLayout L = trimul_layout(a.B, a.N, a.C, a.Ch, a.dtype);
  GNN_TRIMUL_DISPATCH(launch_contract)
}

int trimul_out(const gnn_trimul_args& a, hipStream_t st) {
  if (int rc = check_args(a, "out")) return rc;
  const TrimulLayout L = trimul_layout(a.B, a.N, a.C, a.Ch, a.dtype);
  GNN_TRIMUL_DISPATCH(launch_out)
}

}  // namespace gnn
