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
//                       is transposed through LDS), then out = (LN(o) Wpo^T + bpo) * g.
//
// Workspace (element type = input dtype): a, b, o are [B, Ch, N, NP] with a row pitch
// NP = round_up(N, 32) so every row is 16-byte aligned; g is [B, N, N, C].
#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

constexpr int NT = 256;  // threads per workgroup (4 waves)
constexpr int PT = 128;  // pixels per workgroup in the projection / output stages

__host__ __device__ inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

template <typename T>
__device__ __forceinline__ float ld_or(const void* p, int64_t i, float dflt) {
  return p ? TypeOps<T>::to_f32(((const T*)p)[i]) : dflt;
}

__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Row pitch (elements) of the LDS pixel tiles: 16 B of padding keeps the fragment reads
// of consecutive rows on distinct banks.
template <typename T>
__host__ __device__ constexpr int lds_pad() {
  return (int)(16 / sizeof(T));
}

// ============================== stage 1: LN-in + projections ==============================
template <typename T, int PREC>
__global__ __launch_bounds__(NT) void trimul_proj_kernel(const gnn_trimul_args a, int64_t NP,
                                                         size_t off_a, size_t off_b,
                                                         size_t off_g) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* zs = reinterpret_cast<T*>(smem_raw);
  const int C = (int)a.C, Ch = (int)a.Ch, N = (int)a.N;
  const int ZR = C + lds_pad<T>();

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

  // ---- load the x tile (PT pixels x C channels) into LDS
  const T* __restrict__ x = (const T*)a.x;
  const int cpp = C / 8;  // 8-element chunks per pixel
  for (int c = tid; c < PT * cpp; c += NT) {
    const int pl = c / cpp, k0 = (c % cpp) * 8;
    V8 v = zero8<T>();
    if (c0 + pl < N) v = load8(x + pix_index(pl) * C + k0);
    store8(&zs[pl * ZR + k0], v);
  }
  __syncthreads();

  // ---- LayerNorm, 2 threads per pixel, in place
  {
    const int pl = tid >> 1, half = tid & 1;
    const int k0 = half * (C / 2);
    float sum = 0.f;
    for (int k = k0; k < k0 + C / 2; k += 8) {
      f32x8 v = TypeOps<T>::to_f32(load8(&zs[pl * ZR + k]));
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += v[e];
    }
    sum += __shfl_xor(sum, 1);
    const float mean = sum / (float)C;
    float sq = 0.f;
    for (int k = k0; k < k0 + C / 2; k += 8) {
      f32x8 v = TypeOps<T>::to_f32(load8(&zs[pl * ZR + k]));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[e] - mean;
        sq += d * d;
      }
    }
    sq += __shfl_xor(sq, 1);
    const float rstd = 1.0f / sqrtf(sq / (float)C + a.eps);
    for (int k = k0; k < k0 + C / 2; k += 8) {
      f32x8 v = TypeOps<T>::to_f32(load8(&zs[pl * ZR + k]));
#pragma unroll
      for (int e = 0; e < 8; ++e)
        v[e] = (v[e] - mean) * rstd * ld_or<T>(a.ln_in_w, k + e, 1.f) + ld_or<T>(a.ln_in_b, k + e, 0.f);
      store8(&zs[pl * ZR + k], TypeOps<T>::from_f32(v));
    }
  }
  __syncthreads();

  // ---- projections. Units: [0, npg) gated p units of 32 channels of the 2*Ch projection
  // (p and its gate in one wave), then C/32 units of the output gate.
  const int npg = 2 * Ch / 32;
  const int nunits = npg + C / 32;
  const int nk = C / 16;
  T* __restrict__ a_cm = (T*)((unsigned char*)a.workspace + off_a);
  T* __restrict__ b_cm = (T*)((unsigned char*)a.workspace + off_b);
  T* __restrict__ gout = (T*)((unsigned char*)a.workspace + off_g);
  const T* __restrict__ wp = (const T*)a.p_in_w;
  const T* __restrict__ wg = (const T*)a.g_in_w;
  const T* __restrict__ wgo = (const T*)a.g_out_w;

  for (int u = wave; u < nunits; u += 4) {
    if (u < npg) {
      const int cc0 = 32 * u;
      float bp[16], bg[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ch = cc0 + 8 * (r / 4) + 4 * g + (r % 4);
        bp[r] = ld_or<T>(a.p_in_b, ch, 0.f);
        bg[r] = ld_or<T>(a.g_in_b, ch, 0.f);
      }
      for (int sub = 0; sub < PT / 32; ++sub) {
        f32x16 accp, accg;
#pragma unroll
        for (int r = 0; r < 16; ++r) accp[r] = accg[r] = 0.f;
        for (int k = 0; k < nk; ++k) {
          const V8 zf = load8(&zs[(32 * sub + l32) * ZR + 16 * k + 8 * g]);
          const V8 wpf = load8(wp + (int64_t)(cc0 + l32) * C + 16 * k + 8 * g);
          const V8 wgf = load8(wg + (int64_t)(cc0 + l32) * C + 16 * k + 8 * g);
          Mma<T, PREC>::step(accp, wpf, zf);  // [channel][pixel]
          Mma<T, PREC>::step(accg, wgf, zf);
        }
        const int pl = 32 * sub + l32;
        if (c0 + pl < N) {
          float mval = 1.f;
          if (a.mask) {
            const int cpos = c0 + pl;
            const int pp = outgoing ? row : cpos;
            const int qq = outgoing ? cpos : row;
            mval = TypeOps<T>::to_f32(((const T*)a.mask)[b * a.mask_stride[0] + pp * a.mask_stride[1] +
                                                         qq * a.mask_stride[2]]);
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int ch = cc0 + 8 * (r / 4) + 4 * g + (r % 4);
            const float v = (accp[r] + bp[r]) * sigmoid_acc(accg[r] + bg[r]) * mval;
            T* dst = ch < Ch ? a_cm : b_cm;
            const int chh = ch < Ch ? ch : ch - Ch;
            dst[(((int64_t)b * Ch + chh) * N + row) * NP + c0 + pl] = TypeOps<T>::from_f32(v);
          }
        }
      }
    } else {
      const int ch = 32 * (u - npg) + l32;
      const float bgo = ld_or<T>(a.g_out_b, ch, 0.f);
      for (int sub = 0; sub < PT / 32; ++sub) {
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        for (int k = 0; k < nk; ++k) {
          const V8 zf = load8(&zs[(32 * sub + l32) * ZR + 16 * k + 8 * g]);
          const V8 wf = load8(wgo + (int64_t)ch * C + 16 * k + 8 * g);
          Mma<T, PREC>::step(acc, zf, wf);  // [pixel][channel]
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int pl = 32 * sub + 8 * (r / 4) + 4 * g + (r % 4);
          if (c0 + pl < N) gout[pix_index(pl) * C + ch] = TypeOps<T>::from_f32(sigmoid_acc(acc[r] + bgo));
        }
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
template <typename T, int PREC>
__global__ __launch_bounds__(NT) void trimul_out_kernel(const gnn_trimul_args a, int64_t NP,
                                                        size_t off_g, size_t off_o) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int C = (int)a.C, Ch = (int)a.Ch, N = (int)a.N;
  const int OR = PT + lds_pad<T>();   // raw o tile [Ch][PT]
  const int ZR = Ch + lds_pad<T>();   // normalised tile [PT][Ch]
  T* ot = reinterpret_cast<T*>(smem_raw);
  T* zs = ot + Ch * OR;

  const int ntile = (N + PT - 1) / PT;
  const int ct = blockIdx.x % ntile;
  const int p = (blockIdx.x / ntile) % N;
  const int b = blockIdx.x / (ntile * N);
  const int q0 = ct * PT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;

  const T* __restrict__ ocm = (const T*)((const unsigned char*)a.workspace + off_o);
  const T* __restrict__ gg = (const T*)((const unsigned char*)a.workspace + off_g);
  T* __restrict__ out = (T*)a.out;

  // ---- o tile, channel-major: rows are channels, PT consecutive pixels each
  for (int c = tid; c < Ch * (PT / 8); c += NT) {
    const int ch = c / (PT / 8), k0 = (c % (PT / 8)) * 8;
    V8 v = zero8<T>();
    if (q0 + k0 < N) v = load8(ocm + (((int64_t)b * Ch + ch) * N + p) * NP + q0 + k0);
    store8(&ot[ch * OR + k0], v);
  }
  __syncthreads();

  // ---- LayerNorm over channels, 2 threads per pixel; result pixel-major in zs
  {
    const int pl = tid >> 1, half = tid & 1;
    const int k0 = half * (Ch / 2);
    float sum = 0.f;
    for (int k = k0; k < k0 + Ch / 2; ++k) sum += TypeOps<T>::to_f32(ot[k * OR + pl]);
    sum += __shfl_xor(sum, 1);
    const float mean = sum / (float)Ch;
    float sq = 0.f;
    for (int k = k0; k < k0 + Ch / 2; ++k) {
      const float d = TypeOps<T>::to_f32(ot[k * OR + pl]) - mean;
      sq += d * d;
    }
    sq += __shfl_xor(sq, 1);
    const float rstd = 1.0f / sqrtf(sq / (float)Ch + a.eps);
    for (int k = k0; k < k0 + Ch / 2; k += 8) {
      f32x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        v[e] = (TypeOps<T>::to_f32(ot[(k + e) * OR + pl]) - mean) * rstd *
                   ld_or<T>(a.ln_out_w, k + e, 1.f) +
               ld_or<T>(a.ln_out_b, k + e, 0.f);
      store8(&zs[pl * ZR + k], TypeOps<T>::from_f32(v));
    }
  }
  __syncthreads();

  // ---- out[pixel][c] = (z Wpo^T + bpo) * g; units = pixel sub-tile x 32 output channels
  const T* __restrict__ wpo = (const T*)a.p_out_w;
  const int nct = C / 32;
  const int nk = Ch / 16;
  for (int u = wave; u < (PT / 32) * nct; u += 4) {
    const int ps = u / nct, ctile = u % nct;
    const int ch = 32 * ctile + l32;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    for (int k = 0; k < nk; ++k) {
      const V8 zf = load8(&zs[(32 * ps + l32) * ZR + 16 * k + 8 * g]);
      const V8 wf = load8(wpo + (int64_t)ch * Ch + 16 * k + 8 * g);
      Mma<T, PREC>::step(acc, zf, wf);  // [pixel][channel]
    }
    const float bpo = ld_or<T>(a.p_out_b, ch, 0.f);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = q0 + 32 * ps + 8 * (r / 4) + 4 * g + (r % 4);
      if (q < N) {
        const int64_t pix = ((int64_t)b * N + p) * N + q;
        const float gv = TypeOps<T>::to_f32(gg[pix * C + ch]);
        out[pix * C + ch] = TypeOps<T>::from_f32((acc[r] + bpo) * gv);
      }
    }
  }
}

template <typename T, int PREC>
int launch_proj(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  const int64_t ntile = (a.N + PT - 1) / PT;
  const size_t smem = (size_t)PT * (a.C + lds_pad<T>()) * sizeof(T);
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
  const int64_t ntile = (a.N + PT - 1) / PT;
  const size_t smem =
      ((size_t)a.Ch * (PT + lds_pad<T>()) + (size_t)PT * (a.Ch + lds_pad<T>())) * sizeof(T);
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
  if ((size_t)PT * (a.C + 16 / e) * e > 160 * 1024 ||
      ((size_t)a.Ch * (PT + 16 / e) + (size_t)PT * (a.Ch + 16 / e)) * e > 160 * 1024)
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
