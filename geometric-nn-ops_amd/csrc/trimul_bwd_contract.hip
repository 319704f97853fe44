// Backward of the trimul contraction for 16-bit types: the two N^3 products of the gradient of
// o_c = A_c B_c^T per (batch, channel) plane c,
//     dA_c = dO_c B_c        (dA[i][k] = sum_j dO[i][j] B[j][k])
//     dB_c = dO_c^T A_c      (dB[j][k] = sum_i dO[i][j] A[i][k]),
// i.e. the backward of the einsum in _combine_projections (geometric_nn_ops_torch/triangle/
// _reference/trimul.py:44-54), which the reference leaves to autograd.
//
// Both products are C[m][n] = sum_c X[c][m] Y[c][n] with each operand stored column-blocked,
// [NP / 32 column blocks][rows][32 columns] (NP = round_up(N, 32)), the contraction index c
// being the row. That is how the forward's workspace already holds A and B (k-blocked:
// [k / 32][i][k % 32], so A[i][k] is row i, column k), so they are read in place; dO is
// supplied in the two layouts [i / 32][j][i % 32] (for dA) and [j / 32][i][j % 32] (for dB),
// rows zero-padded to NP. Operand rows past N of A and B are read from row N - 1: the dO rows
// they meet are zero.
//
// Kernel: the forward's DMA pipeline (global_load_lds_dwordx4 straight into LDS, STAGES - 1
// stages of 32 contraction rows in flight, one s_barrier per stage) with a BM x 256 output
// tile, but both operands are staged as they are stored, 32 rows x 64 bytes per 32-column
// block, and MFMA fragments are read down the columns with gfx950's ds_read_b64_tr_b16: a
// lane gets 4 consecutive rows of one column per read, two reads give the 8 contraction
// values of a fragment. Both operands use the same read pattern, so they agree on which
// contraction index each fragment element holds (element e of k-step kk is row
// 16 kk + 8 (e / 4) + 4 g + e % 4 of the stage) and the products are exact pairings.
#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

template <int BM>
struct ContractTT {
  static constexpr int BN = 256, BK = 32;
  static constexpr int NW = BM / 32;  // waves: a (BM / 64) x 2 grid of 64 x 128 wave tiles
  static constexpr int NTH = 64 * NW;
  static constexpr int STAGES = BM == 256 ? 4 : 3;
  static constexpr int BLK_BYTES = BK * 64;  // one 32-column block of a stage: 32 rows x 64 B
  static constexpr int X_BYTES = BM / 32 * BLK_BYTES, Y_BYTES = BN / 32 * BLK_BYTES;
  static constexpr int STAGE_BYTES = X_BYTES + Y_BYTES;
  static constexpr int QX = BM / 16 / NW, QY = BN / 16 / NW;  // 16-row DMA instructions per wave
  static constexpr int QPS = QX + QY;
  static constexpr int SP = BN + 8;     // epilogue row pitch (elements)
  static constexpr int EROWS = 128;     // epilogue rows per pass
  static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
  static_assert(EROWS * SP * 2 <= LDS_BYTES, "epilogue pass must fit the stage buffers");
  static_assert(QX * 16 * NW == BM && QY * 16 * NW == BN, "DMA split");
};

typedef __attribute__((address_space(3))) void lds_void_t;

template <int N_>
__device__ __forceinline__ void wait_vm_lgkm0_tt() {
  static_assert(N_ >= 0 && N_ < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x070 | N_);  // vmcnt(N_) expcnt(7) lgkmcnt(0)
}

// 4 consecutive rows of one 16-bit column of an LDS block with 64-byte rows, transposed
// across the lanes of each 16-lane group by ds_read_b64_tr_b16.
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V4 lds_read_tr4(const unsigned char* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(__attribute__((address_space(3))) const unsigned char*)p);
  return __builtin_bit_cast(typename TypeOps<T>::V4, v);
}

// One product over `planes` planes: X = [planes][NP / 32][x_rows][32], Y = [planes][NP / 32][y_rows][32],
// O = [planes][N][NP] (row m, column n; only m, n < N are written).
template <typename T, int BM>
__global__ __launch_bounds__(ContractTT<BM>::NTH, BM == 256 ? 1 : 2) void trimul_contract_tt_kernel(
    const T* __restrict__ X, int64_t x_rows, const T* __restrict__ Y, int64_t y_rows, T* __restrict__ O, int N,
    int64_t NP) {
  static_assert(sizeof(T) == 2, "16-bit operands");
  typedef typename TypeOps<T>::V8 V8;
  typedef typename TypeOps<T>::V4 V4;
  typedef ContractTT<BM> Cfg;
  __shared__ __align__(16) unsigned char smem[Cfg::LDS_BYTES];

  const int nbk = (int)(NP / 32);  // column blocks (and contraction stages)
  const int nti = (N + BM - 1) / BM;
  const int ntj = (N + Cfg::BN - 1) / Cfg::BN;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int tj = w % ntj;
  const int ti = (w / ntj) % nti;
  const int64_t plane = w / ((uint32_t)ntj * nti);
  const T* Xp = X + plane * nbk * x_rows * 32;
  const T* Yp = Y + plane * nbk * y_rows * 32;
  T* Op = O + plane * N * NP;
  const int m0 = ti * BM, n0 = tj * Cfg::BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  // DMA: instruction q of a wave moves 16 rows x 64 bytes of one column block (half hb of the
  // stage's 32 rows of block hb / 2); lane -> row lane / 4, 16-byte chunk lane % 4, so the
  // block lands in LDS exactly as stored. Source rows past the operand's rows repeat its last
  // row; blocks past NP / 32 repeat the last block (their outputs are not stored).
  const int drow = lane >> 2, dch = lane & 3;
  const T* xsrc[Cfg::QX];
  const T* ysrc[Cfg::QY];
  int xrow[Cfg::QX], yrow[Cfg::QY];
#pragma unroll
  for (int q = 0; q < Cfg::QX; ++q) {
    const int hb = Cfg::QX * wave + q;
    const int blk = min(m0 / 32 + hb / 2, nbk - 1);
    xsrc[q] = Xp + (int64_t)blk * x_rows * 32 + 8 * dch;
    xrow[q] = 16 * (hb & 1) + drow;
  }
#pragma unroll
  for (int q = 0; q < Cfg::QY; ++q) {
    const int hb = Cfg::QY * wave + q;
    const int blk = min(n0 / 32 + hb / 2, nbk - 1);
    ysrc[q] = Yp + (int64_t)blk * y_rows * 32 + 8 * dch;
    yrow[q] = 16 * (hb & 1) + drow;
  }
  auto issue = [&](int kt) {
    unsigned char* st = smem + (kt % Cfg::STAGES) * Cfg::STAGE_BYTES;
#pragma unroll
    for (int q = 0; q < Cfg::QX; ++q) {
      const int64_t r = min((int64_t)(32 * kt + xrow[q]), x_rows - 1);
      __builtin_amdgcn_global_load_lds((const void*)(xsrc[q] + r * 32),
                                       (lds_void_t*)(st + (Cfg::QX * wave + q) * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < Cfg::QY; ++q) {
      const int64_t r = min((int64_t)(32 * kt + yrow[q]), y_rows - 1);
      __builtin_amdgcn_global_load_lds((const void*)(ysrc[q] + r * 32),
                                       (lds_void_t*)(st + Cfg::X_BYTES + (Cfg::QY * wave + q) * 1024), 16, 0, 0);
    }
  };
  // transposed fragment of column l32 of block `blk` (k-step kk): rows 4g + (lane % 16) / 4 and
  // those 8 further down, 4 columns per 16-lane group
  const int tr_r = lane & 15;
  const int tr_off = ((tr_r >> 2) * 32 + 16 * ((lane >> 4) & 1) + 4 * (tr_r & 3)) * 2 + 4 * g * 64;
  auto frag = [&](const unsigned char* blk, int kk) -> V8 {
    const unsigned char* p = blk + 16 * kk * 64 + tr_off;
    const V4 lo = lds_read_tr4<T>(p);
    const V4 hi = lds_read_tr4<T>(p + 8 * 64);
    V8 f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = lo[e];
      f[e + 4] = hi[e];
    }
    return f;
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int y = 0; y < 4; ++y)
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[y][x][r] = 0.f;

  const int nkt = nbk;
#pragma unroll
  for (int st = 0; st < Cfg::STAGES - 1; ++st)
    if (st < nkt) issue(st);
  for (int kt = 0; kt < nkt; ++kt) {
    // this wave's DMA of stage kt has landed and its reads of stage kt - 1 have returned;
    // after the barrier every wave's stage kt is in LDS and the buffer of kt - 1 is free
    const int ahead = min(Cfg::STAGES - 2, nkt - 1 - kt);
    if (ahead >= 2)
      wait_vm_lgkm0_tt<2 * Cfg::QPS>();
    else if (ahead == 1)
      wait_vm_lgkm0_tt<Cfg::QPS>();
    else
      wait_vm_lgkm0_tt<0>();
    asm volatile("s_barrier" ::: "memory");
    if (kt + Cfg::STAGES - 1 < nkt) issue(kt + Cfg::STAGES - 1);
    const unsigned char* sx = smem + (kt % Cfg::STAGES) * Cfg::STAGE_BYTES;
    const unsigned char* sy = sx + Cfg::X_BYTES;
    constexpr int KS = Cfg::BK / 16;
    V8 xf[KS][2], yf[KS][4];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
      for (int x = 0; x < 2; ++x) xf[kk][x] = frag(sx + (2 * wm + x) * Cfg::BLK_BYTES, kk);
#pragma unroll
      for (int y = 0; y < 4; ++y) yf[kk][y] = frag(sy + (4 * wn + y) * Cfg::BLK_BYTES, kk);
    }
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int y = 0; y < 4; ++y)
#pragma unroll
        for (int x = 0; x < 2; ++x) Mma<T, PREC_NATIVE>::step(acc[y][x], yf[kk][y], xf[kk][x]);
    __builtin_amdgcn_sched_group_barrier(0x100, 12 * KS, 0);  // the LDS reads, in order
    __builtin_amdgcn_sched_group_barrier(0x008, 8 * KS, 0);   // then the MFMAs
  }

  // acc[y][x][r] = C[m = m0 + 64wm + 32x + l32][n = n0 + 128wn + 32y + 8(r/4) + 4g + r%4]
  T* ot = reinterpret_cast<T*>(smem);
  constexpr int CPR = Cfg::BN / 8;  // 16-byte chunks per output row
#pragma unroll
  for (int ep = 0; ep < BM / Cfg::EROWS; ++ep) {
    __syncthreads();  // stage buffers (or the previous pass) free
    if ((wm >> 1) == ep) {
#pragma unroll
      for (int y = 0; y < 4; ++y)
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const f32x4 v = {acc[y][x][4 * rg], acc[y][x][4 * rg + 1], acc[y][x][4 * rg + 2],
                             acc[y][x][4 * rg + 3]};
            store4(&ot[(64 * (wm & 1) + 32 * x + l32) * Cfg::SP + 128 * wn + 32 * y + 8 * rg + 4 * g],
                   TypeOps<T>::from_f32(v));
          }
    }
    __syncthreads();
#pragma unroll 4
    for (int c = tid; c < Cfg::EROWS * CPR; c += Cfg::NTH) {
      const int r = c / CPR, cn = (c % CPR) * 8;
      const int m = m0 + Cfg::EROWS * ep + r;
      if (m < N && n0 + cn < N) store8(Op + (int64_t)m * NP + n0 + cn, load8(&ot[r * Cfg::SP + cn]));
    }
  }
}

template <typename T, int BM>
int launch_tt(const T* X, int64_t x_rows, const T* Y, int64_t y_rows, T* O, int64_t planes, int N, int64_t NP,
              hipStream_t st) {
  typedef ContractTT<BM> Cfg;
  const int64_t nblk = planes * ((N + BM - 1) / BM) * ((N + Cfg::BN - 1) / Cfg::BN);
  hipLaunchKernelGGL((trimul_contract_tt_kernel<T, BM>), dim3((uint32_t)nblk), dim3(Cfg::NTH), 0, st, X, x_rows,
                     Y, y_rows, O, N, NP);
  return (int)hipGetLastError();
}

template <typename T>
int contract_bwd_t(const gnn_trimul_contract_bwd_args& a, hipStream_t st) {
  const int N = (int)a.N;
  const int64_t NP = (a.N + 31) / 32 * 32;
  // dA[i][k] = sum_j dO[i][j] B[j][k]:  X = dO as [i / 32][j][i % 32], Y = B
  // dB[j][k] = sum_i dO[i][j] A[i][k]:  X = dO as [j / 32][i][j % 32], Y = A
  auto run = [&](auto bm) {
    constexpr int BMv = decltype(bm)::value;
    int rc = launch_tt<T, BMv>((const T*)a.do_i, NP, (const T*)a.b, a.N, (T*)a.da, a.planes, N, NP, st);
    if (rc != 0) return rc;
    return launch_tt<T, BMv>((const T*)a.do_j, NP, (const T*)a.a, a.N, (T*)a.db, a.planes, N, NP, st);
  };
  if (N >= 512) return run(std::integral_constant<int, 256>{});
  return run(std::integral_constant<int, 128>{});
}

// ---- relayouts between the pixel-major rows of the op ([B, N, N, channels]) and per-channel
// planes. A lane moves an 8 x 8 block (8 positions along a plane row x 8 channels): eight
// 16-byte loads, a transpose in registers, eight 16-byte stores. Lane = (channel octet
// lane / 8, position octet lane % 8), so each load instruction reads 128 contiguous bytes per
// eight lanes on the side whose rows run along the positions, and each store writes 128
// contiguous bytes per eight lanes on the side whose rows run along the channels (64 bytes
// where a 32-column block ends). One wave covers 64 positions x 64 channels.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// w[j] = column j of the 8 x 8 16-bit matrix whose rows are v[0..7] (row r = 8 elements)
__device__ __forceinline__ void transpose8x8_16(const u32x4_t (&v)[8], u32x4_t (&w)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t a = v[2 * m][j >> 1], b = v[2 * m + 1][j >> 1];
      w[j][m] = (j & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
}

constexpr int RL_THREADS = 256;  // 4 waves, one 64 x 64 block each

// planes [B * Ch][N][src_ld] -> pixel rows [B N N][dst_ld] at channel dst_c0; plane element
// (r, s) is pixel (r, s), or (s, r) when transposed. Block = (b, r, 64 s, 64 channels).
__global__ __launch_bounds__(RL_THREADS) void planes_to_pixels_kernel(const gnn_trimul_relayout_args a,
                                                                      int64_t nblocks) {
  const int64_t N = a.N, Ch = a.Ch;
  const int64_t nsb = (N + 63) / 64, ncb = (Ch + 63) / 64;
  const int64_t blk = (int64_t)blockIdx.x * (RL_THREADS / 64) + (threadIdx.x >> 6);
  if (blk >= nblocks) return;
  const int lane = threadIdx.x & 63;
  int64_t t = blk;
  const int64_t cb = t % ncb;
  t /= ncb;
  const int64_t sb = t % nsb;
  t /= nsb;
  const int64_t r = t % N, b = t / N;
  const int64_t c0 = cb * 64 + 8 * (lane >> 3), s0 = sb * 64 + 8 * (lane & 7);
  if (c0 >= Ch || s0 >= N) return;
  const uint16_t* src = (const uint16_t*)a.src;
  uint16_t* dst = (uint16_t*)a.dst;
  u32x4_t v[8], w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    v[i] = *reinterpret_cast<const u32x4_t*>(src + ((b * Ch + c0 + i) * N + r) * a.src_ld + s0);
  transpose8x8_16(v, w);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t s = s0 + j;
    if (s < N) {
      const int64_t y = a.transposed ? s : r, x = a.transposed ? r : s;
      *reinterpret_cast<u32x4_t*>(dst + ((b * N + y) * N + x) * a.dst_ld + a.dst_c0 + c0) = w[j];
    }
  }
}

// pixel rows [B N N][src_ld] (channels src_c0 ..) -> per-plane row blocks [B * Ch][NP / 32][NP][32]:
// element (i, j) of plane (b, c) at ((i / 32) NP + j) 32 + i % 32 (i-blocked), or at
// ((j / 32) NP + i) 32 + j % 32 when transposed (j-blocked); zero outside i, j < N.
// Block = (b, the row index of the layout, 64 blocked positions, 64 channels).
__global__ __launch_bounds__(RL_THREADS) void pixels_to_blocked_kernel(const gnn_trimul_relayout_args a,
                                                                       int64_t nblocks) {
  const int64_t N = a.N, Ch = a.Ch, NP = (a.N + 31) / 32 * 32;
  const int64_t nsb = (NP + 63) / 64, ncb = (Ch + 63) / 64;
  const int64_t blk = (int64_t)blockIdx.x * (RL_THREADS / 64) + (threadIdx.x >> 6);
  if (blk >= nblocks) return;
  const int lane = threadIdx.x & 63;
  int64_t t = blk;
  const int64_t cb = t % ncb;
  t /= ncb;
  const int64_t sb = t % nsb;
  t /= nsb;
  const int64_t row = t % NP, b = t / NP;  // j (i-blocked) or i (j-blocked)
  const int64_t c0 = cb * 64 + 8 * (lane >> 3), s0 = sb * 64 + 8 * (lane & 7);  // s: the blocked index
  if (c0 >= Ch || s0 >= NP) return;
  const uint16_t* src = (const uint16_t*)a.src;
  uint16_t* dst = (uint16_t*)a.dst;
  u32x4_t v[8], w[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int64_t i = a.transposed ? row : s0 + q, j = a.transposed ? s0 + q : row;
    if (i < N && j < N)
      v[q] = *reinterpret_cast<const u32x4_t*>(src + ((b * N + i) * N + j) * a.src_ld + a.src_c0 + c0);
    else
      v[q] = u32x4_t{0u, 0u, 0u, 0u};
  }
  transpose8x8_16(v, w);
  const int64_t off = ((s0 / 32) * NP + row) * 32 + s0 % 32;
#pragma unroll
  for (int c = 0; c < 8; ++c)
    *reinterpret_cast<u32x4_t*>(dst + (b * Ch + c0 + c) * NP * NP + off) = w[c];
}

}  // namespace

int trimul_relayout(const gnn_trimul_relayout_args& a, hipStream_t st) {
  const int64_t ncb = (a.Ch + 63) / 64;
  int64_t nblocks;
  if (a.mode == GNN_RELAYOUT_PLANES_TO_PIXELS) {
    nblocks = a.B * a.N * ((a.N + 63) / 64) * ncb;
  } else {
    const int64_t NP = (a.N + 31) / 32 * 32;
    nblocks = a.B * NP * ((NP + 63) / 64) * ncb;
  }
  const int64_t grid = (nblocks + RL_THREADS / 64 - 1) / (RL_THREADS / 64);
  if (grid >= ((int64_t)1 << 31)) return set_error(GNN_ERR_UNSUPPORTED, "trimul_relayout: grid too large");
  if (a.mode == GNN_RELAYOUT_PLANES_TO_PIXELS)
    hipLaunchKernelGGL(planes_to_pixels_kernel, dim3((uint32_t)grid), dim3(RL_THREADS), 0, st, a, nblocks);
  else
    hipLaunchKernelGGL(pixels_to_blocked_kernel, dim3((uint32_t)grid), dim3(RL_THREADS), 0, st, a, nblocks);
  return (int)hipGetLastError();
}

int trimul_contract_bwd(const gnn_trimul_contract_bwd_args& a, hipStream_t st) {
  if (a.dtype == GNN_BF16) return contract_bwd_t<bf16>(a, st);
  return contract_bwd_t<f16>(a, st);
}

}  // namespace gnn
