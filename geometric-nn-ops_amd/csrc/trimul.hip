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
// Workspace (element type = input dtype), NP = round_up(N, 32): o is [B, Ch, N, NP] (16-byte
// aligned rows); g is [B, N, N, C]; a and b hold the same N x NP matrix per channel, k-blocked
// as [B, Ch, NP / 32, N, 32] for 16-bit types (zeros in columns N .. NP-1) and row-major
// [B, Ch, N, NP] for fp32.
#include "gnn_common.hpp"
#include "gnn_internal.hpp"

#include <algorithm>
#include <string>
#include <type_traits>

namespace gnn {

namespace {

constexpr int NT = 256;  // threads per workgroup (4 waves)
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

// Element offset of (plane, row i, column k) in the a / b operands of the contraction
// (plane = batch * Ch + channel, k < NP). 16-bit types: k-blocked [plane][NP / 32][N][32], so
// that one 32-column pipeline stage of a block of rows is a single contiguous range;
// fp32: row-major [plane][N][NP].
template <typename T>
__host__ __device__ inline int64_t ab_offset(int64_t plane, int row, int k, int N, int64_t NP) {
  if constexpr (sizeof(T) == 2)
    return ((plane * (NP / 32) + k / 32) * N + row) * 32 + (k % 32);
  else
    return (plane * N + row) * NP + k;
}

// Sum over the 8 lanes 8k .. 8k + 7 (every lane gets it) with DPP lane moves instead of
// LDS-routed shuffles: pairs (quad_perm 1,0,3,2), quads (2,3,0,1), then the two quads of the
// half-row (row_half_mirror pairs lane i with 7 - i, which lies in the other quad).
__device__ __forceinline__ float sum8_dpp(float x) {
  auto mv = [](float v, int ctrl) {
    int r;
    switch (ctrl) {
      case 0: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false); break;
      case 1: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false); break;
      default: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false); break;
    }
    return __int_as_float(r);
  };
  x += mv(x, 0);
  x += mv(x, 1);
  return x + mv(x, 2);
}

// Orders LDS accesses of the lanes of one wave (a wave executes its LDS operations in
// order; this keeps the compiler from moving them across the exchange).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ============================== stage 1: LN-in + projections ==============================
// Persistent kernel: PW waves per workgroup, as many workgroups as fit on the device at
// once, each looping over pixel tiles of PTP pixels along one row ('outgoing') or column
// ('incoming') of the pair grid. Work per tile: the 2*Ch gated projection in units of 32
// channels (p and its gate g_in together, over all PTP pixels), and the output gate g_out
// in items of 32 channels x 32 pixels. Wave w takes projection units w, w + PW, ... and
// gate items w, w + PW, ...; while a wave's unit does not change between tiles (C = Ch =
// 128: one unit of each kind per wave) its weight fragments and biases stay in registers
// for the whole launch.
//
// The x of the next tile is loaded into registers while the current tile's MFMAs and
// epilogues run, 8 threads per pixel, each holding up to XM 8-channel chunks of it. A thread
// reduces its chunks to a LayerNorm partial (mean, M2); after one barrier it merges the
// pixel's 8 partials (the pairwise update of Chan, Golub and LeVeque: exact for the
// combined mean and sum of squared deviations), normalises its chunks and writes z into the
// single LDS tile, which a second barrier hands to the next iteration.
constexpr int PW = 8;          // waves per projection workgroup
constexpr int PNT = 64 * PW;   // threads per projection workgroup
constexpr int PTP = 64;        // pixels per tile
constexpr int PSUB = PTP / 32; // 32-pixel sub-tiles per tile

// Epilogue staging of a projection unit: [32 channels][SPT * 32 pixels] (128-byte channel
// rows), reused as [32 pixels][32 channels] by the gate items.
template <typename T>
__host__ __device__ constexpr int proj_spt() {
  return sizeof(T) == 2 ? 2 : 1;
}
template <typename T>
__host__ __device__ constexpr int proj_er() {
  return 32 * proj_spt<T>() + lds_pad<T>();
}
template <typename T>
__host__ __device__ constexpr int proj_ebuf_elems() {
  return 32 * proj_er<T>();
}

// LDS of the projection stage (byte offsets, 16-byte aligned): z tile [PTP][C + pad] (T),
// one staging tile per wave (T), LayerNorm partials [8][PTP] (float2), LN gamma / beta [C]
// and the tile's mask values [PTP] (fp32).
struct ProjLds {
  size_t zs, ebuf, red, lnw, mk, total;
};
template <typename T>
__host__ __device__ inline ProjLds proj_lds(int64_t C) {
  ProjLds L;
  L.zs = 0;
  L.ebuf = ((size_t)PTP * (C + lds_pad<T>()) * sizeof(T) + 15) / 16 * 16;
  L.red = L.ebuf + (size_t)PW * proj_ebuf_elems<T>() * sizeof(T);
  L.lnw = L.red + 8 * (size_t)PTP * 2 * sizeof(float);
  L.mk = L.lnw + ((2 * (size_t)C * sizeof(float) + 15) / 16 * 16);
  L.total = L.mk + PTP * sizeof(float);
  return L;
}

// Tile t of the projection stage. Outgoing tiles step along a row of the pair grid first,
// incoming tiles along the column index, so concurrently running workgroups read
// neighbouring memory. Local pixel pl of a tile is pair-grid pixel (row, c0 + pl) for
// 'outgoing' and (c0 + pl, row) for 'incoming'.
struct PTile {
  int b, row, c0;
};
__device__ __forceinline__ PTile proj_tile(int64_t t, int N, bool outgoing) {
  const int ntp = (N + PTP - 1) / PTP;
  PTile r;
  if (outgoing) {
    r.c0 = (int)(t % ntp) * PTP;
    const int64_t rest = t / ntp;
    r.row = (int)(rest % N);
    r.b = (int)(rest / N);
  } else {
    r.row = (int)(t % N);
    const int64_t rest = t / N;
    r.c0 = (int)(rest % ntp) * PTP;
    r.b = (int)(rest / ntp);
  }
  return r;
}
// The tiles t, t + G, t + 2G, ... of a persistent workgroup as mixed-radix digits (d0
// fastest, radix r0; then d1, radix r1; then d2), advanced by G's digits with carries: a
// scalar add and compare per digit and step in place of the 64-bit divisions of the tile
// decomposition, which the compiler emulates on the vector ALU (and moves back to scalar
// registers) for every tile.
struct TileWalk {
  int d0, d1, d2, g0, g1, g2, r0, r1;
  __device__ __forceinline__ TileWalk(int64_t t, int64_t G, int r0_, int r1_) : r0(r0_), r1(r1_) {
    d0 = (int)(t % r0);
    const int64_t q = t / r0;
    d1 = (int)(q % r1);
    d2 = (int)(q / r1);
    g0 = (int)(G % r0);
    const int64_t h = G / r0;
    g1 = (int)(h % r1);
    g2 = (int)(h / r1);
  }
  __device__ __forceinline__ void step() {
    d0 += g0;
    const int c0 = d0 >= r0;
    d0 -= c0 ? r0 : 0;
    d1 += g1 + c0;
    const int c1 = d1 >= r1;
    d1 -= c1 ? r1 : 0;
    d2 += g2 + c1;
  }
};
// proj_tile's decomposition for a walk: outgoing (c0 / PTP, row, b), incoming (row, c0 / PTP, b)
__device__ __forceinline__ TileWalk proj_walk(int64_t t, int64_t G, int N, bool outgoing) {
  const int ntp = (N + PTP - 1) / PTP;
  return outgoing ? TileWalk(t, G, ntp, N) : TileWalk(t, G, N, ntp);
}
__device__ __forceinline__ PTile proj_tile(const TileWalk& w, bool outgoing) {
  PTile r;
  r.c0 = (outgoing ? w.d0 : w.d1) * PTP;
  r.row = outgoing ? w.d1 : w.d0;
  r.b = w.d2;
  return r;
}
__device__ __forceinline__ int64_t proj_pix(const PTile& tl, int pl, int N, bool outgoing) {
  const int cpos = tl.c0 + pl;
  const int pp = outgoing ? tl.row : cpos;
  const int qq = outgoing ? cpos : tl.row;
  return ((int64_t)tl.b * N + pp) * N + qq;
}

// The mask value of local pixel pl, requested as raw bits and converted only where the
// tile is normalised (ProjMask::value). A use of a load's result right behind it makes the
// compiler wait for every load in flight (vmcnt is an in-order counter), so converting the
// mask where it is loaded would also wait for the next tile's x, which is requested just
// before it and meant to arrive during the current tile's work. Pixels past N read pixel
// N - 1 (in bounds) and count as 1.
template <typename T>
struct ProjMask {
  typedef typename std::conditional<sizeof(T) == 2, uint16_t, uint32_t>::type Bits;
  Bits bits = 0;
  bool use = false;  // the caller gave a mask and the pixel is inside the grid
  __device__ __forceinline__ void request(const gnn_trimul_args& a, const PTile& tl, int pl, int N, bool outgoing) {
    use = a.mask != nullptr && tl.c0 + pl < N;
    if (a.mask) {  // uniform
      const int cpos = min(tl.c0 + pl, N - 1);
      const int pp = outgoing ? tl.row : cpos;
      const int qq = outgoing ? cpos : tl.row;
      bits = ((const Bits*)a.mask)[tl.b * a.mask_stride[0] + pp * a.mask_stride[1] + qq * a.mask_stride[2]];
    }
  }
  __device__ __forceinline__ float value() const {
    return use ? TypeOps<T>::to_f32(__builtin_bit_cast(T, bits)) : 1.f;
  }
};

// LayerNorm over the first n of the W channels of a row whose other channels are zeros (the
// caller's padding to a multiple of 32; n = 0 means all): the sums over all W channels give
// mean = sum / n, and the sum of squared deviations from that mean over the n real channels
// is the one over all W minus the padded zeros' (W - n) mean^2.
struct LnWidth {
  float inv_n;  // 1 / n
  float npad;   // W - n
  __device__ __forceinline__ LnWidth(int64_t n, int W) {
    const int nn = n > 0 && n < W ? (int)n : W;
    inv_n = 1.0f / (float)nn;
    npad = (float)(W - nn);
  }
  // the variance from the sum of squared deviations q over all W channels about `mean`
  __device__ __forceinline__ float var(float q, float mean) const { return (q - npad * mean * mean) * inv_n; }
};

// Chunks of x per thread that the tile load must hold: ceil(C / 64), rounded up to 2, 4, 8.
__host__ __device__ inline int proj_xm(int64_t C) { return C <= 128 ? 2 : C <= 256 ? 4 : 8; }

template <typename T, int PREC, int XM>
__global__ __launch_bounds__(PNT, 1) void trimul_proj_kernel(const gnn_trimul_args a, int64_t NP,
                                                             size_t off_a, size_t off_b,
                                                             size_t off_g) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int C = (int)a.C, Ch = (int)a.Ch, N = (int)a.N;
  const ProjLds Ld = proj_lds<T>(C);
  const int ZR = C + lds_pad<T>();
  constexpr int SPT = proj_spt<T>();
  constexpr int ER = proj_er<T>();       // unit staging [32 channels][ER]
  constexpr int EG = 32 + lds_pad<T>();  // gate staging [32 pixels][EG]
  constexpr int KCH = sizeof(T) == 2 ? 8 : 4;  // k-steps of weight fragments held in registers
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  T* zs = reinterpret_cast<T*>(smem_raw + Ld.zs);
  T* ebuf = reinterpret_cast<T*>(smem_raw + Ld.ebuf) + wave * proj_ebuf_elems<T>();
  float2* red = reinterpret_cast<float2*>(smem_raw + Ld.red);
  float* lnw = reinterpret_cast<float*>(smem_raw + Ld.lnw);
  float* lnb = lnw + C;
  float* mk = reinterpret_cast<float*>(smem_raw + Ld.mk);

  const bool outgoing = a.outgoing != 0;
  const int64_t ntiles = (int64_t)a.B * N * ((N + PTP - 1) / PTP);
  typedef PTile Tile;
  auto tile_of = [&](int64_t t) -> Tile { return proj_tile(t, N, outgoing); };
  auto pix_index = [&](const Tile& tl, int pl) -> int64_t { return proj_pix(tl, pl, N, outgoing); };

  // ---- tile load + LayerNorm, thread = (pixel xpl, part xpart) holding chunks xpart + 8j
  const int xpl = tid >> 3, xpart = tid & 7, cpp = C / 8;
  V8 xr[XM];
  ProjMask<T> mreg;
  auto load_x = [&](const Tile& tl) {
    const bool in = tl.c0 + xpl < N;
    const T* src = (const T*)a.x + (in ? pix_index(tl, xpl) * C : 0);
#pragma unroll
    for (int j = 0; j < XM; ++j) {
      const int ci = xpart + 8 * j;
      xr[j] = zero8<T>();
      if (in && ci < cpp) xr[j] = load8(src + 8 * ci);
    }
    mreg.request(a, tl, tid & (PTP - 1), N, outgoing);  // used by the threads tid < PTP
  };
  auto ln_partial = [&]() {
    float s = 0.f, n = 0.f;
#pragma unroll
    for (int j = 0; j < XM; ++j)
      if (xpart + 8 * j < cpp) {
        const f32x8 v = TypeOps<T>::to_f32(xr[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[e];
        n += 8.f;
      }
    const float mean = n > 0.f ? s / n : 0.f;
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < XM; ++j)
      if (xpart + 8 * j < cpp) {
        const f32x8 v = TypeOps<T>::to_f32(xr[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = v[e] - mean;
          m2 += d * d;
        }
      }
    red[xpart * PTP + xpl] = make_float2(mean, m2);
  };
  auto ln_finish = [&]() {
    float2 pr[8];
    float nj[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pr[j] = red[j * PTP + xpl];
      nj[j] = cpp > j ? 8.f * (float)((cpp - j + 7) / 8) : 0.f;  // elements held by part j
    }
    float mean = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) mean += nj[j] * pr[j].x;
    mean /= (float)C;
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = pr[j].x - mean;
      m2 += pr[j].y + nj[j] * d * d;
    }
    float var = m2 / (float)C;
    if (a.ln_in_channels > 0 && a.ln_in_channels < C) {  // padded channels: real-width statistics
      const LnWidth lw(a.ln_in_channels, C);
      const float mean_r = mean * (float)C * lw.inv_n;
      const float dm = mean - mean_r;
      var = lw.var(m2 + (float)C * dm * dm, mean_r);
      mean = mean_r;
    }
    const float rstd = 1.0f / sqrtf(var + a.eps);
#pragma unroll
    for (int j = 0; j < XM; ++j) {
      const int ci = xpart + 8 * j;
      if (ci < cpp) {
        f32x8 v = TypeOps<T>::to_f32(xr[j]);
        const f32x4 w0 = *reinterpret_cast<const f32x4*>(lnw + 8 * ci);
        const f32x4 w1 = *reinterpret_cast<const f32x4*>(lnw + 8 * ci + 4);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(lnb + 8 * ci);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(lnb + 8 * ci + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (v[e] - mean) * rstd * w0[e] + b0[e];
          v[e + 4] = (v[e + 4] - mean) * rstd * w1[e] + b1[e];
        }
        store8(&zs[xpl * ZR + 8 * ci], TypeOps<T>::from_f32(v));
      }
    }
    if (tid < PTP) mk[tid] = mreg.value();
  };

  // ---- projections of one tile
  const int nk = C / 16;
  const int npg = 2 * Ch / 32, ngo = C / 32;
  T* __restrict__ a_cm = (T*)((unsigned char*)a.workspace + off_a);
  T* __restrict__ b_cm = (T*)((unsigned char*)a.workspace + off_b);
  T* __restrict__ gout = (T*)(a.gate ? (unsigned char*)a.gate : (unsigned char*)a.workspace + off_g);
  const T* __restrict__ wp = (const T*)a.p_in_w;
  const T* __restrict__ wg = (const T*)a.g_in_w;
  const T* __restrict__ wgo = (const T*)a.g_out_w;
  V8 wpf[KCH], wgf[KCH], wof[KCH];
  float bp = 0.f, bg = 0.f, bgo[16];
  int wp_unit = -1, wo_unit = -1;

  auto compute = [&](const Tile& tl) {
    // gated projection units: acc = [pixel][channel], row = pixel 32s + 8(r/4) + 4g + r%4,
    // col = channel 32u + l32; staged as [channel][pixel] for 128-byte row stores
    for (int u = wave; u < npg; u += PW) {
      const int ch = 32 * u + l32;
      const T* wprow = wp + (int64_t)ch * C + 8 * g;
      const T* wgrow = wg + (int64_t)ch * C + 8 * g;
      auto load_w = [&](int kc) {
#pragma unroll
        for (int j = 0; j < KCH; ++j)
          if (kc + j < nk) {
            wpf[j] = load8(wprow + 16 * (kc + j));
            wgf[j] = load8(wgrow + 16 * (kc + j));
          }
      };
      if (u != wp_unit) {
        bp = ld_or<T>(a.p_in_b, ch, 0.f);
        bg = ld_or<T>(a.g_in_b, ch, 0.f);
        if (nk <= KCH) load_w(0);
        wp_unit = u;
      }
      for (int s0 = 0; s0 < PSUB; s0 += SPT) {
#pragma unroll
        for (int s2 = 0; s2 < SPT; ++s2) {
          const int s = s0 + s2;
          f32x16 accp, accg;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            accp[r] = bp;
            accg[r] = bg;
          }
          for (int kc = 0; kc < nk; kc += KCH) {
            if (nk > KCH) load_w(kc);
#pragma unroll
            for (int j = 0; j < KCH; ++j) {
              if (kc + j >= nk) break;
              const V8 zf = load8(&zs[(32 * s + l32) * ZR + 16 * (kc + j) + 8 * g]);
              Mma<T, PREC>::step(accp, zf, wpf[j]);
              Mma<T, PREC>::step(accg, zf, wgf[j]);
            }
          }
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int pt = 8 * rg + 4 * g;  // pixel within the sub-tile
            const f32x4 m4 = *reinterpret_cast<const f32x4*>(&mk[32 * s + pt]);
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = accp[4 * rg + e] * sigmoid_acc(accg[4 * rg + e]) * m4[e];
            store4(&ebuf[l32 * ER + 32 * s2 + pt], TypeOps<T>::from_f32(v));
          }
        }
        wave_lds_sync();
        // 16-byte stores, 4 * SPT lanes per channel row of 32 * SPT pixels
#pragma unroll
        for (int i = 0; i < 2 * SPT; ++i) {
          const int c = lane + 64 * i;
          const int crow = c / (4 * SPT), p0 = (c % (4 * SPT)) * 8;
          const int chg = 32 * u + crow;
          T* dst = chg < Ch ? a_cm : b_cm;
          const int chh = chg < Ch ? chg : chg - Ch;
          const int pl = 32 * s0 + p0;
          T* drow = dst + ab_offset<T>((int64_t)tl.b * Ch + chh, tl.row, tl.c0 + pl, N, NP);
          const V8 val = load8(&ebuf[crow * ER + p0]);
          if (tl.c0 + pl + 8 <= N) {
            store8(drow, val);
          } else if (tl.c0 + pl < NP) {  // row tail: pixels N .. NP-1 are written as zeros
            V8 v = val;
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (tl.c0 + pl + e >= N) v[e] = TypeOps<T>::from_f32(0.f);
            store8(drow, v);
          }
        }
        wave_lds_sync();
      }
    }
    // output-gate items (unit uo, sub-tile s): acc = [channel][pixel], row = channel
    // 32uo + 8(r/4) + 4g + r%4, col = pixel 32s + l32; staged as [pixel][channel]
    for (int it = wave; it < ngo * PSUB; it += PW) {
      const int uo = it % ngo, s = it / ngo;
      const int c00 = 32 * uo;
      const T* wrow = wgo + (int64_t)(c00 + l32) * C + 8 * g;
      auto load_w = [&](int kc) {
#pragma unroll
        for (int j = 0; j < KCH; ++j)
          if (kc + j < nk) wof[j] = load8(wrow + 16 * (kc + j));
      };
      if (uo != wo_unit) {
#pragma unroll
        for (int r = 0; r < 16; ++r) bgo[r] = ld_or<T>(a.g_out_b, c00 + 8 * (r / 4) + 4 * g + (r % 4), 0.f);
        if (nk <= KCH) load_w(0);
        wo_unit = uo;
      }
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = bgo[r];
      for (int kc = 0; kc < nk; kc += KCH) {
        if (nk > KCH) load_w(kc);
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
          if (kc + j >= nk) break;
          const V8 zf = load8(&zs[(32 * s + l32) * ZR + 16 * (kc + j) + 8 * g]);
          Mma<T, PREC>::step(acc, wof[j], zf);
        }
      }
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = sigmoid_acc(acc[4 * rg + e]);
        store4(&ebuf[l32 * EG + 8 * rg + 4 * g], TypeOps<T>::from_f32(v));
      }
      wave_lds_sync();
      // 16-byte stores, 4 lanes per 32-channel pixel row segment
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = lane + 64 * i;
        const int px = c / 4, k0 = (c % 4) * 8;
        const int pl = 32 * s + px;
        if (tl.c0 + pl < N) store8(gout + pix_index(tl, pl) * C + c00 + k0, load8(&ebuf[px * EG + k0]));
      }
      wave_lds_sync();
    }
  };

  for (int c = tid; c < C; c += PNT) {
    lnw[c] = ld_or<T>(a.ln_in_w, c, 1.f);
    lnb[c] = ld_or<T>(a.ln_in_b, c, 0.f);
  }
  int64_t t = blockIdx.x;
  if (t >= ntiles) return;  // uniform over the workgroup
  Tile cur = tile_of(t);
  load_x(cur);
  ln_partial();
  __syncthreads();
  ln_finish();
  __syncthreads();
  for (; t < ntiles; t += gridDim.x) {
    const int64_t tn = t + gridDim.x;
    const bool has_next = tn < ntiles;  // uniform over the workgroup
    Tile nxt = cur;
    if (has_next) {
      nxt = tile_of(tn);
      load_x(nxt);
    }
    compute(cur);
    if (has_next) ln_partial();
    __syncthreads();  // z / mask of this tile consumed, partials of the next one published
    if (has_next) ln_finish();
    __syncthreads();
    cur = nxt;
  }
}

// ---- stage 1, fp32 under bf16x3: C = CK in {64, 128}, c_hidden <= 128 ---------------------
// The generic kernel's tile walk, two-barrier LayerNorm and epilogues, with every MFMA
// operand split into bf16 hi / lo halves once instead of at each product: z where the
// LayerNorm writes it to LDS (two bf16 planes), a wave's projection weights (its one unit:
// 32 rows of p_in and of g_in, 2 Ch / 32 <= PW) when the launch starts (registers, for the
// whole launch) and the output-gate weights when the workgroup starts (two bf16 planes in
// LDS). The MFMA loops then only read fragments; a product is lo*hi + hi*lo + hi*hi in fp32
// accumulators. Accumulators start at zero and the biases join after the product.
template <int CK>
struct ProjX3Lds {
  static constexpr int ZB = CK + 8;  // bf16 per z / gate-weight row (16 B of padding)
  static constexpr int ER = 32 + 4;  // fp32 per staging row
  static constexpr size_t zh = 0;
  static constexpr size_t zl = zh + (size_t)PTP * ZB * 2;
  static constexpr size_t woh = zl + (size_t)PTP * ZB * 2;
  static constexpr size_t wol = woh + (size_t)CK * ZB * 2;
  static constexpr size_t ebuf = wol + (size_t)CK * ZB * 2;
  static constexpr size_t red = ebuf + (size_t)PW * 32 * ER * 4;
  static constexpr size_t lnw = red + 8 * (size_t)PTP * 8;
  static constexpr size_t lnb = lnw + CK * 4;
  static constexpr size_t bgo = lnb + CK * 4;
  static constexpr size_t mk = bgo + CK * 4;
  static constexpr size_t total = mk + PTP * 4;
};

__device__ __forceinline__ f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// FIXED (CK = c_hidden = 128, 128 N NP bytes below 2^31): every wave owns one projection unit
// and one gate item, the next tile's x is requested unconditionally (the last tile requests
// itself again) and the a / b / g stores are buffer stores over ranges whose ends drop the
// lanes past the row, so no memory access sits in a branch: with one, the compiler's
// memory-counter waits at the join count the path without it, and the waits for the next
// tile's loads also wait for the stores issued after them.
template <int CK, bool FIXED>
__global__ __launch_bounds__(PNT, 1) void trimul_proj_x3_kernel(const gnn_trimul_args a, int64_t NP,
                                                                size_t off_a, size_t off_b, size_t off_g) {
  typedef ProjX3Lds<CK> S;
  constexpr int XM = CK / 64;  // 8-channel chunks of x per thread
  constexpr int NK = CK / 16;  // k-steps
  constexpr int ZB = S::ZB, ER = S::ER;
  constexpr int NGO = CK / 32;  // output-gate units
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* zh = reinterpret_cast<bf16*>(smem_raw + S::zh);
  bf16* zl = reinterpret_cast<bf16*>(smem_raw + S::zl);
  bf16* woh = reinterpret_cast<bf16*>(smem_raw + S::woh);
  bf16* wol = reinterpret_cast<bf16*>(smem_raw + S::wol);
  float2* red = reinterpret_cast<float2*>(smem_raw + S::red);
  float* lnw = reinterpret_cast<float*>(smem_raw + S::lnw);
  float* lnb = reinterpret_cast<float*>(smem_raw + S::lnb);
  float* bgo = reinterpret_cast<float*>(smem_raw + S::bgo);
  float* mk = reinterpret_cast<float*>(smem_raw + S::mk);
  const int Ch = (int)a.Ch, N = (int)a.N;
  // wave from readfirstlane: the buffer-store resources built from it are then scalar (a
  // resource the compiler cannot prove uniform costs a loop over its distinct values per store)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l32 = lane & 31,
            g = lane >> 5;
  float* ebuf = reinterpret_cast<float*>(smem_raw + S::ebuf) + wave * 32 * ER;
  const bool outgoing = a.outgoing != 0;
  const int64_t ntiles = (int64_t)a.B * N * ((N + PTP - 1) / PTP);

  // ---- once per workgroup: LayerNorm parameters, gate-out weights (split) and biases
  for (int c = tid; c < CK; c += PNT) {
    lnw[c] = ld_or<float>(a.ln_in_w, c, 1.f);
    lnb[c] = ld_or<float>(a.ln_in_b, c, 0.f);
    bgo[c] = ld_or<float>(a.g_out_b, c, 0.f);
  }
  for (int c = tid; c < CK * CK / 8; c += PNT) {
    const int row = c / (CK / 8), k0 = (c % (CK / 8)) * 8;
    bf16x8 hi, lo;
    split_bf16(load8((const float*)a.g_out_w + (int64_t)row * CK + k0), hi, lo);
    store8(&woh[row * ZB + k0], hi);
    store8(&wol[row * ZB + k0], lo);
  }
  // ---- once per wave: its projection unit's weights, split (B operand: column = channel
  // 32 * wave + l32, k = 16 kk + 8 g + e)
  static_assert(!FIXED || (CK == 128 && NGO * PSUB == PW), "FIXED: one unit and one gate item per wave");
  const int npg = 2 * Ch / 32;
  const bool has_unit = FIXED || wave < npg;  // uniform over the wave
  bf16x8 wph[NK], wpl[NK], wgh[NK], wgl[NK];
  float bp = 0.f, bg = 0.f;
  {
    const int ch = has_unit ? 32 * wave + l32 : 0;
    const float* wprow = (const float*)a.p_in_w + (int64_t)ch * CK + 8 * g;
    const float* wgrow = (const float*)a.g_in_w + (int64_t)ch * CK + 8 * g;
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      split_bf16(load8(wprow + 16 * k), wph[k], wpl[k]);
      split_bf16(load8(wgrow + 16 * k), wgh[k], wgl[k]);
    }
    bp = ld_or<float>(a.p_in_b, ch, 0.f);
    bg = ld_or<float>(a.g_in_b, ch, 0.f);
  }

  // ---- tile load + LayerNorm: thread = (pixel xpl, part xpart) holding chunks xpart + 8j.
  // Pixels past N read pixel N - 1 (in bounds); their results are never stored.
  const int xpl = tid >> 3, xpart = tid & 7;
  f32x8 xr[XM];
  ProjMask<float> mreg;
  auto load_x = [&](const PTile& tl) {
    const float* src = (const float*)a.x + proj_pix(tl, min(xpl, N - 1 - tl.c0), N, outgoing) * CK;
#pragma unroll
    for (int j = 0; j < XM; ++j) xr[j] = load8(src + 8 * (xpart + 8 * j));
    mreg.request(a, tl, tid & (PTP - 1), N, outgoing);  // used by the threads tid < PTP
  };
  auto ln_partial = [&]() {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < XM; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) s += xr[j][e];
    const float mean = s * (1.0f / (8 * XM));
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < XM; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = xr[j][e] - mean;
        m2 += d * d;
      }
    red[xpart * PTP + xpl] = make_float2(mean, m2);
  };
  const LnWidth lw(a.ln_in_channels, CK);
  auto ln_finish = [&]() {
    float2 pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pr[j] = red[j * PTP + xpl];
    float mean = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) mean += pr[j].x;
    mean *= 0.125f;  // every part holds 8 * XM channels
    float m2 = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = pr[j].x - mean;
      m2 += pr[j].y + (float)(8 * XM) * d * d;
    }
    // real-width statistics when the channels past ln_in_channels are padding zeros
    const float mean_r = mean * (float)CK * lw.inv_n;
    const float dm = mean - mean_r;
    const float var = lw.var(m2 + (float)CK * dm * dm, mean_r);
    const float rstd = 1.0f / sqrtf(var + a.eps);
#pragma unroll
    for (int j = 0; j < XM; ++j) {
      const int ci = xpart + 8 * j;
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(lnw + 8 * ci);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(lnw + 8 * ci + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(lnb + 8 * ci);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(lnb + 8 * ci + 4);
      f32x8 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = (xr[j][e] - mean_r) * rstd * w0[e] + b0[e];
        v[e + 4] = (xr[j][e + 4] - mean_r) * rstd * w1[e] + b1[e];
      }
      bf16x8 hi, lo;
      split_bf16(v, hi, lo);
      store8(&zh[xpl * ZB + 8 * ci], hi);
      store8(&zl[xpl * ZB + 8 * ci], lo);
    }
    if (tid < PTP) mk[tid] = mreg.value();
  };

  float* __restrict__ a_cm = (float*)((unsigned char*)a.workspace + off_a);
  float* __restrict__ b_cm = (float*)((unsigned char*)a.workspace + off_b);
  float* __restrict__ gout = (float*)(a.gate ? (unsigned char*)a.gate : (unsigned char*)a.workspace + off_g);

  auto compute = [&](const PTile& tl) {
    // gated projection unit: acc = [pixel][channel], row = pixel 32s + 8(r/4) + 4g + r%4,
    // col = channel 32 * wave + l32; staged as [channel][pixel] for 128-byte row stores
    if (has_unit) {
#pragma unroll FIXED ? PSUB : 1  // FIXED: the store count behind the x loads is then known
      for (int s = 0; s < PSUB; ++s) {
        f32x16 accp, accg;
#pragma unroll
        for (int r = 0; r < 16; ++r) accp[r] = accg[r] = 0.f;
        if (FIXED) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int k = 0; k < NK; ++k) {
          const int o = (32 * s + l32) * ZB + 16 * k + 8 * g;
          const bf16x8 h = load8(&zh[o]), l = load8(&zl[o]);
          accp = mfma_bf16(l, wph[k], accp);
          accg = mfma_bf16(l, wgh[k], accg);
          accp = mfma_bf16(h, wpl[k], accp);
          accg = mfma_bf16(h, wgl[k], accg);
          accp = mfma_bf16(h, wph[k], accp);
          accg = mfma_bf16(h, wgh[k], accg);
        }
        if (FIXED) __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int pt = 8 * rg + 4 * g;  // pixel within the sub-tile
          const f32x4 m4 = *reinterpret_cast<const f32x4*>(&mk[32 * s + pt]);
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = (accp[4 * rg + e] + bp) * sigmoid_acc(accg[4 * rg + e] + bg) * m4[e];
          store4(&ebuf[l32 * ER + pt], v);
        }
        wave_lds_sync();
        if constexpr (FIXED) {
          // the unit's 32 channel planes all belong to a or all to b (c_hidden = 128): one
          // buffer range over them; lanes past the padded row are dropped
          const bool in_a = 32 * wave < Ch;
          float* base = (in_a ? a_cm : b_cm) + ab_offset<float>((int64_t)tl.b * Ch + 32 * wave - (in_a ? 0 : Ch), 0, 0, N, NP);
          const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(base, (int)(32 * (int64_t)N * NP * sizeof(float)));
          const bool tail_tile = tl.c0 + PTP > N;  // uniform
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int c = lane + 64 * i;
            const int crow = c / 4, p0 = (c % 4) * 8;
            const int k = tl.c0 + 32 * s + p0;
            f32x8 val = load8(&ebuf[crow * ER + p0]);
            if (tail_tile) {  // row tail: pixels N .. NP-1 are written as zeros
#pragma unroll
              for (int e = 0; e < 8; ++e)
                if (k + e >= N) val[e] = 0.f;
            }
            const uint32_t off = k < NP ? (uint32_t)((crow * N + tl.row) * (int)NP + k) * (uint32_t)sizeof(float) : BUFFER_OOB;
            buffer_store(f32x4{val[0], val[1], val[2], val[3]}, rs, off);
            buffer_store(f32x4{val[4], val[5], val[6], val[7]}, rs, off + 16u);
          }
          wave_lds_sync();
          continue;
        }
        // 32-byte stores, 4 lanes per channel row of 32 pixels
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int c = lane + 64 * i;
          const int crow = c / 4, p0 = (c % 4) * 8;
          const int chg = 32 * wave + crow;
          float* dst = chg < Ch ? a_cm : b_cm;
          const int chh = chg < Ch ? chg : chg - Ch;
          const int pl = 32 * s + p0;
          float* drow = dst + ab_offset<float>((int64_t)tl.b * Ch + chh, tl.row, tl.c0 + pl, N, NP);
          f32x8 val = load8(&ebuf[crow * ER + p0]);
          if (tl.c0 + pl + 8 <= N) {
            store8(drow, val);
          } else if (tl.c0 + pl < NP) {  // row tail: pixels N .. NP-1 are written as zeros
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (tl.c0 + pl + e >= N) val[e] = 0.f;
            store8(drow, val);
          }
        }
        wave_lds_sync();
      }
    }
    // output-gate items (unit uo, sub-tile s): acc = [channel][pixel], row = channel
    // 32uo + 8(r/4) + 4g + r%4, col = pixel 32s + l32; staged as [pixel][channel]
#pragma unroll 1
    for (int it = wave; FIXED || it < NGO * PSUB; it += PW) {  // FIXED: item `wave`, always
      const int uo = it % NGO, s = it / NGO;
      const int c00 = 32 * uo;
      f32x16 accx, acch;  // cross terms, hi * hi
#pragma unroll
      for (int r = 0; r < 16; ++r) accx[r] = acch[r] = 0.f;
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const int ow = (c00 + l32) * ZB + 16 * k + 8 * g;
        const int oz = (32 * s + l32) * ZB + 16 * k + 8 * g;
        const bf16x8 whf = load8(&woh[ow]), wlf = load8(&wol[ow]);
        const bf16x8 zhf = load8(&zh[oz]), zlf = load8(&zl[oz]);
        accx = mfma_bf16(wlf, zhf, accx);
        acch = mfma_bf16(whf, zhf, acch);
        accx = mfma_bf16(whf, zlf, accx);
      }
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int c0 = c00 + 8 * rg + 4 * g;
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bgo[c0]);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = sigmoid_acc(accx[4 * rg + e] + acch[4 * rg + e] + b4[e]);
        store4(&ebuf[l32 * ER + 8 * rg + 4 * g], v);
      }
      wave_lds_sync();
      if constexpr (FIXED) {
        // one buffer range from the tile's first pixel to the end of its last one (pixel
        // stride CK outgoing, N CK incoming): the lanes of pixels past N fall outside it
        const int pstride = outgoing ? CK : N * CK;
        const int npix = min(N - tl.c0, PTP);
        const __amdgpu_buffer_rsrc_t rs =
            buffer_rsrc(gout + proj_pix(tl, 0, N, outgoing) * CK, ((npix - 1) * pstride + CK) * (int)sizeof(float));
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int c = lane + 64 * i;
          const int px = c / 4, k0 = (c % 4) * 8;
          const uint32_t off = (uint32_t)((32 * s + px) * pstride + c00 + k0) * (uint32_t)sizeof(float);
          const f32x8 val = load8(&ebuf[px * ER + k0]);
          buffer_store(f32x4{val[0], val[1], val[2], val[3]}, rs, off);
          buffer_store(f32x4{val[4], val[5], val[6], val[7]}, rs, off + 16u);
        }
        wave_lds_sync();
        break;
      }
      // 32-byte stores, 4 lanes per 32-channel pixel row segment
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = lane + 64 * i;
        const int px = c / 4, k0 = (c % 4) * 8;
        const int pl = 32 * s + px;
        if (tl.c0 + pl < N) store8(gout + proj_pix(tl, pl, N, outgoing) * CK + c00 + k0, load8(&ebuf[px * ER + k0]));
      }
      wave_lds_sync();
    }
  };

  int64_t t = blockIdx.x;
  if (t >= ntiles) return;  // uniform over the workgroup
  PTile cur = proj_tile(t, N, outgoing);
  load_x(cur);
  ln_partial();
  __syncthreads();  // partials, LayerNorm parameters and gate weights published
  ln_finish();
  __syncthreads();
  TileWalk walk = proj_walk(t + gridDim.x, gridDim.x, N, outgoing);  // the next tile
  for (; t < ntiles; t += gridDim.x) {
    const int64_t tn = t + gridDim.x;
    const bool has_next = tn < ntiles;  // uniform over the workgroup
    PTile nxt = cur;
    const PTile wt = proj_tile(walk, outgoing);
    walk.step();
    if constexpr (FIXED) {
      nxt = has_next ? wt : cur;
      load_x(nxt);
      compute(cur);
      ln_partial();
      __syncthreads();  // z / mask of this tile consumed, partials of the next one published
      ln_finish();
      __syncthreads();
      cur = nxt;
      continue;
    }
    if (has_next) {
      nxt = wt;
      load_x(nxt);
    }
    compute(cur);
    if (has_next) ln_partial();
    __syncthreads();  // z / mask of this tile consumed, partials of the next one published
    if (has_next) ln_finish();
    __syncthreads();
    cur = nxt;
  }
}

// ---- stage 1, fixed-width variant: 16-bit types with C = CK in {64, 128} ----------------
// Same work split and tile order as trimul_proj_kernel, with C known at compile time so the
// k loops unroll and a wave's gate MFMAs and second sub-tile can overlap the first
// sub-tile's epilogue. Differences: the output-gate weights and biases live in LDS (loaded
// once per workgroup), gate items stage through a tile of their own, the z tile is
// double-buffered and the LayerNorm is wave-local (the 8 threads of a pixel are lanes of
// one wave and reduce with cross-lane shuffles: the same two-pass mean / variance), so a
// tile costs one barrier. A wave's gate item covers one of the two 32-pixel sub-tiles of its
// projection unit, so the unit visits that sub-tile first and the gate MFMAs reuse its z
// fragments (3 LDS fragment reads per k-step for 5 MFMAs). Accumulators start at zero and
// the biases join in the epilogue, as the reference's linear layers add them (after the
// product); the gates fold theirs into the exp2 argument. A tile whose mask values are all
// one skips the mask multiply.
// Column swizzle of the epilogue staging tiles: rows 16 .. 31 swap their 16-column halves,
// so that rows r and r + 16 (the same banks with a pitch of 8 mod 16 elements) do not collide.
#ifndef GNN_PROJ_EBSW
#define GNN_PROJ_EBSW 1
#endif
__device__ __forceinline__ int EBSW(int row) { return GNN_PROJ_EBSW ? (row & 16) : 0; }

template <int CK>
struct ProjFastLds {
  static constexpr int ZR = CK + 8;  // z and gate-weight row pitch (16-bit elements)
  static constexpr int ER = 72;      // unit staging [32 channels][64 pixels + 8]
  static constexpr int EG = 40;      // gate staging [32 pixels][32 channels + 8]
  static constexpr size_t zs = 0;                                  // [2][PTP][ZR]
  static constexpr size_t wgo = zs + 2 * (size_t)PTP * ZR * 2;     // [CK][ZR]
  static constexpr size_t ebuf = wgo + (size_t)CK * ZR * 2;        // [PW][32][ER]
  static constexpr size_t gbuf = ebuf + (size_t)PW * 32 * ER * 2;  // [PW][32][EG]
  static constexpr size_t bgo = gbuf + (size_t)PW * 32 * EG * 2;   // [CK] fp32
  static constexpr size_t lnw = bgo + (size_t)CK * 4;              // gamma, beta [2][CK] fp32
  static constexpr size_t mk = lnw + 2 * (size_t)CK * 4;           // [2][PTP] fp32
  static constexpr size_t mk1 = mk + 2 * (size_t)PTP * 4;          // [2] int: tile mask all ones
  static constexpr size_t total = mk1 + 16;
};

template <typename T, int CK, int CHK>  // CHK: c_hidden at compile time, 0 = from the arguments
__global__ __launch_bounds__(PNT, 1) void trimul_proj_fast_kernel(const gnn_trimul_args a, int64_t NP,
                                                                  size_t off_a, size_t off_b,
                                                                  size_t off_g) {
  static_assert(sizeof(T) == 2 && (CK == 64 || CK == 128), "fixed-width projection: 16-bit, C in {64, 128}");
  typedef typename TypeOps<T>::V8 V8;
  typedef ProjFastLds<CK> LD;
  constexpr int ZR = LD::ZR, ER = LD::ER, EG = LD::EG;
  constexpr int NKS = CK / 16;  // k-steps
  constexpr int XMF = CK / 64;  // x chunks per thread (8 threads per pixel)
  constexpr int NGI = CK / 16;  // gate items (CK / 32 units x 2 sub-tiles), at most one per wave
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int Ch = CHK ? CHK : (int)a.Ch, N = (int)a.N;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  // the wave index as a scalar, so that unit and gate-item addresses and the buffer
  // resources built from them stay in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  T* zs = reinterpret_cast<T*>(smem_raw + LD::zs);
  T* wgo_s = reinterpret_cast<T*>(smem_raw + LD::wgo);
  T* ebuf = reinterpret_cast<T*>(smem_raw + LD::ebuf) + wave * 32 * ER;
  T* gbuf = reinterpret_cast<T*>(smem_raw + LD::gbuf) + wave * 32 * EG;
  float* bgo_s = reinterpret_cast<float*>(smem_raw + LD::bgo);
  float* lnw = reinterpret_cast<float*>(smem_raw + LD::lnw);
  float* lnb = lnw + CK;
  float* mk = reinterpret_cast<float*>(smem_raw + LD::mk);
  int* mk1 = reinterpret_cast<int*>(smem_raw + LD::mk1);
  const LnWidth lnw_in(a.ln_in_channels, CK);
  const bool outgoing = a.outgoing != 0;
  const int64_t ntiles = (int64_t)a.B * N * ((N + PTP - 1) / PTP);
  constexpr float NLOG2E = -1.4426950408889634f;

  // ---- per-workgroup constants
  {
    const T* wgo = (const T*)a.g_out_w;
    for (int c = tid; c < CK * CK / 8; c += PNT) {
      const int r = c / (CK / 8), k0 = (c % (CK / 8)) * 8;
      store8(&wgo_s[r * ZR + k0], load8(wgo + r * CK + k0));
    }
    for (int c = tid; c < CK; c += PNT) {
      bgo_s[c] = ld_or<T>(a.g_out_b, c, 0.f) * NLOG2E;  // the exp2 argument's bias term
      lnw[c] = ld_or<T>(a.ln_in_w, c, 1.f);
      lnb[c] = ld_or<T>(a.ln_in_b, c, 0.f);
    }
  }

  // ---- tile load + wave-local LayerNorm: thread = (pixel xpl, part xpart), chunks xpart + 8j
  const int xpl = tid >> 3, xpart = tid & 7;
  // Pixels past N load pixel N - 1 (finite values; their z only reaches their own outputs,
  // which are stored as zeros or not at all), so the loads need no select and never wait
  // for the previous tile's loads into the same registers.
  auto load_x = [&](V8 (&xr)[XMF], ProjMask<T>& mreg, const PTile& tl) {
    const T* src = (const T*)a.x + proj_pix(tl, min(xpl, N - 1 - tl.c0), N, outgoing) * CK;
#pragma unroll
    for (int j = 0; j < XMF; ++j) xr[j] = load8(src + 8 * (xpart + 8 * j));
    mreg.request(a, tl, tid & (PTP - 1), N, outgoing);  // used by the threads tid < PTP
  };
  auto ln_store = [&](const V8 (&xr)[XMF], const ProjMask<T>& mreg, int nb) {
    f32x8 v[XMF];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < XMF; ++j) {
      v[j] = TypeOps<T>::to_f32(xr[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[j][e];
    }
    s = sum8_dpp(s);
    const float mean = s * lnw_in.inv_n;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < XMF; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[j][e] - mean;
        q += d * d;
      }
    q = sum8_dpp(q);
    const float rstd = __builtin_amdgcn_rsqf(lnw_in.var(q, mean) + a.eps);  // as torch's rsqrt
#pragma unroll
    for (int j = 0; j < XMF; ++j) {
      const int k = 8 * (xpart + 8 * j);
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(lnw + k);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(lnw + k + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(lnb + k);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(lnb + k + 4);
      f32x8 z;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        z[e] = (v[j][e] - mean) * rstd * w0[e] + b0[e];
        z[e + 4] = (v[j][e + 4] - mean) * rstd * w1[e] + b1[e];
      }
      store8(&zs[(nb * PTP + xpl) * ZR + k], TypeOps<T>::from_f32(z));
    }
    if (tid < PTP) {  // wave 0 (PTP = 64): the tile's mask values and whether all are one
      const float mv = mreg.value();
      mk[nb * PTP + tid] = mv;
      const bool all1 = __ballot(mv != 1.f) == 0;
      if (tid == 0) mk1[nb] = all1;
    }
  };

  // ---- projections of one tile
  const int npg = 2 * Ch / 32;
  T* __restrict__ a_cm = (T*)((unsigned char*)a.workspace + off_a);
  T* __restrict__ b_cm = (T*)((unsigned char*)a.workspace + off_b);
  T* __restrict__ gout = (T*)(a.gate ? (unsigned char*)a.gate : (unsigned char*)a.workspace + off_g);
  V8 wpf[NKS], wgf[NKS];
  float bp = 0.f, bg = 0.f;
  int wp_unit = -1;
  // FIXED (c_hidden = 128): wave w owns projection unit w for the whole launch. Its weights
  // are loaded (and waited for) before the tile loop, the tile loop has no unit loop, and
  // the a / b / g stores are buffer stores issued unconditionally. With a load or a store in
  // a branch of the tile loop the compiler's memory-counter waits take the count of the
  // path without it: the k loop then waited for the next tile's x and the next tile's
  // LayerNorm for the stores just issued.
  constexpr bool FIXED = CHK != 0 && 2 * CHK == 32 * PW;
  if constexpr (FIXED) {
    const int ch = 32 * wave + l32;
    const T* wprow = (const T*)a.p_in_w + (int64_t)ch * CK + 8 * g;
    const T* wgrow = (const T*)a.g_in_w + (int64_t)ch * CK + 8 * g;
#pragma unroll
    for (int k = 0; k < NKS; ++k) {
      wpf[k] = load8(wprow + 16 * k);
      wgf[k] = load8(wgrow + 16 * k);
    }
    bp = ld_or<T>(a.p_in_b, ch, 0.f);
    bg = ld_or<T>(a.g_in_b, ch, 0.f) * NLOG2E;  // the exp2 argument's bias term
    wp_unit = wave;
    // consumed here, so that no load before the loop is still counted inside it
#pragma unroll
    for (int k = 0; k < NKS; ++k) asm volatile("" ::"v"(wpf[k]), "v"(wgf[k]));
    asm volatile("" ::"v"(bp), "v"(bg));
  }
  // FIXED (C = c_hidden = 128): 8 gate items for 8 waves, so every wave has one, and the gate
  // stores are unconditional (a store under a condition makes the next tile's LayerNorm wait
  // for the unit's stores as well)
  static_assert(!FIXED || NGI == PW, "FIXED: one gate item per wave");
  const bool has_go = FIXED || wave < NGI;
  const int uo = wave % (CK / 32), so = wave / (CK / 32);  // this wave's gate item

  // the unit's sub-tiles in the order (so, 1 - so): the gate item's sub-tile first
  const int s_first = has_go ? so : 0;

  // global stores of a staged projection unit / gate item (16-byte stores from the wave's
  // staging tile)
  auto store_unit = [&](const PTile& tl, int u) {
    // 8 lanes per 64-pixel channel row: lane = (channel row lane / 8 + 8 i, pixels
    // 8 (lane % 8) ..). c_hidden is a multiple of 32, so the unit's 32 channels all belong to
    // a or all to b, and store i is store 0 moved by 8 channel planes.
    const int crow0 = lane >> 3, p0 = (lane & 7) * 8;
    const bool in_a = 32 * u < Ch;
    const int chh0 = 32 * u + crow0 - (in_a ? 0 : Ch);
    const int64_t pstep = ab_offset<T>(8, 0, 0, N, NP);  // 8 channel planes
    const bool full = tl.c0 + p0 + 8 <= N, tail = !full && tl.c0 + p0 < NP;
    if constexpr (FIXED) {
      // store i covers channel planes 8i .. 8i + 7 of the unit: one buffer range each (the
      // launcher keeps 8 planes below 2^31 bytes); lanes past the padded row are dropped
      T* base = (in_a ? a_cm : b_cm) + ab_offset<T>((int64_t)tl.b * Ch + 32 * u - (in_a ? 0 : Ch), 0, 0, N, NP);
      // ab_offset(crow0, row, k) in 32 bits (below 8 planes, so below 2^30 elements)
      const int k = tl.c0 + p0;
      const uint32_t off = k < NP ? ((((crow0 * (int)(NP >> 5) + (k >> 5)) * N + tl.row) << 5) + (k & 31)) *
                                        (uint32_t)sizeof(T)
                                  : BUFFER_OOB;
      const bool tail_tile = tl.c0 + PTP > N;  // uniform
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        V8 v = load8(&ebuf[(crow0 + 8 * i) * ER + (p0 ^ EBSW(crow0 + 8 * i))]);
        if (tail_tile) {  // row tail: pixels N .. NP-1 are written as zeros
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (k + e >= N) v[e] = TypeOps<T>::from_f32(0.f);
        }
        buffer_store(v, buffer_rsrc(base + i * pstep, (int)(pstep * (int64_t)sizeof(T))), off);
      }
      return;
    }
    T* drow = (in_a ? a_cm : b_cm) + ab_offset<T>((int64_t)tl.b * Ch + chh0, tl.row, tl.c0 + p0, N, NP);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const V8 val = load8(&ebuf[(crow0 + 8 * i) * ER + (p0 ^ EBSW(crow0 + 8 * i))]);
      if (full) {
        store8(drow + i * pstep, val);
      } else if (tail) {  // row tail: pixels N .. NP-1 are written as zeros
        V8 v = val;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (tl.c0 + p0 + e >= N) v[e] = TypeOps<T>::from_f32(0.f);
        store8(drow + i * pstep, v);
      }
    }
  };
  auto store_gate = [&](const PTile& tl) {
    // 4 lanes per 32-channel pixel row segment; store 1 is store 0 moved by 16 pixels along
    // the tile (a column step outgoing, a row step incoming)
    const int px = lane >> 2, k0 = (lane & 3) * 8, pl = 32 * so + px;
    const int64_t step16 = (outgoing ? 16 : 16 * (int64_t)N) * CK;
    if constexpr (FIXED) {
      // one buffer range from the tile's first pixel to the end of its last one (pixel
      // stride CK outgoing, N CK incoming): the lanes of pixels past N fall outside it
      const int pstride = outgoing ? CK : N * CK;  // below 2^31 / 128 (the launcher's bound on N)
      const int npix = min(N - tl.c0, PTP);
      const __amdgpu_buffer_rsrc_t rs =
          buffer_rsrc(gout + proj_pix(tl, 0, N, outgoing) * CK, ((npix - 1) * pstride + CK) * (int)sizeof(T));
      const uint32_t off = (uint32_t)(pl * pstride + 32 * uo + k0) * (uint32_t)sizeof(T);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        buffer_store(load8(&gbuf[(px + 16 * i) * EG + (k0 ^ EBSW(px + 16 * i))]), rs,
                     off + (uint32_t)(16 * i * pstride) * (uint32_t)sizeof(T));
      return;
    }
    T* dst = gout + proj_pix(tl, pl, N, outgoing) * CK + 32 * uo + k0;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (tl.c0 + pl + 16 * i < N) store8(dst + i * step16, load8(&gbuf[(px + 16 * i) * EG + (k0 ^ EBSW(px + 16 * i))]));
  };

  auto compute = [&](const PTile& tl, int cb) {
    const T* z = zs + cb * PTP * ZR;
    const float* m = mk + cb * PTP;
    const bool all1 = mk1[cb] != 0;
    // gate item: acc = [channel][pixel], row = channel 32uo + 8(r/4) + 4g + r%4, col = pixel
    // 32so + l32 (zero-initialised; bias in the epilogue)
    f32x16 accgo;
#pragma unroll
    for (int r = 0; r < 16; ++r) accgo[r] = 0.f;
    const T* zrow0 = z + (32 * s_first + l32) * ZR + 8 * g;        // sub-tile s_first
    const T* zrow1 = z + (32 * (1 - s_first) + l32) * ZR + 8 * g;  // the other one
    const T* wgrow_s = wgo_s + (32 * uo + l32) * ZR + 8 * g;
    bool go_done = !has_go;
    // gated projection units: acc = [pixel][channel], row = pixel 32s + 8(r/4) + 4g + r%4,
    // col = channel 32u + l32; staged as [channel][pixel] for 128-byte row stores
    const int u_end = FIXED ? wave + 1 : npg;  // FIXED: exactly unit `wave`
    for (int u = wave; u < u_end; u += PW) {
      const int ch = 32 * u + l32;
      if (!FIXED && u != wp_unit) {
        const T* wprow = (const T*)a.p_in_w + (int64_t)ch * CK + 8 * g;
        const T* wgrow = (const T*)a.g_in_w + (int64_t)ch * CK + 8 * g;
#pragma unroll
        for (int k = 0; k < NKS; ++k) {
          wpf[k] = load8(wprow + 16 * k);
          wgf[k] = load8(wgrow + 16 * k);
        }
        bp = ld_or<T>(a.p_in_b, ch, 0.f);
        bg = ld_or<T>(a.g_in_b, ch, 0.f) * NLOG2E;  // the exp2 argument's bias term
        wp_unit = u;
      }
      f32x16 accp[PSUB], accg[PSUB];
#pragma unroll
      for (int s = 0; s < PSUB; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          accp[s][r] = 0.f;
          accg[s][r] = 0.f;
        }
      auto kloop = [&](auto with_go) {
#pragma unroll
        for (int k = 0; k < NKS; ++k) {
          const V8 z0 = load8(zrow0 + 16 * k);
          const V8 z1 = load8(zrow1 + 16 * k);
          Mma<T, PREC_NATIVE>::step(accp[0], z0, wpf[k]);
          Mma<T, PREC_NATIVE>::step(accg[0], z0, wgf[k]);
          if constexpr (decltype(with_go)::value) Mma<T, PREC_NATIVE>::step(accgo, load8(wgrow_s + 16 * k), z0);
          Mma<T, PREC_NATIVE>::step(accp[1], z1, wpf[k]);
          Mma<T, PREC_NATIVE>::step(accg[1], z1, wgf[k]);
        }
      };
      // the matrix pipe first: a wave that reaches its MFMAs takes the pipe ahead of the
      // other wave of its SIMD, which then runs its epilogue beside them (0.5-1 us)
      __builtin_amdgcn_s_setprio(1);
      if (!go_done) {
        kloop(std::true_type{});
        go_done = true;
      } else {
        kloop(std::false_type{});
      }
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int s = 0; s < PSUB; ++s) {
        const int sub = s == 0 ? s_first : 1 - s_first;
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int pt = 32 * sub + 8 * rg + 4 * g;  // pixel within the tile
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = (accp[s][4 * rg + e] + bp) *
                   __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(accg[s][4 * rg + e], NLOG2E, bg)));
          if (!all1) {
            const f32x4 m4 = *reinterpret_cast<const f32x4*>(&m[pt]);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] *= m4[e];
          }
          store4(&ebuf[l32 * ER + (pt ^ EBSW(l32))], TypeOps<T>::from_f32(v));
        }
      }
      wave_lds_sync();
      store_unit(tl, u);
      wave_lds_sync();
    }
    if (!go_done) {  // no projection unit this tile: the gate item on its own
#pragma unroll
      for (int k = 0; k < NKS; ++k) Mma<T, PREC_NATIVE>::step(accgo, load8(wgrow_s + 16 * k), load8(zrow0 + 16 * k));
    }
    if (has_go) {
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const f32x4 nb4 = *reinterpret_cast<const f32x4*>(&bgo_s[32 * uo + 8 * rg + 4 * g]);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(accgo[4 * rg + e], NLOG2E, nb4[e])));
        store4(&gbuf[l32 * EG + ((8 * rg + 4 * g) ^ EBSW(l32))], TypeOps<T>::from_f32(v));
      }
      wave_lds_sync();
      store_gate(tl);
    }
  };

  int64_t t = blockIdx.x;
  if (t >= ntiles) return;  // uniform over the workgroup
  V8 xr[XMF];
  ProjMask<T> mreg;
  PTile cur = proj_tile(t, N, outgoing);
  load_x(xr, mreg, cur);
  __syncthreads();  // LN parameters and gate weights in LDS
  ln_store(xr, mreg, 0);
  __syncthreads();
  int cb = 0;
  TileWalk walk = proj_walk(t + gridDim.x, gridDim.x, N, outgoing);  // the next tile
  for (; t < ntiles; t += gridDim.x) {
    const int64_t tn = t + gridDim.x;
    const bool has_next = tn < ntiles;  // uniform over the workgroup
    // the next tile's x (the current one's again after the last tile: unconditional, so the
    // compiler sees no path on which these loads are still in flight at the next iteration)
    const PTile nxt = has_next ? proj_tile(walk, outgoing) : cur;
    walk.step();
    load_x(xr, mreg, nxt);
    compute(cur, cb);
    ln_store(xr, mreg, cb ^ 1);  // after the last tile into the free buffer: nobody reads it
    __syncthreads();  // tile cb consumed by every wave, tile cb ^ 1 complete
    cb ^= 1;
    cur = nxt;
  }
}

// ---- stage 1, ping-pong variant: 16-bit types with C = c_hidden = 128 ---------------------
// The fixed-width kernel above runs every wave of its workgroup through the same sequence
// (MFMAs, then the sigmoid epilogue, then the next tile's LayerNorm) between two barriers, so
// the two waves that share a SIMD (w and w + 4) are always in the same phase and the matrix
// pipe idles while the vector ALU works and the other way round. Here the workgroup is two
// groups of four waves, A = waves 0-3 (one per SIMD) and B = waves 4-7, run half a tile
// apart: in one barrier interval A runs the MFMAs of tile t while B runs the epilogue of tile
// t - 1 and a half of the LayerNorm of tile t + 1, and in the next interval the roles swap.
// Wave w owns projection unit w (32 channels of [a; b] with their g_in gate, weights in
// registers for the whole launch) and gate item w (32 output-gate channels, 32(w % 4)..,
// over the 32-pixel half w / 4 of the tile). Each group normalises the 32 pixels of its own
// half (8 lanes per pixel, wave-local sums), so z of a tile is complete after the two
// epilogue intervals that precede its first MFMA interval. Intervals (s = 0 .. 2 nt, with a
// barrier after each; tiles t = 0 .. nt - 1 are this workgroup's):
//   s = 2t:     A: MFMAs of t (z buffer t % 2), x of t + 1 requested (its half).
//               B: epilogue of t - 1, LayerNorm of t + 1 (its half) into z buffer (t + 1) % 2.
//   s = 2t + 1: A: epilogue of t, LayerNorm of t + 1 (its half).
//               B: MFMAs of t, x of t + 2 requested (its half).
// The mask values of a tile (read by the epilogues) are kept in three LDS slots, because B
// reads tile t's while writing tile t + 2's.
struct ProjPPLds {
  static constexpr int CK = 128;
  static constexpr int ZR = CK + 8;  // z and gate-weight row pitch (16-bit elements)
  static constexpr int ER = 72;      // unit staging [32 channels][64 pixels + 8]
  static constexpr int EG = 40;      // gate staging [32 pixels][32 channels + 8]
  static constexpr size_t zs = 0;                                  // [2][PTP][ZR]
  static constexpr size_t wgo = zs + 2 * (size_t)PTP * ZR * 2;     // [CK][ZR]
  static constexpr size_t ebuf = wgo + (size_t)CK * ZR * 2;        // [PW][32][ER]
  static constexpr size_t gbuf = ebuf + (size_t)PW * 32 * ER * 2;  // [PW][32][EG]
  static constexpr size_t bgo = gbuf + (size_t)PW * 32 * EG * 2;   // [CK] fp32
  static constexpr size_t lnw = bgo + (size_t)CK * 4;              // gamma, beta [2][CK] fp32
  static constexpr size_t mk = lnw + 2 * (size_t)CK * 4;           // [3][PTP] fp32
  static constexpr size_t mk1 = mk + 3 * (size_t)PTP * 4;          // [3][2] int: half all ones
  static constexpr size_t total = mk1 + 32;
};

template <typename T>
__global__ __launch_bounds__(PNT, 1) void trimul_proj_pp_kernel(const gnn_trimul_args a, int64_t NP,
                                                                size_t off_a, size_t off_b, size_t off_g) {
  static_assert(sizeof(T) == 2, "ping-pong projection: 16-bit types");
  typedef typename TypeOps<T>::V8 V8;
  typedef ProjPPLds LD;
  constexpr int CK = LD::CK, Ch = CK;
  constexpr int ZR = LD::ZR, ER = LD::ER, EG = LD::EG;
  constexpr int NKS = CK / 16;  // k-steps
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int N = (int)a.N;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;  // 0: group A, 1: group B
  T* zs = reinterpret_cast<T*>(smem_raw + LD::zs);
  T* wgo_s = reinterpret_cast<T*>(smem_raw + LD::wgo);
  T* ebuf = reinterpret_cast<T*>(smem_raw + LD::ebuf) + wave * 32 * ER;
  T* gbuf = reinterpret_cast<T*>(smem_raw + LD::gbuf) + wave * 32 * EG;
  float* bgo_s = reinterpret_cast<float*>(smem_raw + LD::bgo);
  float* lnw = reinterpret_cast<float*>(smem_raw + LD::lnw);
  float* lnb = lnw + CK;
  float* mk = reinterpret_cast<float*>(smem_raw + LD::mk);
  int* mk1 = reinterpret_cast<int*>(smem_raw + LD::mk1);
  const LnWidth lnw_in(a.ln_in_channels, CK);
  const bool outgoing = a.outgoing != 0;
  const int64_t ntiles = (int64_t)a.B * N * ((N + PTP - 1) / PTP);
  if ((int64_t)blockIdx.x >= ntiles) return;  // uniform over the workgroup
  const int nt = (int)((ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x);  // this workgroup's tiles
  constexpr float NLOG2E = -1.4426950408889634f;
  auto tile_of = [&](int k) { return proj_tile((int64_t)blockIdx.x + (int64_t)k * gridDim.x, N, outgoing); };

  // ---- per-workgroup constants
  {
    const T* wgo = (const T*)a.g_out_w;
    for (int c = tid; c < CK * CK / 8; c += PNT) {
      const int r = c / (CK / 8), k0 = (c % (CK / 8)) * 8;
      store8(&wgo_s[r * ZR + k0], load8(wgo + r * CK + k0));
    }
    for (int c = tid; c < CK; c += PNT) {
      bgo_s[c] = ld_or<T>(a.g_out_b, c, 0.f) * NLOG2E;  // the exp2 argument's bias term
      lnw[c] = ld_or<T>(a.ln_in_w, c, 1.f);
      lnb[c] = ld_or<T>(a.ln_in_b, c, 0.f);
    }
  }

  // ---- the group's half of a tile: thread (pixel xpl, part xpart), chunks xpart + 8j
  const int gt = tid & 255;
  const int xpl = 32 * grp + (gt >> 3), xpart = gt & 7;
  V8 xr[2];
  ProjMask<T> mreg;
  auto load_x = [&](const PTile& tl) {  // pixels past N load pixel N - 1, as in the kernel above
    const T* src = (const T*)a.x + proj_pix(tl, min(xpl, N - 1 - tl.c0), N, outgoing) * CK;
#pragma unroll
    for (int j = 0; j < 2; ++j) xr[j] = load8(src + 8 * (xpart + 8 * j));
    mreg.request(a, tl, 32 * grp + (gt & 31), N, outgoing);  // used by the threads gt < 32
  };
  auto ln_store = [&](int k) {  // LayerNorm of the half of local tile k held in xr
    const int zb = k & 1, mb = k % 3;
    f32x8 v[2];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      v[j] = TypeOps<T>::to_f32(xr[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[j][e];
    }
    s = sum8_dpp(s);
    const float mean = s * lnw_in.inv_n;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[j][e] - mean;
        q += d * d;
      }
    q = sum8_dpp(q);
    const float rstd = __builtin_amdgcn_rsqf(lnw_in.var(q, mean) + a.eps);  // as torch's rsqrt
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kk = 8 * (xpart + 8 * j);
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(lnw + kk);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(lnw + kk + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(lnb + kk);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(lnb + kk + 4);
      f32x8 z;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        z[e] = (v[j][e] - mean) * rstd * w0[e] + b0[e];
        z[e + 4] = (v[j][e + 4] - mean) * rstd * w1[e] + b1[e];
      }
      store8(&zs[(zb * PTP + xpl) * ZR + kk], TypeOps<T>::from_f32(z));
    }
    if (gt < 32) {  // first wave of the group: its half's mask values and whether all are one
      const float mv = mreg.value();
      mk[mb * PTP + 32 * grp + gt] = mv;
      const bool all1 = __ballot(mv != 1.f) == 0;
      if (gt == 0) mk1[2 * mb + grp] = all1;
    }
  };

  // ---- the wave's weights (one projection unit, one gate item), for the whole launch
  const int u = wave, ch = 32 * u + l32;
  const int uo = wave & 3, so = grp;  // gate item: channels 32 uo .., pixels 32 so ..
  V8 wpf[NKS], wgf[NKS];
  {
    const T* wprow = (const T*)a.p_in_w + (int64_t)ch * CK + 8 * g;
    const T* wgrow = (const T*)a.g_in_w + (int64_t)ch * CK + 8 * g;
#pragma unroll
    for (int k = 0; k < NKS; ++k) {
      wpf[k] = load8(wprow + 16 * k);
      wgf[k] = load8(wgrow + 16 * k);
    }
  }
  const float bp = ld_or<T>(a.p_in_b, ch, 0.f);
  const float bg = ld_or<T>(a.g_in_b, ch, 0.f) * NLOG2E;  // the exp2 argument's bias term
  T* __restrict__ a_cm = (T*)((unsigned char*)a.workspace + off_a);
  T* __restrict__ b_cm = (T*)((unsigned char*)a.workspace + off_b);
  T* __restrict__ gout = (T*)(a.gate ? (unsigned char*)a.gate : (unsigned char*)a.workspace + off_g);

  // accumulators carried from a wave's MFMA interval to its epilogue interval:
  // accp / accg [sub][r]: pixel 32 sub' + 8(r/4) + 4g + r%4 (sub' = so for sub 0, 1 - so for
  // sub 1), channel ch; accgo[r]: gate channel 32 uo + 8(r/4) + 4g + r%4, pixel 32 so + l32
  f32x16 accp[PSUB], accg[PSUB], accgo;
  auto mfma = [&](int k) {
    const T* z = zs + (k & 1) * PTP * ZR;
    const T* zrow0 = z + (32 * so + l32) * ZR + 8 * g;        // the gate item's half first
    const T* zrow1 = z + (32 * (1 - so) + l32) * ZR + 8 * g;
    const T* wgrow_s = wgo_s + (32 * uo + l32) * ZR + 8 * g;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      accp[0][r] = 0.f;
      accp[1][r] = 0.f;
      accg[0][r] = 0.f;
      accg[1][r] = 0.f;
      accgo[r] = 0.f;
    }
#pragma unroll
    for (int kk = 0; kk < NKS; ++kk) {
      const V8 z0 = load8(zrow0 + 16 * kk);
      const V8 z1 = load8(zrow1 + 16 * kk);
      const V8 wg = load8(wgrow_s + 16 * kk);
      Mma<T, PREC_NATIVE>::step(accp[0], z0, wpf[kk]);
      Mma<T, PREC_NATIVE>::step(accg[0], z0, wgf[kk]);
      Mma<T, PREC_NATIVE>::step(accgo, wg, z0);
      Mma<T, PREC_NATIVE>::step(accp[1], z1, wpf[kk]);
      Mma<T, PREC_NATIVE>::step(accg[1], z1, wgf[kk]);
    }
  };
  // epilogue, first half: the gated values into the wave's staging tiles (LDS)
  auto epilogue_stage = [&](int k) {
    const int mb = k % 3;
    const float* m = mk + mb * PTP;
    const bool all1 = mk1[2 * mb] != 0 && mk1[2 * mb + 1] != 0;
#pragma unroll
    for (int s = 0; s < PSUB; ++s) {
      const int sub = s == 0 ? so : 1 - so;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int pt = 32 * sub + 8 * rg + 4 * g;  // pixel within the tile
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (accp[s][4 * rg + e] + bp) *
                 __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(accg[s][4 * rg + e], NLOG2E, bg)));
        if (!all1) {
          const f32x4 m4 = *reinterpret_cast<const f32x4*>(&m[pt]);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] *= m4[e];
        }
        store4(&ebuf[l32 * ER + (pt ^ EBSW(l32))], TypeOps<T>::from_f32(v));
      }
    }
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const f32x4 nb4 = *reinterpret_cast<const f32x4*>(&bgo_s[32 * uo + 8 * rg + 4 * g]);
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(accgo[4 * rg + e], NLOG2E, nb4[e])));
      store4(&gbuf[l32 * EG + ((8 * rg + 4 * g) ^ EBSW(l32))], TypeOps<T>::from_f32(v));
    }
    wave_lds_sync();
  };
  // epilogue, second half: the staging tiles to global memory with 16-byte stores. Issued
  // after the interval's LayerNorm: its wait for the x loads (vmcnt counts loads and stores
  // in order) then covers no store of this tile.
  auto epilogue_store = [&](int k) {
    const PTile tl = tile_of(k);
    // unit: 8 lanes per 64-pixel channel row (store i: 8 channel planes on)
    {
      const int crow0 = lane >> 3, p0 = (lane & 7) * 8;
      const bool in_a = 32 * u < Ch;
      const int chh0 = 32 * u + crow0 - (in_a ? 0 : Ch);
      T* drow = (in_a ? a_cm : b_cm) + ab_offset<T>((int64_t)tl.b * Ch + chh0, tl.row, tl.c0 + p0, N, NP);
      const int64_t pstep = ab_offset<T>(8, 0, 0, N, NP);
      const bool full = tl.c0 + p0 + 8 <= N, tail = !full && tl.c0 + p0 < NP;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const V8 val = load8(&ebuf[(crow0 + 8 * i) * ER + (p0 ^ EBSW(crow0 + 8 * i))]);
        if (full) {
          store8(drow + i * pstep, val);
        } else if (tail) {  // row tail: pixels N .. NP-1 are written as zeros
          V8 vv = val;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (tl.c0 + p0 + e >= N) vv[e] = TypeOps<T>::from_f32(0.f);
          store8(drow + i * pstep, vv);
        }
      }
    }
    // gate item: 4 lanes per 32-channel pixel row segment
    {
      const int px = lane >> 2, k0 = (lane & 3) * 8, pl = 32 * so + px;
      T* dst = gout + proj_pix(tl, pl, N, outgoing) * CK + 32 * uo + k0;
      const int64_t step16 = (outgoing ? 16 : 16 * (int64_t)N) * CK;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (tl.c0 + pl + 16 * i < N) store8(dst + i * step16, load8(&gbuf[(px + 16 * i) * EG + (k0 ^ EBSW(px + 16 * i))]));
    }
    wave_lds_sync();  // the staging tiles are rewritten by the next epilogue
  };

  // ---- prologue: tile 0 normalised by both groups; B requests its half of tile 1
  load_x(tile_of(0));
  __syncthreads();  // LN parameters and gate weights in LDS
  ln_store(0);
  if (grp == 1) load_x(tile_of(min(1, nt - 1)));
  __syncthreads();

  // Each group runs its own loop, so that the compiler sees the real alternation of its
  // intervals (a loop over s with both kinds of interval behind a branch makes it assume an
  // MFMA interval may follow another, and wait there for loads that have long completed,
  // and with them, vmcnt being in order, for every store since). Both loops execute 2 nt + 1
  // barriers.
  // The x loads and LayerNorms past the last tile are done anyway, on the last tile's x into
  // slots nobody reads any more (z slot (nt + 1) % 2 and mask slots nt % 3, (nt + 1) % 3 are
  // free by then): kept unconditional, they leave the compiler no path on which a load is
  // still in flight at the next interval.
  if (grp == 0) {
    for (int k = 0; k < nt; ++k) {
      mfma(k);  // s = 2k
      load_x(tile_of(min(k + 1, nt - 1)));
      __syncthreads();
      epilogue_stage(k);  // s = 2k + 1
      ln_store(k + 1);
      epilogue_store(k);
      __syncthreads();
    }
    __syncthreads();  // s = 2 nt: B's last epilogue
  } else {
    ln_store(1);  // s = 0
    __syncthreads();
    for (int k = 0; k < nt; ++k) {
      mfma(k);  // s = 2k + 1
      load_x(tile_of(min(k + 2, nt - 1)));
      __syncthreads();
      epilogue_stage(k);  // s = 2k + 2
      ln_store(k + 2);
      epilogue_store(k);
      __syncthreads();
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

// fp32 under bf16x3 (what 'tf32' resolves to on gfx950): trimul_contract_kernel's schedule
// (one stage of k held in registers while the previous one multiplies), but each fp32 stage
// is split into bf16 hi / lo planes once, where it is written to LDS, so the inner loop reads
// hi / lo fragments and issues the three bf16 MFMAs (lo hi + hi lo + hi hi) with no VALU
// work; splitting per product instead repeats the split of every fragment for each of the
// MFMAs that reuse it. Tiles of BM x BM output elements, 4 waves of BM / 2 x BM / 2, two
// workgroups per CU. Each k-stage waits for a global load issued one stage earlier, so the
// kernel's time is about (tile rounds) x (N / 32 stages) x (load latency): BM = 192 cuts the
// rounds where the tile count allows (C5's N = 384: 512 tiles of 192 fill the 512 slots
// once; 1152 tiles of 128 took three rounds). With KFULL (N a multiple of 32) the loads are
// unconditional: rows past N read row N - 1, whose products land in output rows that are not
// stored. Measured slower: the projection writing a and b as bf16 hi / lo planes in the
// 16-bit layout and the DMA-fed 16-bit contraction reading both planes (128 x 256 tiles,
// three 48 KB stages, one workgroup per CU: 81 us).
template <int BM>
struct ContractX3 {
  static constexpr int BK = 32;
  static constexpr int ROW = BK + 8;  // bf16 elements per LDS row (16 B of padding)
  static constexpr int WT = BM / 64;  // 32 x 32 MFMA tiles per wave and dimension
};

template <int BM, bool KFULL>
__global__ __launch_bounds__(NT, 2) void trimul_contract_x3_kernel(const float* __restrict__ A,
                                                                  const float* __restrict__ Bm,
                                                                  float* __restrict__ O, int N, int64_t NP) {
  typedef ContractX3<BM> Cfg;
  constexpr int WT = Cfg::WT;
  __shared__ __align__(16) bf16 ash[BM * Cfg::ROW], asl[BM * Cfg::ROW];
  __shared__ __align__(16) bf16 bsh[BM * Cfg::ROW], bsl[BM * Cfg::ROW];

  const int nt = (N + BM - 1) / BM;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int tj = w % nt;
  const int ti = (w / nt) % nt;
  const int64_t plane = w / ((uint32_t)nt * nt);
  const int64_t poff = plane * N * NP;
  const float* Ap = A + poff;
  const float* Bp = Bm + poff;
  float* Op = O + poff;
  const int i0 = ti * BM, j0 = tj * BM;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  constexpr int CPR = Cfg::BK / 8;   // 8-element chunks per row per stage
  constexpr int CH = BM * CPR / NT;  // chunks per thread per operand
  static_assert(CH * NT == BM * CPR, "whole chunks per thread");
  f32x8 ra[CH], rb[CH];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NT;
      const int r = c / CPR, kc = k0 + (c % CPR) * 8;
      if constexpr (KFULL) {
        ra[i] = load8(Ap + (int64_t)min(i0 + r, N - 1) * NP + kc);
        rb[i] = load8(Bp + (int64_t)min(j0 + r, N - 1) * NP + kc);
      } else {
        ra[i] = f32x8{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        rb[i] = ra[i];
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
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NT;
      const int r = c / CPR, kl = (c % CPR) * 8;
      bf16x8 hi, lo;
      split_bf16(ra[i], hi, lo);
      store8(&ash[r * Cfg::ROW + kl], hi);
      store8(&asl[r * Cfg::ROW + kl], lo);
      split_bf16(rb[i], hi, lo);
      store8(&bsh[r * Cfg::ROW + kl], hi);
      store8(&bsl[r * Cfg::ROW + kl], lo);
    }
  };

  f32x16 acc[WT][WT];
#pragma unroll
  for (int x = 0; x < WT; ++x)
#pragma unroll
    for (int y = 0; y < WT; ++y)
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
      bf16x8 bh[WT], bl[WT];
#pragma unroll
      for (int y = 0; y < WT; ++y) {
        const int o = ((BM / 2) * wn + 32 * y + l32) * Cfg::ROW + 16 * kk + 8 * g;
        bh[y] = load8(&bsh[o]);
        bl[y] = load8(&bsl[o]);
      }
#pragma unroll
      for (int x = 0; x < WT; ++x) {
        const int o = ((BM / 2) * wm + 32 * x + l32) * Cfg::ROW + 16 * kk + 8 * g;
        const bf16x8 ah = load8(&ash[o]), al = load8(&asl[o]);
#pragma unroll
        for (int y = 0; y < WT; ++y) {
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh[y], acc[x][y], 0, 0, 0);
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl[y], acc[x][y], 0, 0, 0);
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh[y], acc[x][y], 0, 0, 0);
        }
      }
    }
    __syncthreads();
    if (has_next) store();
    __syncthreads();
  }

  // acc[x][y][r] = o[i0 + (BM / 2)wm + 32x + 8(r/4) + 4g + r%4][j0 + (BM / 2)wn + 32y + l32]
#pragma unroll
  for (int x = 0; x < WT; ++x)
#pragma unroll
    for (int y = 0; y < WT; ++y) {
      const int j = j0 + (BM / 2) * wn + 32 * y + l32;
      if (j >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + (BM / 2) * wm + 32 * x + 8 * (r / 4) + 4 * g + (r % 4);
        if (i < N) Op[(int64_t)i * NP + j] = acc[x][y][r];
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
// tile), so its latency hides behind the LayerNorm / the previous pass. fp32 under bf16x3
// splits each fragment at its product; writing the normalised tile as bf16 hi / lo planes
// once and splitting each p_out fragment once measured slower (65 against 61 us at
// N = 384, C = c_hidden = 128).
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
  return (out_region1_elems(Ch, pad) + (size_t)PTO * (Ch + pad)) * elem + (2 * (size_t)Ch + 8 * PTO + OPC) * 4;
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

// CK / CHK: c_z / c_hidden fixed at compile time (0 = taken from the arguments), so the
// common 128 / 128 instantiation folds its loop bounds, chunk divisions and address strides.
template <typename T, int PREC, int CK, int CHK>
__global__ __launch_bounds__(NT, 2) void trimul_out_kernel(const gnn_trimul_args a, int64_t NP,
                                                           size_t off_g, size_t off_o) {
  typedef typename TypeOps<T>::V8 V8;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int C = CK ? CK : (int)a.C, Ch = CHK ? CHK : (int)a.Ch, N = (int)a.N;
  const int OR = PTO + lds_pad<T>();  // raw o tile [Ch][OR]
  const int ZR = Ch + lds_pad<T>();   // normalised tile [PTO][ZR]
  const int YR = OPC + lds_pad<T>();  // pass tile [PTO][YR]
  T* ot = reinterpret_cast<T*>(smem_raw);
  T* ys = ot;  // the o tile is dead once the LayerNorm has written zs
  T* zs = ot + out_region1_elems(Ch, lds_pad<T>());
  float* lnw = reinterpret_cast<float*>(zs + (size_t)PTO * ZR);
  float* lnb = lnw + Ch;
  float* red = lnb + Ch;        // LayerNorm partial sums [8 * PTO]
  float* bpo_s = red + 8 * PTO;  // p_out bias of the current pass [OPC]

  const int ntile = (N + PTO - 1) / PTO;
  const int ct = blockIdx.x % ntile;
  const int p = (blockIdx.x / ntile) % N;
  const int b = blockIdx.x / (ntile * N);
  const int q0 = ct * PTO;
  const int npix = N - q0 < PTO ? N - q0 : PTO;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;

  const T* __restrict__ ocm = (const T*)((const unsigned char*)a.workspace + off_o);
  const int64_t blk = (((int64_t)b * N + p) * N + q0) * C;
  const T* __restrict__ gblk =
      (const T*)(a.gate ? (const unsigned char*)a.gate : (const unsigned char*)a.workspace + off_g) + blk;
  T* __restrict__ oblk = (T*)a.out + blk;

  V8 gr[OCH];
  out_load_g<T>(gr, gblk, C, 0, (C < OPC ? C : OPC) / 8, npix, tid);
  // p_out fragments of this wave's first 32-channel tile, first KPF k-steps, loaded now so
  // their latency overlaps the o tile load and the LayerNorm
  constexpr int KPF = sizeof(T) == 2 ? 8 : 4;
  const T* __restrict__ wpo = (const T*)a.p_out_w;
  const int nk = Ch / 16;
  V8 wpf[KPF];
  if (32 * wave < C) {
    const T* wrow0 = wpo + (int64_t)(32 * wave + l32) * Ch + 8 * g;
#pragma unroll
    for (int k = 0; k < KPF; ++k)
      if (k < nk) wpf[k] = load8(wrow0 + 16 * k);
  }

  for (int c = tid; c < Ch; c += NT) {
    lnw[c] = ld_or<T>(a.ln_out_w, c, 1.f);
    lnb[c] = ld_or<T>(a.ln_out_b, c, 0.f);
  }
  for (int c = tid; c < (C < OPC ? C : OPC); c += NT) bpo_s[c] = ld_or<T>(a.p_out_b, c, 0.f);
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

  // ---- LayerNorm over channels. Thread = (pixel pair pp = tid % 32, channel part
  // tid / 32 of Ch / 8 channels): 32-bit LDS reads of two neighbouring pixels, the lanes of a
  // wave covering 64 consecutive pixels of one channel row; the parts' partial sums meet in
  // LDS. Two passes (mean, then squared deviations), as F.layer_norm.
  {
    const int pp = tid & 31, part = tid >> 5;
    const int kc = Ch / 8, k0 = part * kc;
    typedef T T2 __attribute__((ext_vector_type(2)));
    auto pair = [&](int k) -> f32x2 {
      return __builtin_convertvector(*reinterpret_cast<const T2*>(&ot[k * OR + 2 * pp]), f32x2);
    };
    float2* red2 = reinterpret_cast<float2*>(red);  // [8 parts][32 pairs]
    f32x2 s2 = {0.f, 0.f};
    for (int k = k0; k < k0 + kc; ++k) s2 += pair(k);
    red2[part * 32 + pp] = make_float2(s2[0], s2[1]);
    __syncthreads();
    f32x2 mean = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float2 v = red2[j * 32 + pp];
      mean += f32x2{v.x, v.y};
    }
    const LnWidth lw(a.ln_out_channels, Ch);
    mean *= lw.inv_n;
    f32x2 q2 = {0.f, 0.f};
    for (int k = k0; k < k0 + kc; ++k) {
      const f32x2 d = pair(k) - mean;
      q2 += d * d;
    }
    __syncthreads();  // every part has read the sums
    red2[part * 32 + pp] = make_float2(q2[0], q2[1]);
    __syncthreads();
    f32x2 var = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float2 v = red2[j * 32 + pp];
      var += f32x2{v.x, v.y};
    }
    const float rs0 = __builtin_amdgcn_rsqf(lw.var(var[0], mean[0]) + a.eps);  // as torch's rsqrt
    const float rs1 = __builtin_amdgcn_rsqf(lw.var(var[1], mean[1]) + a.eps);
    for (int k = k0; k < k0 + kc; k += 8) {
      f32x8 v0, v1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const f32x2 x = pair(k + e);
        v0[e] = (x[0] - mean[0]) * rs0 * lnw[k + e] + lnb[k + e];
        v1[e] = (x[1] - mean[1]) * rs1 * lnw[k + e] + lnb[k + e];
      }
      store8(&zs[(2 * pp) * ZR + k], TypeOps<T>::from_f32(v0));
      store8(&zs[(2 * pp + 1) * ZR + k], TypeOps<T>::from_f32(v1));
    }
  }
  __syncthreads();

  // ---- out = (z Wpo^T + bpo) * g, in passes of OPC output channels.
  // acc[s] = [cout][pixel]: cout = c0 + 32 wave + 8(r/4) + 4g + r%4, pixel = 32s + l32.
  for (int c0 = 0; c0 < C; c0 += OPC) {
    const int W = C - c0 < OPC ? C - c0 : OPC;
    if (32 * wave < W) {
      const int cw = c0 + 32 * wave;
      float bpo[16];
      if (c0 == 0) {  // first pass: from LDS
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bpo_s[32 * wave + 8 * rg + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) bpo[4 * rg + e] = b4[e];
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) bpo[r] = ld_or<T>(a.p_out_b, cw + 4 * g + 8 * (r / 4) + (r % 4), 0.f);
      }
      const T* wrow = wpo + (int64_t)(cw + l32) * Ch + 8 * g;
      f32x16 acc[PTO / 32];
#pragma unroll
      for (int s = 0; s < PTO / 32; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][r] = 0.f;
      if (c0 == 0) {
#pragma unroll
        for (int k = 0; k < KPF; ++k) {
          if (k >= nk) break;
#pragma unroll
          for (int s = 0; s < PTO / 32; ++s) {
            const V8 zf = load8(&zs[(32 * s + l32) * ZR + 16 * k + 8 * g]);
            Mma<T, PREC>::step(acc[s], wpf[k], zf);
          }
        }
      }
      for (int k = c0 == 0 ? KPF : 0; k < nk; ++k) {
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

// ---- stage 3, persistent variant: 16-bit types with C = c_hidden = 128 -------------------
// The kernel above starts each 64-pixel tile with its o and g loads and ends it with the out
// stores, so every workgroup's lifetime carries a memory round trip that only the other
// workgroups of its CU can hide. Here GNN_OUTP_WGS workgroups per CU walk the tiles t,
// t + grid, ... and keep the next tile's o and g in registers while the current tile is
// normalised, projected and written: o of t + grid is requested as soon as o of t is in LDS,
// g of t + grid as soon as g of t has been used. The p_out fragments of a wave's 32 output
// channels stay in registers for the whole launch. Every load is issued unconditionally
// (columns past N read the unused tail of o's rows, pixels past N of g re-read the tile's
// last pixel: neither reaches a stored result, the LayerNorm and the product being per
// pixel) and the out stores are buffer stores whose range ends at the tile's last pixel, so
// the hardware drops the lanes past N. No store sits in a branch, and the compiler's memory
// counter waits for a tile's loads then never cover the stores issued after them.
// fp32 inputs under the bf16x3 split (X3) take the same walk with every operand split into
// bf16 hi / lo halves once: the p_out fragments at launch, the normalised tile where the
// LayerNorm writes it (two bf16 planes); the products are lo*hi + hi*lo + hi*hi, as the
// per-tile kernel's, on the same split values in the same order.
#ifndef GNN_OUTP_WGS  // workgroups per CU the register allocation is held to
#define GNN_OUTP_WGS 3
#endif
#ifndef GNN_OUT_PERSIST  // 0: the per-tile kernel for C = c_hidden = 128 too
#define GNN_OUT_PERSIST 1
#endif
#ifndef GNN_OUTP_WGS_X3  // the same for the fp32 (bf16x3) instantiation (72 KB of LDS each)
#define GNN_OUTP_WGS_X3 2
#endif
// LDS of the persistent output stage: region 1 (the raw o tile, then the pass tile), the
// normalised tile (T, or two bf16 planes under X3), LayerNorm gamma / beta, partial sums and
// the p_out bias (fp32).
template <typename T>
__host__ __device__ constexpr size_t outp_zplane_bytes() {
  return sizeof(T) == 4 ? 2 * (size_t)PTO * (128 + 8) * 2 : (size_t)PTO * (128 + lds_pad<T>()) * sizeof(T);
}
template <typename T>
__host__ __device__ inline size_t outp_lds_bytes() {
  return out_region1_elems(128, lds_pad<T>()) * sizeof(T) + outp_zplane_bytes<T>() + (2 * 128 + 8 * PTO + OPC) * 4;
}

template <typename T>
__global__ __launch_bounds__(NT, sizeof(T) == 4 ? GNN_OUTP_WGS_X3 : GNN_OUTP_WGS) void trimul_out_persist_kernel(
    const gnn_trimul_args a, int64_t NP, size_t off_g, size_t off_o) {
  typedef typename TypeOps<T>::V8 V8;
  constexpr bool X3 = sizeof(T) == 4;  // fp32 under bf16x3
  constexpr int C = 128, Ch = 128, PAD = lds_pad<T>();
  constexpr int OR = PTO + PAD, ZR = Ch + (X3 ? 8 : PAD), YR = OPC + PAD;
  constexpr int NKS = Ch / 16;                 // k-steps of p_out
  constexpr int OCO = Ch * (PTO / 8) / NT;     // 8-pixel o chunks per thread
  constexpr int OCG = PTO * C / 8 / NT;        // 8-channel g / out chunks per thread
  typedef typename std::conditional<X3, bf16, T>::type ZT;  // the normalised tile's element
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* ot = reinterpret_cast<T*>(smem_raw);
  T* ys = ot;  // the raw o tile is dead once the LayerNorm has written zs
  ZT* zs = reinterpret_cast<ZT*>(ot + out_region1_elems(Ch, PAD));  // X3: the hi plane
  ZT* zsl = zs + (size_t)PTO * ZR;                                   // X3: the lo plane
  float* lnw = reinterpret_cast<float*>(smem_raw + out_region1_elems(Ch, PAD) * sizeof(T) + outp_zplane_bytes<T>());
  float* lnb = lnw + Ch;
  float* red = lnb + Ch;         // LayerNorm partial sums [8 * PTO]
  float* bpo_s = red + 8 * PTO;  // p_out bias [C]
  const int N = (int)a.N;
  const int ntile = (N + PTO - 1) / PTO;
  const int64_t ntiles = (int64_t)a.B * N * ntile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const T* __restrict__ ocm = (const T*)((const unsigned char*)a.workspace + off_o);
  const T* __restrict__ gbase =
      (const T*)(a.gate ? (const unsigned char*)a.gate : (const unsigned char*)a.workspace + off_g);

  for (int c = tid; c < Ch; c += NT) {
    lnw[c] = ld_or<T>(a.ln_out_w, c, 1.f);
    lnb[c] = ld_or<T>(a.ln_out_b, c, 0.f);
  }
  for (int c = tid; c < C; c += NT) bpo_s[c] = ld_or<T>(a.p_out_b, c, 0.f);
  // rows 32 wave + l32 of p_out_w: as loaded (16-bit), or split into hi / lo halves (X3)
  typedef typename std::conditional<X3, bf16x8, V8>::type WF;
  WF wpf[NKS], wpl[X3 ? NKS : 1];
  {
    const T* wrow = (const T*)a.p_out_w + (int64_t)(32 * wave + l32) * Ch + 8 * g;
#pragma unroll
    for (int k = 0; k < NKS; ++k) {
      if constexpr (X3)
        split_bf16(load8(wrow + 16 * k), wpf[k], wpl[k]);
      else
        wpf[k] = load8(wrow + 16 * k);
    }
  }

  // tiles as (pixel tile d0, row p = d1, batch b = d2) digits of a TileWalk
  // o chunk i of a thread: channel (tid + i NT) / 8, pixels 8 ((tid + i NT) % 8) ..
  auto load_o = [&](V8 (&ov)[OCO], const TileWalk& w) {
    const int q0 = w.d0 * PTO, p = w.d1, b = w.d2;
#pragma unroll
    for (int i = 0; i < OCO; ++i) {
      const int c = tid + i * NT, ch = c >> 3, col = min(q0 + (c & 7) * 8, (int)NP - 8);
      ov[i] = load8(ocm + (((int64_t)b * Ch + ch) * N + p) * NP + col);
    }
  };
  // g / out chunk i: pixel (tid + i NT) / 16, channels 8 ((tid + i NT) % 16) ..
  auto load_g = [&](V8 (&gr)[OCG], const TileWalk& w) {
    const int64_t row = (int64_t)w.d2 * N + w.d1;
    const int q0 = w.d0 * PTO, last = min(N - q0, PTO) - 1;
    const T* gblk = gbase + (row * N + q0) * C;
#pragma unroll
    for (int i = 0; i < OCG; ++i) {
      const int idx = tid + i * NT, px = min(idx >> 4, last);
      gr[i] = load8(gblk + (int64_t)px * C + 8 * (idx & 15));
    }
  };

  // o of tile t is written to LDS at the end of the previous iteration (before the loop for
  // the first tile), so that every wait for a tile's loads sees the same later requests: the
  // out stores (OCG) and the g loads (OCG) of the tile before it
  auto put_o = [&](const V8 (&ov)[OCO]) {
#pragma unroll
    for (int i = 0; i < OCO; ++i) {
      const int c = tid + i * NT;
      store8(&ot[(c >> 3) * OR + (c & 7) * 8], ov[i]);
    }
  };
  // tiles t (w0), t + grid (w1) and t + 2 grid (w2); past the last tile a load requests the
  // last one again, so that the loads stay unconditional
  int64_t t = blockIdx.x;
  if (t >= ntiles) return;  // uniform over the workgroup
  const int64_t G = gridDim.x;
  TileWalk w0(t, G, ntile, N), w1 = w0, w2 = w0;
  w1.step();
  w2.step();
  w2.step();
  V8 ov[OCO], gr[OCG];
  load_o(ov, w0);
  load_g(gr, w0);
  put_o(ov);
  load_o(ov, t + G < ntiles ? w1 : w0);
  for (; t < ntiles; t += G) {
    const bool n1 = t + G < ntiles, n2 = t + 2 * G < ntiles;  // uniform
    const int64_t row = (int64_t)w0.d2 * N + w0.d1;
    const int q0 = w0.d0 * PTO, npix = min(N - q0, PTO);
    __syncthreads();  // the o tile (and, on the first tile, the LayerNorm parameters) in LDS

    // ---- LayerNorm over channels, as the per-tile kernel: thread = (pixel pair tid % 32,
    // channel part tid / 32 of 16 channels), two passes through LDS partial sums
    {
      const int pp = tid & 31, part = tid >> 5, k0 = part * (Ch / 8);
      typedef T T2 __attribute__((ext_vector_type(2)));
      auto pair = [&](int k) -> f32x2 {
        return __builtin_convertvector(*reinterpret_cast<const T2*>(&ot[k * OR + 2 * pp]), f32x2);
      };
      float2* red2 = reinterpret_cast<float2*>(red);  // [8 parts][32 pairs]
      f32x2 s2 = {0.f, 0.f};
#pragma unroll
      for (int k = k0; k < k0 + Ch / 8; ++k) s2 += pair(k);
      red2[part * 32 + pp] = make_float2(s2[0], s2[1]);
      __syncthreads();
      f32x2 mean = {0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float2 v = red2[j * 32 + pp];
        mean += f32x2{v.x, v.y};
      }
      const LnWidth lw(a.ln_out_channels, Ch);
      mean *= lw.inv_n;
      f32x2 q2 = {0.f, 0.f};
#pragma unroll
      for (int k = k0; k < k0 + Ch / 8; ++k) {
        const f32x2 d = pair(k) - mean;
        q2 += d * d;
      }
      __syncthreads();  // every part has read the sums
      red2[part * 32 + pp] = make_float2(q2[0], q2[1]);
      __syncthreads();
      f32x2 var = {0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float2 v = red2[j * 32 + pp];
        var += f32x2{v.x, v.y};
      }
      const float rs0 = __builtin_amdgcn_rsqf(lw.var(var[0], mean[0]) + a.eps);  // as torch's rsqrt
      const float rs1 = __builtin_amdgcn_rsqf(lw.var(var[1], mean[1]) + a.eps);
#pragma unroll
      for (int k = k0; k < k0 + Ch / 8; k += 8) {
        f32x8 v0, v1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const f32x2 x = pair(k + e);
          v0[e] = (x[0] - mean[0]) * rs0 * lnw[k + e] + lnb[k + e];
          v1[e] = (x[1] - mean[1]) * rs1 * lnw[k + e] + lnb[k + e];
        }
        if constexpr (X3) {
          bf16x8 h0, l0, h1, l1;
          split_bf16(v0, h0, l0);
          split_bf16(v1, h1, l1);
          store8(&zs[(2 * pp) * ZR + k], h0);
          store8(&zsl[(2 * pp) * ZR + k], l0);
          store8(&zs[(2 * pp + 1) * ZR + k], h1);
          store8(&zsl[(2 * pp + 1) * ZR + k], l1);
        } else {
          store8(&zs[(2 * pp) * ZR + k], TypeOps<T>::from_f32(v0));
          store8(&zs[(2 * pp + 1) * ZR + k], TypeOps<T>::from_f32(v1));
        }
      }
    }
    __syncthreads();

    // ---- y = z Wpo^T + bpo on MFMA: acc[s] = [cout][pixel], cout = 32 wave + 8(r/4) + 4g +
    // r%4, pixel = 32s + l32; rounded to T into the pass tile ys
    {
      f32x16 acc[PTO / 32];
#pragma unroll
      for (int s = 0; s < PTO / 32; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][r] = 0.f;
#pragma unroll
      for (int k = 0; k < NKS; ++k)
#pragma unroll
        for (int s = 0; s < PTO / 32; ++s) {
          const int zo = (32 * s + l32) * ZR + 16 * k + 8 * g;
          if constexpr (X3) {  // lo * hi + hi * lo + hi * hi, as Mma<float, PREC_BF16X3>
            const bf16x8 zh = load8(&zs[zo]), zl = load8(&zsl[zo]);
            acc[s] = mfma_bf16(wpl[k], zh, acc[s]);
            acc[s] = mfma_bf16(wpf[k], zl, acc[s]);
            acc[s] = mfma_bf16(wpf[k], zh, acc[s]);
          } else {
            Mma<T, PREC_NATIVE>::step(acc[s], wpf[k], load8(&zs[zo]));
          }
        }
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bpo_s[32 * wave + 8 * rg + 4 * g]);
#pragma unroll
        for (int s = 0; s < PTO / 32; ++s) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[s][4 * rg + e] + b4[e];
          store4(&ys[(32 * s + l32) * YR + 32 * wave + 8 * rg + 4 * g], TypeOps<T>::from_f32(v));
        }
      }
    }
    __syncthreads();

    // ---- out = y * g over the contiguous block of the tile's pixels; the buffer's range
    // ends at pixel npix, so the lanes of pixels past N are dropped
    {
      T* oblk = (T*)a.out + (row * N + q0) * C;
      const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(oblk, npix * C * (int)sizeof(T));
#pragma unroll
      for (int i = 0; i < OCG; ++i) {
        const int idx = tid + i * NT, px = idx >> 4, c8 = idx & 15;
        const f32x8 y = TypeOps<T>::to_f32(load8(&ys[px * YR + 8 * c8]));
        const V8 val = TypeOps<T>::from_f32(y * TypeOps<T>::to_f32(gr[i]));
        const uint32_t off = (uint32_t)((px * C + 8 * c8) * (int)sizeof(T));
        if constexpr (X3) {  // 32 bytes: two 16-byte stores
          buffer_store(f32x4{val[0], val[1], val[2], val[3]}, rs, off);
          buffer_store(f32x4{val[4], val[5], val[6], val[7]}, rs, off + 16u);
        } else {
          buffer_store(val, rs, off);
        }
      }
    }
    load_g(gr, n1 ? w1 : w0);
    __syncthreads();  // ys (region 1) is rewritten by the next tile's o
    put_o(ov);
    load_o(ov, n2 ? w2 : (n1 ? w1 : w0));
    w0 = w1;
    w1 = w2;
    w2.step();
  }
}

// ---- stage 2, 16-bit types: BM x 256 tiles fed by a global->LDS DMA pipeline -------------
// Workgroup tile: BM rows of A (i) x 256 rows of B (j), BM = 128 (4 waves, 3 stages) or 256
// (8 waves, 4 stages); wave (wm, wn) of the (BM / 64) x 2 grid owns 64 i x 128 j as 2 x 4
// accumulators of 32 x 32, computed as O^T blocks (rows = j) so a lane holds 4 consecutive j
// of one i per register group. k advances in stages of 32 (64 bytes per row): every wave
// issues global_load_lds_dwordx4 for its share of a stage STAGES - 1 stages ahead of the one
// it multiplies, so operands never pass through registers. Within a stage row r keeps its
// four 16-byte chunks XOR-swizzled by (r / 4) % 4, which makes the fragment reads (16
// consecutive rows, one chunk each) hit 16 distinct bank groups. The K range runs to NP =
// round_up(N, 32): the projection stage writes zeros into columns N .. NP-1 of a and b. Rows
// past N are loaded from row N-1 (their outputs are never stored). The finished tile is
// staged in LDS, 128 rows at a time, and written with 16-byte row stores. The larger tile
// halves the L2 -> LDS bytes per flop, which bound the 128-row tile. At N = 512 the kernel
// moves its a / b / o bytes at about 4.5 TB/s, near the 4.9 TB/s a device-to-device copy
// reaches; measured without gain: a fifth stage (160 KB of LDS: GNN_CONTRACT_STAGES256=5,
// also slower at N = 1024, 303 against 294 us), and reading the next stage's fragments into
// a second register set while the current stage multiplies. At N = 1024 (37% of the MFMA
// peak) the vendor's batched GEMM on the same operands (torch.bmm, hipBLASLt) takes 279 us.
#ifndef GNN_CONTRACT_STAGES256  // DMA pipeline stages of the 256-row tile (32 KB each)
#define GNN_CONTRACT_STAGES256 4
#endif
template <int BM>
struct ContractDma {
  static constexpr int BN = 256, BK = 32;
  static constexpr int NW = BM / 32;                      // waves
  static constexpr int NTH = 64 * NW;                     // threads
  static constexpr int STAGES = BM == 256 ? GNN_CONTRACT_STAGES256 : 3;
  static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int QA = BM / 16 / NW, QB = BN / 16 / NW;  // DMA instructions per wave
  static constexpr int QPS = QA + QB;                          // ... per stage
  static constexpr int SP = BN + 8;                            // epilogue row pitch (elements)
  static constexpr int EROWS = 128;                            // epilogue rows per pass
  static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
  static_assert(EROWS * SP * 2 <= LDS_BYTES, "epilogue pass must fit the stage buffers");
  static_assert(QA * 16 * NW == BM && QB * 16 * NW == BN, "DMA split");
};

typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt vmcnt(N_) expcnt(7) lgkmcnt(0); the 6-bit vmcnt field is split into bits 3:0
// and 15:14 of the immediate
template <int N_>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N_ >= 0 && N_ < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x070 | (N_ & 15) | ((N_ >> 4) << 14));
}

template <typename T, int BM>
__global__ __launch_bounds__(ContractDma<BM>::NTH, BM == 256 ? 1 : 2) void trimul_contract_dma_kernel(
    const T* __restrict__ A, const T* __restrict__ Bm, T* __restrict__ O, int N, int64_t NP) {
  static_assert(sizeof(T) == 2, "16-bit operands");
  typedef typename TypeOps<T>::V8 V8;
  typedef ContractDma<BM> Cfg;
  constexpr int NTH = Cfg::NTH;
  __shared__ __align__(16) unsigned char smem[Cfg::LDS_BYTES];

  const int nti = (N + BM - 1) / BM;
  const int ntj = (N + Cfg::BN - 1) / Cfg::BN;
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int tj = w % ntj;
  const int ti = (w / ntj) % nti;
  const int64_t plane = w / ((uint32_t)ntj * nti);
  const int64_t poff = plane * N * NP;
  const T* Ap = A + poff;  // k-blocked operands: stage kt of row r at ((kt * N) + r) * 32
  const T* Bp = Bm + poff;
  T* Op = O + poff;
  const int i0 = ti * BM, j0 = tj * Cfg::BN;
  const int64_t stage_stride = (int64_t)N * Cfg::BK;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  // DMA source addresses of this lane: instruction q of a wave fills 16 rows x 64 bytes;
  // lane -> (row lane / 4, physical chunk lane % 4) holding logical chunk p ^ ((row / 4) % 4).
  const int drow = lane >> 2, dphys = lane & 3;
  const T* asrc[Cfg::QA];
  const T* bsrc[Cfg::QB];
#pragma unroll
  for (int q = 0; q < Cfg::QA; ++q) {
    const int r = 16 * Cfg::QA * wave + 16 * q + drow;
    const int c = dphys ^ ((r >> 2) & 3);
    asrc[q] = Ap + (int64_t)min(i0 + r, N - 1) * Cfg::BK + 8 * c;
  }
#pragma unroll
  for (int q = 0; q < Cfg::QB; ++q) {
    const int r = 16 * Cfg::QB * wave + 16 * q + drow;
    const int c = dphys ^ ((r >> 2) & 3);
    bsrc[q] = Bp + (int64_t)min(j0 + r, N - 1) * Cfg::BK + 8 * c;
  }
  auto issue = [&](int kt) {
    unsigned char* st = smem + (kt % Cfg::STAGES) * Cfg::STAGE_BYTES;
    const int64_t k0 = kt * stage_stride;
#pragma unroll
    for (int q = 0; q < Cfg::QA; ++q)
      __builtin_amdgcn_global_load_lds((const void*)(asrc[q] + k0),
                                       (lds_void_t*)(st + (16 * Cfg::QA * wave + 16 * q) * 64), 16, 0, 0);
#pragma unroll
    for (int q = 0; q < Cfg::QB; ++q)
      __builtin_amdgcn_global_load_lds((const void*)(bsrc[q] + k0),
                                       (lds_void_t*)(st + Cfg::A_BYTES + (16 * Cfg::QB * wave + 16 * q) * 64),
                                       16, 0, 0);
  };
  // fragment (row r, logical chunk c) of a stage operand
  auto frag = [&](const unsigned char* base, int r, int c) -> V8 {
    return *reinterpret_cast<const V8*>(base + r * 64 + ((c ^ ((r >> 2) & 3)) << 4));
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int y = 0; y < 4; ++y)
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[y][x][r] = 0.f;

  const int nkt = (int)(NP / Cfg::BK);
#pragma unroll
  for (int st = 0; st < Cfg::STAGES - 1; ++st)
    if (st < nkt) issue(st);
  for (int kt = 0; kt < nkt; ++kt) {
    // This wave's DMA of stage kt is its oldest outstanding one (QPS instructions per stage,
    // later stages issued after it) and its fragment reads of stage kt - 1 have returned;
    // after the barrier every wave's stage kt has landed and stage (kt - 1) % STAGES is no
    // longer read. A plain s_barrier (with a compiler memory clobber) replaces
    // __syncthreads, whose fence would also wait for the DMA of the later stages.
    const int ahead = min(Cfg::STAGES - 2, nkt - 1 - kt);  // stages issued after kt
    if (Cfg::STAGES >= 5 && ahead >= 3)
      wait_vm_lgkm0<3 * Cfg::QPS>();
    else if (ahead >= 2)
      wait_vm_lgkm0<2 * Cfg::QPS>();
    else if (ahead == 1)
      wait_vm_lgkm0<Cfg::QPS>();
    else
      wait_vm_lgkm0<0>();
    asm volatile("s_barrier" ::: "memory");
    if (kt + Cfg::STAGES - 1 < nkt) issue(kt + Cfg::STAGES - 1);
    const unsigned char* sa = smem + (kt % Cfg::STAGES) * Cfg::STAGE_BYTES;
    const unsigned char* sb = sa + Cfg::A_BYTES;
    // all fragment reads of the stage first, so their latency is exposed once per stage
    constexpr int KS = Cfg::BK / 16;
    V8 af[KS][2], bf[KS][4];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
      for (int x = 0; x < 2; ++x) af[kk][x] = frag(sa, 64 * wm + 32 * x + l32, 2 * kk + g);
#pragma unroll
      for (int y = 0; y < 4; ++y) bf[kk][y] = frag(sb, 128 * wn + 32 * y + l32, 2 * kk + g);
    }
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int y = 0; y < 4; ++y)
#pragma unroll
        for (int x = 0; x < 2; ++x) Mma<T, PREC_NATIVE>::step(acc[y][x], bf[kk][y], af[kk][x]);
    __builtin_amdgcn_sched_group_barrier(0x100, 6 * KS, 0);  // the LDS reads, in order
    __builtin_amdgcn_sched_group_barrier(0x008, 8 * KS, 0);  // then the MFMAs
  }

  // acc[y][x][r] = o[i = i0 + 64wm + 32x + l32][j = j0 + 128wn + 32y + 8(r/4) + 4g + r%4]
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
    for (int c = tid; c < Cfg::EROWS * CPR; c += NTH) {
      const int r = c / CPR, cj = (c % CPR) * 8;
      const int i = i0 + Cfg::EROWS * ep + r;
      if (i < N && j0 + cj < N) store8(Op + (int64_t)i * NP + j0 + cj, load8(&ot[r * Cfg::SP + cj]));
    }
  }
}

template <typename T>
size_t out_smem(const gnn_trimul_args& a) {
  return out_lds_bytes(a.Ch, sizeof(T));
}

template <typename T, int PREC, int XM>
int launch_proj_xm(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  const int64_t ntiles = a.B * a.N * ((a.N + PTP - 1) / PTP);
  const size_t smem = proj_lds<T>(a.C).total;
  const void* fn = (const void*)trimul_proj_kernel<T, PREC, XM>;
  if (smem > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  const int64_t grid = std::min<int64_t>(ntiles, persistent_grid(fn, PNT, smem));
  hipLaunchKernelGGL((trimul_proj_kernel<T, PREC, XM>), dim3((uint32_t)grid), dim3(PNT), smem, st, a, NP,
                     L.off_a, L.off_b, L.off_g);
  return (int)hipGetLastError();
}

template <typename T, int CK, int CHK>
int launch_proj_fast(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  const int64_t ntiles = a.B * a.N * ((a.N + PTP - 1) / PTP);
  constexpr size_t smem = ProjFastLds<CK>::total;
  const void* fn = (const void*)trimul_proj_fast_kernel<T, CK, CHK>;
  (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  const int64_t grid = std::min<int64_t>(ntiles, persistent_grid(fn, PNT, smem));
  hipLaunchKernelGGL((trimul_proj_fast_kernel<T, CK, CHK>), dim3((uint32_t)grid), dim3(PNT), smem, st, a, NP,
                     L.off_a, L.off_b, L.off_g);
  return (int)hipGetLastError();
}

#ifndef GNN_PROJ_PINGPONG  // 1: trimul_proj_pp_kernel for C = c_hidden = 128 (measured slower)
#define GNN_PROJ_PINGPONG 0
#endif
template <typename T>
int launch_proj_pp(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  const int64_t ntiles = a.B * a.N * ((a.N + PTP - 1) / PTP);
  constexpr size_t smem = ProjPPLds::total;
  const void* fn = (const void*)trimul_proj_pp_kernel<T>;
  (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  const int64_t grid = std::min<int64_t>(ntiles, persistent_grid(fn, PNT, smem));
  hipLaunchKernelGGL((trimul_proj_pp_kernel<T>), dim3((uint32_t)grid), dim3(PNT), smem, st, a, NP, L.off_a,
                     L.off_b, L.off_g);
  return (int)hipGetLastError();
}

template <int CK, bool FIXED>
int launch_proj_x3(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  const int64_t ntiles = a.B * a.N * ((a.N + PTP - 1) / PTP);
  constexpr size_t smem = ProjX3Lds<CK>::total;
  const void* fn = (const void*)trimul_proj_x3_kernel<CK, FIXED>;
  (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  const int64_t grid = std::min<int64_t>(ntiles, persistent_grid(fn, PNT, smem));
  hipLaunchKernelGGL((trimul_proj_x3_kernel<CK, FIXED>), dim3((uint32_t)grid), dim3(PNT), smem, st, a, NP,
                     L.off_a, L.off_b, L.off_g);
  return (int)hipGetLastError();
}

#ifndef GNN_PROJX3_FIXED
#define GNN_PROJX3_FIXED 1
#endif
template <typename T, int PREC>
int launch_proj(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  if constexpr (sizeof(T) == 4 && PREC == PREC_BF16X3) {
    if (2 * a.Ch <= 32 * PW) {  // one projection unit per wave
      // c_hidden = 128 takes buffer stores over ranges of 32 channel planes (128 N NP bytes)
      if (GNN_PROJX3_FIXED && a.C == 128 && a.Ch == 128 && 128 * a.N * round_up(a.N, 32) < ((int64_t)1 << 31))
        return launch_proj_x3<128, true>(a, L, st);
      if (a.C == 128) return launch_proj_x3<128, false>(a, L, st);
      if (a.C == 64) return launch_proj_x3<64, false>(a, L, st);
    }
  }
  if constexpr (sizeof(T) == 2) {
    if (GNN_PROJ_PINGPONG && a.C == 128 && a.Ch == 128) return launch_proj_pp<T>(a, L, st);
    // c_hidden = 128 takes buffer stores over ranges of 8 channel planes (16 N NP bytes)
    if (a.C == 128 && a.Ch == 128 && 16 * a.N * round_up(a.N, 32) < ((int64_t)1 << 31))
      return launch_proj_fast<T, 128, 128>(a, L, st);
    if (a.C == 128) return launch_proj_fast<T, 128, 0>(a, L, st);
    if (a.C == 64) return launch_proj_fast<T, 64, 0>(a, L, st);
  }
  switch (proj_xm(a.C)) {
    case 2: return launch_proj_xm<T, PREC, 2>(a, L, st);
    case 4: return launch_proj_xm<T, PREC, 4>(a, L, st);
    default:
      if constexpr (sizeof(T) == 2) return launch_proj_xm<T, PREC, 8>(a, L, st);
      return set_error(GNN_ERR_UNSUPPORTED, "trimul: fp32 c_z above 256 is not supported");
  }
}

template <typename T, int BM>
int launch_contract_dma(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st, int64_t NP) {
  typedef ContractDma<BM> D;
  const int64_t nblk = a.B * a.Ch * ((a.N + BM - 1) / BM) * ((a.N + D::BN - 1) / D::BN);
  unsigned char* wsp = (unsigned char*)a.workspace;
  hipLaunchKernelGGL((trimul_contract_dma_kernel<T, BM>), dim3((uint32_t)nblk), dim3(D::NTH), 0, st,
                     (const T*)(wsp + L.off_a), (const T*)(wsp + L.off_b), (T*)(wsp + L.off_o), (int)a.N, NP);
  return (int)hipGetLastError();
}

// fp32 under bf16x3: the tile edge with fewer rounds of workgroups over the device's
// resident slots (each kernel's own occupancy: 162 VGPRs give the 128-tile kernel three
// workgroups per CU, 256 give the 192-tile kernel two; ties keep 128, whose stages multiply
// faster); GNN_CONTRACT_X3_BM = 128 or
// 192 forces one.
#ifndef GNN_CONTRACT_X3_BM
#define GNN_CONTRACT_X3_BM 0
#endif
template <int BM>
int launch_contract_x3_bm(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st, int64_t NP,
                          int64_t nblk) {
  unsigned char* ws = (unsigned char*)a.workspace;
  const float* A = (const float*)(ws + L.off_a);
  const float* Bm = (const float*)(ws + L.off_b);
  float* O = (float*)(ws + L.off_o);
  if (a.N % ContractX3<BM>::BK == 0)
    hipLaunchKernelGGL((trimul_contract_x3_kernel<BM, true>), dim3((uint32_t)nblk), dim3(NT), 0, st, A, Bm, O,
                       (int)a.N, NP);
  else
    hipLaunchKernelGGL((trimul_contract_x3_kernel<BM, false>), dim3((uint32_t)nblk), dim3(NT), 0, st, A, Bm, O,
                       (int)a.N, NP);
  return (int)hipGetLastError();
}

int launch_contract_x3(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st, int64_t NP) {
  auto tiles = [&](int64_t bm) { return a.B * a.Ch * ((a.N + bm - 1) / bm) * ((a.N + bm - 1) / bm); };
  const int64_t t128 = tiles(128), t192 = tiles(192);
  int bm = GNN_CONTRACT_X3_BM;
  if (bm != 128 && bm != 192) {
    const int64_t s128 = persistent_grid((const void*)trimul_contract_x3_kernel<128, true>, NT, 0);
    const int64_t s192 = persistent_grid((const void*)trimul_contract_x3_kernel<192, true>, NT, 0);
    bm = (t192 + s192 - 1) / s192 < (t128 + s128 - 1) / s128 ? 192 : 128;
  }
  return bm == 192 ? launch_contract_x3_bm<192>(a, L, st, NP, t192) : launch_contract_x3_bm<128>(a, L, st, NP, t128);
}

// Smallest N that takes the 256-row contraction tile. Measured at N = 512: the 128-row tile
// is faster on warm inputs (43.8 against 48.5 us) but slower inside the step (56 against
// 49 us), where a and b arrive from the projection kernel rather than from the cache.
#ifndef GNN_CONTRACT_BM256_N
#define GNN_CONTRACT_BM256_N 512
#endif
template <typename T, int PREC>
int launch_contract(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  if constexpr (sizeof(T) == 2) {
    // 256-row tiles once N fills them (half the L2 -> LDS bytes per flop), 128 below
    if (a.N >= GNN_CONTRACT_BM256_N) return launch_contract_dma<T, 256>(a, L, st, NP);
    return launch_contract_dma<T, 128>(a, L, st, NP);
  }
  typedef ContractCfg<T> Cfg;
  const int64_t nblk = a.B * a.Ch * ((a.N + Cfg::BM - 1) / Cfg::BM) * ((a.N + Cfg::BN - 1) / Cfg::BN);
  unsigned char* ws = (unsigned char*)a.workspace;
  if constexpr (sizeof(T) == 4 && PREC == PREC_BF16X3) {
    return launch_contract_x3(a, L, st, NP);
  } else {
    hipLaunchKernelGGL((trimul_contract_kernel<T, PREC>), dim3((uint32_t)nblk), dim3(NT), 0, st,
                       (const T*)(ws + L.off_a), (const T*)(ws + L.off_b), (T*)(ws + L.off_o), (int)a.N,
                       NP);
  }
  return (int)hipGetLastError();
}

template <typename T, int PREC, int CK, int CHK>
int launch_out_w(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  const int64_t NP = round_up(a.N, 32);
  const int64_t ntile = (a.N + PTO - 1) / PTO;
  const size_t smem = out_smem<T>(a);
  if constexpr (((sizeof(T) == 2 && PREC == PREC_NATIVE) || (sizeof(T) == 4 && PREC == PREC_BF16X3)) && CK == 128 &&
                CHK == 128) {
    if (GNN_OUT_PERSIST) {
      const size_t psmem = outp_lds_bytes<T>();
      const void* pf = (const void*)trimul_out_persist_kernel<T>;
      if (psmem > 64 * 1024) (void)hipFuncSetAttribute(pf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)psmem);
      const int64_t grid = std::min<int64_t>(a.B * a.N * ntile, persistent_grid(pf, NT, psmem));
      hipLaunchKernelGGL((trimul_out_persist_kernel<T>), dim3((uint32_t)grid), dim3(NT), psmem, st, a, NP, L.off_g,
                         L.off_o);
      return (int)hipGetLastError();
    }
  }
  const void* fn = (const void*)trimul_out_kernel<T, PREC, CK, CHK>;
  if (smem > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  hipLaunchKernelGGL((trimul_out_kernel<T, PREC, CK, CHK>), dim3((uint32_t)(a.B * a.N * ntile)), dim3(NT),
                     smem, st, a, NP, L.off_g, L.off_o);
  return (int)hipGetLastError();
}

template <typename T, int PREC>
int launch_out(const gnn_trimul_args& a, const TrimulLayout& L, hipStream_t st) {
  if (a.C == 128 && a.Ch == 128) return launch_out_w<T, PREC, 128, 128>(a, L, st);
  return launch_out_w<T, PREC, 0, 0>(a, L, st);
}

int check_args(const gnn_trimul_args& a, const char* who) {
  // the contraction (stage 2) depends on the B * Ch planes and N only: any width
  const bool widths = std::string(who) != "contract";
  if (!a.x || !a.out || !a.p_in_w || !a.g_in_w || !a.p_out_w || !a.g_out_w)
    return set_error(GNN_ERR_ARG, "trimul: x, out and the four projection weights are required");
  if (a.B < 1 || a.N < 1 || a.C < 1 || a.Ch < 1)
    return set_error(GNN_ERR_ARG, "trimul: B, N, C and Ch must be positive");
  if (a.C % 32 != 0 || a.Ch % 32 != 0)
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: c_z and c_hidden must be multiples of 32");
  if (widths && (a.C > 512 || a.Ch > 512))
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: c_z and c_hidden above 512 are not supported");
  if (a.dtype != GNN_BF16 && a.dtype != GNN_F16 && a.dtype != GNN_F32)
    return set_error(GNN_ERR_ARG, "trimul: unknown dtype");
  if (a.ln_in_channels < 0 || a.ln_in_channels > a.C || a.ln_out_channels < 0 || a.ln_out_channels > a.Ch)
    return set_error(GNN_ERR_ARG, "trimul: ln_in_channels / ln_out_channels must lie in [0, C] / [0, Ch]");
  const void* vec[] = {a.x, a.out, a.p_in_w, a.g_in_w, a.p_out_w, a.g_out_w, a.workspace, a.gate};
  for (const void* ptr : vec)
    if (((uintptr_t)ptr) % 16 != 0)
      return set_error(GNN_ERR_ARG, "trimul: x, out, weights, workspace and gate must be 16-byte aligned");
  const size_t e = a.dtype == GNN_F32 ? 4 : 2;
  if (widths && e == 4 && (a.C > 256 || a.Ch > 256))
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: fp32 c_z and c_hidden above 256 are not supported");
  const size_t proj_bytes = e == 2 ? proj_lds<bf16>(a.C).total : proj_lds<float>(a.C).total;
  const size_t out_lds = out_lds_bytes(a.Ch, e);
  if (widths && (proj_bytes > 160 * 1024 || out_lds > 160 * 1024))
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: channel count too large for the LDS tiles");
  if (a.B * a.N * ((a.N + PTO - 1) / PTO) >= ((int64_t)1 << 31))
    return set_error(GNN_ERR_UNSUPPORTED, "trimul: grid too large");
  const TrimulLayout L = trimul_layout(a.B, a.N, a.C, a.Ch, a.dtype);
  // with a separate gate buffer the workspace holds a, b and o only (the gate region is last)
  if (!a.workspace || a.workspace_bytes < (a.gate ? L.off_g : L.total))
    return set_error(GNN_ERR_WORKSPACE, "trimul: workspace missing or smaller than gnn_trimul_workspace_bytes() "
                                        "(its gate offset when args.gate is set)");
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
  L.off_o = 2 * cm;
  L.off_g = 3 * cm;  // last, so that a caller with its own gate buffer can stop the workspace there
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
