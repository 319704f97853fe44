// Triangle attention forward for gfx950 (MI355X).
//
// Computes, for every (b, s, h) row of the pair stack and every query i,
//   o[b,s,i,h,:] = sum_j softmax_j(l_ij) v[b,s,j,h,:],
//   l_ij = scale * q[b,s,i,h,:].k[b,s,j,h,:] + bias[b,h,i,j] + mask_bias[b,s,j]
// which is triangle_attention_torch (geometric_nn_ops_torch/triangle/_reference/
// triangle_attention.py:11-44) and the Triton forward it stands in for
// (geometric_nn_ops_torch/triangle/_kernels/triangle_attention.py:48-365).
//
// Design (one workgroup = 4 waves x 32 queries, for R consecutive N_seq rows s of one
// (b, h); a wave owns the same 32 queries in every one of its R rows):
//   * The score tile is computed transposed, S^T = K Q'^T, on 32x32x16 MFMA so that each
//     lane owns ONE query (l % 32) and 16 of the 32 keys of a sub-tile: the
//     softmax statistics are per-lane scalars, the row max needs one cross-half exchange
//     per 64 keys and the row sum none until the end.
//   * O^T = V^T P^T: the probabilities feed the second MFMA straight from the score
//     registers (P^T is the B operand), and the running-max rescale of O is a per-lane
//     scalar multiply.
//   * K (row-major) and V^T of each row are staged per 64-key tile in LDS (16-byte
//     coalesced loads) and shared by the 4 waves. Q' = bf16(q * scale), rounded like the
//     reference's
//     Q * softmax_scale, lives in registers.
//   * The pair bias is read straight from global memory in the MFMA B-fragment layout
//     (lane = query, 8 consecutive keys = 16 bytes), one tile ahead, and added on the MFMA
//     unit: one extra 32x32x16 step per 16 keys multiplies an identity fragment (rows =
//     keys) by the bias fragment (cols = queries), so the bias costs no VALU work (fp32
//     inputs add it on the VALU). The bias plane bias[b, h] is the same for every N_seq
//     row, so each fragment loaded serves the workgroup's R rows: bias traffic and the
//     per-tile barriers are amortised over R rows.
//   * The key mask costs nothing on tiles whose 64 keys are all kept; other tiles add the
//     caller's sentinel (mask_val rounded to the input dtype, in fp32, after the bias)
//     and -inf for keys past N, on the VALU.
//   * p = exp2(s * log2 e - m * log2 e): one FMA and one v_exp_f32 per score for 16-bit
//     inputs and fp32 under the bf16x3 split; fp32 under 'ieee' and rows with no live key
//     (m is then the -1e9 sentinel) use the exact (s - m) * log2 e. The row sum adds the fp32 probabilities before they are
//     rounded for the PV product, as the reference's tl.sum(P_block, 1) does (v_add_f32
//     issues alongside other waves' MFMAs; a v_dot2 on the rounded values holds the
//     matrix pipe).
//   * The running max only moves when a tile raises it by more than 8 ln 2, so most
//     tiles skip the O / l rescale; p then stays below 2^8.
//   * Key tiles whose keys are all masked are skipped when the row has at least one live
//     key (their probabilities are exactly 0 either way). Rows with no live key are
//     computed in full, reproducing the finite-sentinel result of the reference.
//   * Workgroup ids are remapped so the workgroups on one XCD walk consecutive
//     (b, row group, h, q-block) items: the q-blocks sharing K/V, and the heads sharing one
//     bias plane, then hit that XCD's L2.
#include "gnn_common.hpp"
#include "gnn_internal.hpp"

#include <type_traits>

namespace gnn {

namespace {

constexpr int KT = 64;  // keys per LDS tile
constexpr int NTHREADS = 256;
constexpr int MAX_TILES = 512;  // N <= 32768
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_THRESHOLD = 8.0f / LOG2E;  // natural-log units: p <= 2^8

// Tuning (measured on MI355X at N_res = 512, D = 32, bf16): a single LDS stage (two
// barriers per key tile, 14.6 KB) beat double buffering, and one N_seq row per workgroup
// beat sharing the bias fragments across 2 or 4 rows, whose extra K/V staging and
// registers cost more than the bias loads they saved.
#ifndef GNN_ATTN_NBUF
#define GNN_ATTN_NBUF 1
#endif
#ifndef GNN_ATTN_MINBLOCKS
#define GNN_ATTN_MINBLOCKS 2
#endif
#ifndef GNN_ATTN_ROWS
#define GNN_ATTN_ROWS 1
#endif

constexpr int QB = 128;              // queries per workgroup (32 per wave)
constexpr int R = GNN_ATTN_ROWS;     // N_seq rows per workgroup (sharing the bias plane)

// X3: fp32 inputs under the bf16x3 split with DP <= 64 stage K and V as two bf16 planes
// each (hi, lo), split once where the tile is written to LDS, instead of splitting every
// fragment in every wave at every product; the planes are laid out and read like a 16-bit
// input's.
template <typename T, int DP, bool X3 = false>
struct Smem {
  typedef typename std::conditional<X3, bf16, T>::type E;  // staged element type
  static constexpr int PL = X3 ? 2 : 1;                    // planes
  static constexpr int KPAD = (sizeof(E) == 2) ? 8 : 4;    // 16 B per row
  static constexpr int KROW = DP + KPAD;
  // 16-bit types keep V as [key][d] and read V^T fragments with ds_read_b64_tr_b16: a row
  // pitch of 64 B modulo 256 B puts the four 64-byte row windows of one read pass on
  // disjoint banks. fp32 stores V^T [d][key].
  static constexpr bool VTR = sizeof(E) == 2;
  static constexpr int VROW = VTR ? (DP == 32 ? 32 : DP + 32) : KT + 4;
  static constexpr int VSIZE = VTR ? KT * VROW : DP * VROW;
  static constexpr int NBUF = GNN_ATTN_NBUF;
  E k[NBUF][R][PL][KT * KROW];
  E vt[NBUF][R][PL][VSIZE];
  uint64_t tile_live[R][MAX_TILES];  // bit j: key tile*64+j is < N and unmasked in row r
  uint16_t tile_list[MAX_TILES];     // tiles with a live key in some row (all if a row is dead)
  int ntiles_run;
  int row_dead[R];                   // row r has no live key (or does not exist)
};

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 frag_from_acc(const f32x16& p, int t) {
  f32x8 x = {p[8 * t + 0], p[8 * t + 1], p[8 * t + 2], p[8 * t + 3],
             p[8 * t + 4], p[8 * t + 5], p[8 * t + 6], p[8 * t + 7]};
  return TypeOps<T>::from_f32(x);
}

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, lane r supplies the address
// of 4 consecutive 16-bit elements (row r of a 16 x 4 block) and lane i receives element
// i % 4 of rows i / 4, 4 + i / 4, 8 + i / 4 and 12 + i / 4.
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V4 tr_read4(const T* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(__attribute__((address_space(3))) const T*)p);
  return __builtin_bit_cast(typename TypeOps<T>::V4, v);
}

// acc + the 8 fp32 probabilities of fragment t of an accumulator (a pairwise tree)
__device__ __forceinline__ float rowsum_add(const f32x16& p, int t, float acc) {
  const f32x8 v = {p[8 * t + 0], p[8 * t + 1], p[8 * t + 2], p[8 * t + 3],
                   p[8 * t + 4], p[8 * t + 5], p[8 * t + 6], p[8 * t + 7]};
  return acc + (((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7])));
}

// Bias registers of one key tile for one 32-query group. 16-bit: the B fragments of the
// identity MFMA, f[sub][t] = bias[q][sub*32 + 16t + 8g + 0..7]. fp32: the values the lane
// adds on the VALU, f[sub][rg] = bias[q][sub*32 + 8rg + 4g + 0..3].
template <typename T> struct BiasFrag {
  typename TypeOps<T>::V8 f[2][2];
};
template <> struct BiasFrag<float> {
  f32x4 f[2][4];
};

// brow is the bias row of the lane's query (row 0 for queries past N, whose results are
// never stored). Keys of a tile that reaches past N are zero-filled; inside the row pitch
// either way (the host pads it to a multiple of 8).
template <typename T>
__device__ __forceinline__ void load_bias(BiasFrag<T>& bf, const T* brow, bool qok, int kbase, int N,
                                          int g) {
  (void)qok;
  if (kbase + KT <= N) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int t = 0; t < 2; ++t) bf.f[sub][t] = load8(brow + kbase + sub * 32 + 16 * t + 8 * g);
    return;
  }
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key = kbase + sub * 32 + 16 * t + 8 * g;
      bf.f[sub][t] = load8_bias_tail<T>(brow, key, N);
    }
}
template <>
__device__ __forceinline__ void load_bias<float>(BiasFrag<float>& bf, const float* brow, bool qok, int kbase,
                                                 int N, int g) {
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int key = kbase + sub * 32 + 8 * rg + 4 * g;
      bf.f[sub][rg] = (qok && key < N) ? load4(brow + key) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
}

// fp32 bias fragments with every load issued: keys past N read key N - 1 and queries past
// N read row 0 (brow), then take zero, the values load_bias<float> gives them. With the loads
// under a condition the compiler's memory-counter wait for them, at the join, also waits for
// the next tile's K / V loads issued before them.
__device__ __forceinline__ void load_bias_f32_all(BiasFrag<float>& bf, const float* brow, bool qok, int kbase,
                                                  int N, int g) {
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int key = kbase + sub * 32 + 8 * rg + 4 * g;
      const f32x4 v = load4(brow + min(key, N - 1));
      const bool ok = qok && key < N;
#pragma unroll
      for (int e = 0; e < 4; ++e) bf.f[sub][rg][e] = ok ? v[e] : 0.f;
    }
}

enum RowState { ROW_LIVE = 0, ROW_DEAD = 1, ROW_ABSENT = 2 };

// fp32 under the bf16x3 split with DP = 32 runs at GNN_ATTN_X3_WAVES waves per SIMD; above
// two it loads each tile's bias fragments at the top of that tile (not a tile ahead), which
// frees the 32 registers the early copy holds for the whole key loop.
#ifndef GNN_ATTN_X3_WAVES
#define GNN_ATTN_X3_WAVES 3
#endif
// fp32 with DP = 128: workgroups per CU the register allocation is held to. At 2 (256
// registers) the kernel spills 129 registers with a bias; one workgroup per CU measured faster
// (N = 256, 256 rows, H = 4, bias: 449 against 463 us under 'ieee', 316 against 379 under
// 'tf32'). 16-bit inputs keep 2 (16 spilled registers with a bias; one workgroup: 150 against
// 138 us).
#ifndef GNN_ATTN_F32_DP128_BLOCKS
#define GNN_ATTN_F32_DP128_BLOCKS 1
#endif
template <typename T, int PREC, int DP>
__host__ __device__ constexpr int attn_min_blocks() {
  // DP = 256 (16-bit only): one workgroup per CU, the 128 O accumulator registers of a wave
  // in AGPRs beside the q, K / V staging and score registers
  return DP > 128    ? 1
         : DP == 128 ? (sizeof(T) == 4 ? GNN_ATTN_F32_DP128_BLOCKS : GNN_ATTN_MINBLOCKS)
         : (sizeof(T) == 4 && PREC == PREC_BF16X3 && DP <= 32) ? GNN_ATTN_X3_WAVES
                                                               : GNN_ATTN_MINBLOCKS;
}

template <typename T, int PREC, int DP, bool HAS_BIAS>
__global__ __launch_bounds__(NTHREADS, (attn_min_blocks<T, PREC, DP>())) void triattn_fwd_kernel(const gnn_triattn_args a) {
  typedef typename TypeOps<T>::V8 V8;
  typedef typename TypeOps<T>::V4 V4;
  // fp32 under bf16x3, DP <= 64: q, K, V and P split into bf16 hi / lo halves once each
  constexpr bool X3 = sizeof(T) == 4 && PREC == PREC_BF16X3 && DP <= 64;
  typedef Smem<T, DP, X3> S;
  __shared__ S sm;
  constexpr bool BIAS_AHEAD = attn_min_blocks<T, PREC, DP>() <= 2;

  const int N = (int)a.N;
  const int H = (int)a.H;
  const int D = (int)a.D;
  const int nqb = (N + QB - 1) / QB;
  const int nsg = (int)((a.S + R - 1) / R);
  const uint32_t w = xcd_remap(blockIdx.x, gridDim.x);
  const int qb = w % nqb;
  const int h = (w / nqb) % H;
  const int64_t rest = w / ((uint32_t)nqb * H);
  const int s0 = (int)(rest % nsg) * R;
  const int b = (int)(rest / nsg);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int ntiles = (N + KT - 1) / KT;
  const int64_t ksn = a.k_stride[2], vsn = a.v_stride[2];

  const T* kp[R];
  const T* vp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = min(s0 + r, (int)a.S - 1);  // absent rows alias the last row, never used
    kp[r] = (const T*)a.k + b * a.k_stride[0] + s * a.k_stride[1] + h * a.k_stride[3];
    vp[r] = (const T*)a.v + b * a.v_stride[0] + s * a.v_stride[1] + h * a.v_stride[3];
  }

  // ---- key liveness per row: one 64-bit word per key tile, row states, and the tiles to run.
  if (wave == 0) {
    uint64_t any_live = 0;  // lane t%64 accumulates nothing; the list is built by lane 0
    int n = 0;
    bool some_dead = false;
    int nlive_row[R];
#pragma unroll
    for (int r = 0; r < R; ++r) nlive_row[r] = 0;
    for (int t = 0; t < ntiles; ++t) {
      const int key = t * KT + lane;
      uint64_t tile_any = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int s = s0 + r;
        bool live = key < N && s < a.S;
        if (live && a.mask) live = a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)key * a.mask_stride[2]] != 0;
        const uint64_t bits = __ballot(live);
        if (lane == 0) sm.tile_live[r][t] = bits;
        nlive_row[r] += bits != 0;
        tile_any |= bits;
      }
      if (lane == 0 && tile_any != 0) sm.tile_list[n] = (uint16_t)t;
      n += tile_any != 0;
    }
    (void)any_live;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int state = s0 + r >= a.S ? ROW_ABSENT : (nlive_row[r] == 0 ? ROW_DEAD : ROW_LIVE);
      some_dead |= state == ROW_DEAD;
      if (lane == 0) sm.row_dead[r] = state;
    }
    if (some_dead) {  // a row with no live key runs every tile
      for (int t = lane; t < ntiles; t += 64) sm.tile_list[t] = (uint16_t)t;
      n = ntiles;
    }
    if (lane == 0) sm.ntiles_run = n;
  }

  // ---- this wave's queries (the same 32 in every row): Q' fragments per row.
  const int myq = qb * QB + wave * 32 + l32;
  const bool qok = myq < N;
  const T* brow = HAS_BIAS ? (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] +
                                 (int64_t)(qok ? myq : 0) * a.bias_stride[2]
                           : nullptr;
  V8 qf[R][DP / 16];
  bf16x8 qh[R][DP / 16], ql[R][DP / 16];  // X3: the halves of Q'
  f32x16 o[R][DP / 32];
  float m[R], lsum[R], mx[R];  // mx: exact running maximum (m moves lazily)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = min(s0 + r, (int)a.S - 1);
    const T* qp = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3];
#pragma unroll
    for (int t = 0; t < DP / 16; ++t) {
      const int d0 = 16 * t + 8 * g;
      if (qok && d0 < D) {
        f32x8 x = TypeOps<T>::to_f32(load8(qp + myq * a.q_stride[2] + d0));
        if constexpr (X3)
          split_bf16(x * a.scale, qh[r][t], ql[r][t]);
        else
          qf[r][t] = TypeOps<T>::from_f32(x * a.scale);
      } else {
        if constexpr (X3)
          qh[r][t] = ql[r][t] = zero8<bf16>();
        else
          qf[r][t] = zero8<T>();
      }
    }
#pragma unroll
    for (int cc = 0; cc < DP / 32; ++cc)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[r][cc][i] = 0.f;
    m[r] = -INFINITY;
    mx[r] = -INFINITY;
    lsum[r] = 0.f;
  }

  // identity A-fragments for the bias MFMA: element e of lane group g in step t is key
  // 16t + 8g + e; row l32 of the identity holds a 1 there iff l32 is that key.
  V8 idf[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) idf[t][e] = TypeOps<T>::from_f32(l32 == 16 * t + 8 * g + e ? 1.f : 0.f);

  // ---- K / V^T staging: CH chunks of 8 elements of K and of V per thread and row.
  constexpr int CPK = DP / 8;
  constexpr int CH = KT * CPK / NTHREADS;
  V8 kreg[R][CH], vreg[R][CH];
  // chunk i of this thread: key kl[i] of the tile, head-dim columns dc[i] .. + 7; the
  // per-lane address parts are loop invariant
  int kl[CH], dc[CH];
  int64_t koff[CH], voff[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = tid + i * NTHREADS;
    kl[i] = c / CPK;
    dc[i] = (c % CPK) * 8;
    koff[i] = (int64_t)kl[i] * ksn + dc[i];
    voff[i] = (int64_t)kl[i] * vsn + dc[i];
  }
  auto load_kv = [&](int t) {
    if (DP == D && (R == 1 || s0 + R <= a.S)) {
      if (t * KT + KT <= N) {  // full tile: tile base (uniform) + lane part
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const T* kt = kp[r] + (int64_t)t * KT * ksn;
          const T* vt = vp[r] + (int64_t)t * KT * vsn;
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            kreg[r][i] = load8(kt + koff[i]);
            vreg[r][i] = load8(vt + voff[i]);
          }
        }
      } else {  // keys past N read row N-1: finite data whose scores become -inf, p = 0
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            const int key = min(t * KT + kl[i], N - 1);
            kreg[r][i] = load8(kp[r] + (int64_t)key * ksn + dc[i]);
            vreg[r][i] = load8(vp[r] + (int64_t)key * vsn + dc[i]);
          }
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int key = t * KT + kl[i];
        if (key < N && dc[i] < D && s0 + r < a.S) {
          kreg[r][i] = load8(kp[r] + (int64_t)key * ksn + dc[i]);
          vreg[r][i] = load8(vp[r] + (int64_t)key * vsn + dc[i]);
        } else {
          kreg[r][i] = zero8<T>();
          vreg[r][i] = zero8<T>();
        }
      }
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int c = tid + i * NTHREADS;
        const int kl = c / CPK;
        const int d0 = (c % CPK) * 8;
        if constexpr (X3) {
          bf16x8 hi, lo;
          split_bf16(kreg[r][i], hi, lo);
          store8(&sm.k[buf][r][0][kl * S::KROW + d0], hi);
          store8(&sm.k[buf][r][1][kl * S::KROW + d0], lo);
          split_bf16(vreg[r][i], hi, lo);
          store8(&sm.vt[buf][r][0][kl * S::VROW + d0], hi);
          store8(&sm.vt[buf][r][1][kl * S::VROW + d0], lo);
        } else {
          store8(&sm.k[buf][r][0][kl * S::KROW + d0], kreg[r][i]);
          if constexpr (S::VTR) {
            store8(&sm.vt[buf][r][0][kl * S::VROW + d0], vreg[r][i]);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) sm.vt[buf][r][0][(d0 + e) * S::VROW + kl] = vreg[r][i][e];
          }
        }
      }
  };
  // V^T A fragment (16-bit types) of k-step kk of sub-tile sub, head-dim block cc: lane l
  // gets d = 32cc + l % 32 and keys sub*32 + 16kk + 8h + 4g + e (element 4h + e). Each
  // ds_read_b64_tr_b16 hands the 16 lanes of a group a 16 (d) x 4 (key) block: lane r of the
  // group addresses key kb + r / 4, d 16 * ((l / 16) % 2) + 4 * (r % 4) .. + 3, and receives
  // the 4 keys of column d = l % 16 of that block.
  const int tr_r = lane & 15;
  const int tr_off = (tr_r >> 2) * S::VROW + 16 * ((lane >> 4) & 1) + 4 * (tr_r & 3);

  __syncthreads();
  const int nrun = sm.ntiles_run;
  int state[R];
#pragma unroll
  for (int r = 0; r < R; ++r) state[r] = sm.row_dead[r];
  const float mval = a.mask_value;

  BiasFrag<T> bias0;  // this tile's fragments; refilled with the next tile's once used
  if (nrun > 0) {
    const int t0 = sm.tile_list[0];
    load_kv(t0);
    if constexpr (HAS_BIAS && BIAS_AHEAD) load_bias<T>(bias0, brow, qok, t0 * KT, N, g);
    store_kv(0);
  }
  __syncthreads();

  // lane l ^ 32 for the pair maximum, as a ds_bpermute byte index (loop invariant)
  const int xlane = (lane ^ 32) << 2;

  for (int it = 0; it < nrun; ++it) {
    BiasFrag<T>& bc = bias0;
    const int cur = S::NBUF == 2 ? (it & 1) : 0;
    const int t = sm.tile_list[it];
    const bool has_next = it + 1 < nrun;
    const int tn = has_next ? sm.tile_list[it + 1] : t;
    if constexpr (X3 && HAS_BIAS && !BIAS_AHEAD) {
      // this tile's bias before the next tile's K / V (the last tile loads itself again), all
      // unconditional, so the wait for the bias leaves K / V in flight: 181 -> 177 us at C5
      // N = 384 under 'tf32'; under 'ieee' the same change measured 328 -> 349 us
      load_bias_f32_all(bc, brow, qok, t * KT, N, g);
      load_kv(tn);
    } else {
      if (has_next) load_kv(tn);
      if constexpr (HAS_BIAS && !BIAS_AHEAD) load_bias<T>(bc, brow, qok, t * KT, N, g);
    }
    bool bias_next = false;  // bc already holds the next tile's bias

#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint64_t live = sm.tile_live[r][t];
      const bool dead = state[r] == ROW_DEAD;
      if (state[r] == ROW_ABSENT || (!dead && live == 0)) continue;

      // S^T (+ bias): sc[sub][i] is key t*64 + sub*32 + 8*(i/4) + 4g + i%4, query myq.
      f32x16 sc[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) sc[sub][i] = 0.f;
      if constexpr (X3) {  // lo * hi + hi * lo + hi * hi
#pragma unroll
        for (int kk = 0; kk < DP / 16; ++kk)
#pragma unroll
          for (int sub = 0; sub < 2; ++sub) {
            const int off = (sub * 32 + l32) * S::KROW + 16 * kk + 8 * g;
            const bf16x8 kh = load8(&sm.k[cur][r][0][off]), klo = load8(&sm.k[cur][r][1][off]);
            sc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(klo, qh[r][kk], sc[sub], 0, 0, 0);
            sc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, ql[r][kk], sc[sub], 0, 0, 0);
            sc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qh[r][kk], sc[sub], 0, 0, 0);
          }
      } else {
        const T* ks = sm.k[cur][r][0];
#pragma unroll
        for (int kk = 0; kk < DP / 16; ++kk)
#pragma unroll
          for (int sub = 0; sub < 2; ++sub)
            Mma<T, PREC>::step(sc[sub], load8(&ks[(sub * 32 + l32) * S::KROW + 16 * kk + 8 * g]), qf[r][kk]);
      }
      if constexpr (HAS_BIAS) {
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) Mma<T, PREC>::step(sc[sub], idf[t2], bc.f[sub][t2]);
        } else {
#pragma unroll
          for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg)
#pragma unroll
              for (int e = 0; e < 4; ++e) sc[sub][4 * rg + e] += TypeOps<T>::to_f32(bc.f[sub][rg][e]);
        }
        if (BIAS_AHEAD && R == 1 && has_next) {  // the next tile's fragments, as early as possible
          load_bias<T>(bc, brow, qok, tn * KT, N, g);
          bias_next = true;
        }
      }
      if (live != ~0ull) {
        // some key of the tile is masked or past N. Bit 8*(i/4) + i%4 of lb / vb is key
        // sub*32 + 8*(i/4) + 4g + i%4 of the tile.
        const int nvalid = min(KT, N - t * KT);
        const uint64_t valid = nvalid >= 64 ? ~0ull : ((1ull << nvalid) - 1ull);
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          const uint32_t lb = ((uint32_t)(live >> (32 * sub)) >> (4 * g)) & 0x0F0F0F0Fu;
          const uint32_t vb = ((uint32_t)(valid >> (32 * sub)) >> (4 * g)) & 0x0F0F0F0Fu;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int bit = 8 * (i / 4) + (i % 4);
            const float x = ((lb >> bit) & 1u) ? sc[sub][i] : sc[sub][i] + mval;
            sc[sub][i] = ((vb >> bit) & 1u) ? x : -INFINITY;
          }
        }
      }

      // online softmax, lazily rescaled
      float m0 = fmaxf(sc[0][0], sc[0][1]), m1 = fmaxf(sc[1][0], sc[1][1]);
#pragma unroll
      for (int i = 2; i < 16; ++i) {
        m0 = fmaxf(m0, sc[0][i]);
        m1 = fmaxf(m1, sc[1][i]);
      }
      const float mh = fmaxf(m0, m1);
      const float mt = fmaxf(mh, __int_as_float(__builtin_amdgcn_ds_bpermute(xlane, __float_as_int(mh))));
      mx[r] = fmaxf(mx[r], mt);
      if (__any(mt > m[r] + RESCALE_THRESHOLD)) {
        const float mnew = fmaxf(m[r], mt);
        const float alpha = fast_exp2((m[r] - mnew) * LOG2E);  // 0 on the first tile (m = -inf)
        m[r] = mnew;
        lsum[r] *= alpha;
#pragma unroll
        for (int cc = 0; cc < DP / 32; ++cc)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[r][cc][i] *= alpha;
      }
      V8 pf[2][2];
      bf16x8 ph[2][2], pl[2][2];  // X3: the halves of P^T
      const float nm = -m[r] * LOG2E;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        if ((sizeof(T) == 2 || X3) && !dead) {
          // the folded FMA leaves a residual below half an ulp of s * log2 e; after the
          // 16-bit rounding of p the row maximum still maps to exactly 1 (under the bf16x3
          // split the residual, a relative 2^-24 of s * log2 e, is far below the split's
          // own error on the scores)
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[sub][i] = fast_exp2(__builtin_fmaf(sc[sub][i], LOG2E, nm));
        } else {  // fp32, or m is the collapsed sentinel: subtract first so s - m is exact
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[sub][i] = fast_exp2((sc[sub][i] - m[r]) * LOG2E);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          if constexpr (X3)
            split_bf16(frag_from_acc<float>(sc[sub], kk), ph[sub][kk], pl[sub][kk]);
          else
            pf[sub][kk] = frag_from_acc<T>(sc[sub], kk);
          lsum[r] = rowsum_add(sc[sub], kk, lsum[r]);
        }
      }

      // O^T += V^T P^T. Fragment element e of k-step kk of sub-tile sub is key
      // sub*32 + 16*kk + 8*(e/4) + 4g + e%4 in both operands.
      if constexpr (X3) {
#pragma unroll
        for (int cc = 0; cc < DP / 32; ++cc)
#pragma unroll
          for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
              const int off = (sub * 32 + 16 * kk + 4 * g) * S::VROW + 32 * cc + tr_off;
              bf16x8 vh, vl;
#pragma unroll
              for (int p = 0; p < 2; ++p) {
                const bf16* vb = &sm.vt[cur][r][p][off];
                const bf16x4 lo4 = tr_read4<bf16>(vb), hi4 = tr_read4<bf16>(vb + 8 * S::VROW);
                bf16x8& vf = p == 0 ? vh : vl;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  vf[e] = lo4[e];
                  vf[e + 4] = hi4[e];
                }
              }
              o[r][cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl, ph[sub][kk], o[r][cc], 0, 0, 0);
              o[r][cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, pl[sub][kk], o[r][cc], 0, 0, 0);
              o[r][cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, ph[sub][kk], o[r][cc], 0, 0, 0);
            }
      } else {
        const T* vs = sm.vt[cur][r][0];
#pragma unroll
        for (int cc = 0; cc < DP / 32; ++cc)
#pragma unroll
          for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
              V4 lo, hi;
              if constexpr (S::VTR) {
                const T* vb = &vs[(sub * 32 + 16 * kk + 4 * g) * S::VROW + 32 * cc + tr_off];
                lo = tr_read4<T>(vb);
                hi = tr_read4<T>(vb + 8 * S::VROW);
              } else {
                const T* vrow = &vs[(32 * cc + l32) * S::VROW + sub * 32 + 16 * kk + 4 * g];
                lo = load4(vrow);
                hi = load4(vrow + 8);
              }
              V8 vf;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                vf[e] = lo[e];
                vf[e + 4] = hi[e];
              }
              Mma<T, PREC>::step(o[r][cc], vf, pf[sub][kk]);
            }
      }
    }

    if (BIAS_AHEAD && HAS_BIAS && has_next && !bias_next) load_bias<T>(bc, brow, qok, tn * KT, N, g);
    if constexpr (S::NBUF == 2) {
      // the other stage was last read in the previous iteration, before its barrier
      if (has_next) store_kv(cur ^ 1);
      __syncthreads();
    } else {
      __syncthreads();
      if (has_next) store_kv(0);
      __syncthreads();
    }
  }

  // ---- normalise and store. o[r][cc][i] is O[s0 + r][myq][32cc + 8*(i/4) + 4g + i%4].
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float ltot = pair_sum(lsum[r]);
    if (!qok || state[r] == ROW_ABSENT) continue;
    const float inv = 1.0f / ltot;
    const int s = s0 + r;
    T* orow = (T*)a.o + b * a.o_stride[0] + s * a.o_stride[1] + h * a.o_stride[3] + (int64_t)myq * a.o_stride[2];
#pragma unroll
    for (int cc = 0; cc < DP / 32; ++cc)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int d0 = 32 * cc + 8 * rg + 4 * g;
        if (d0 < D) {
          f32x4 x = {o[r][cc][4 * rg] * inv, o[r][cc][4 * rg + 1] * inv, o[r][cc][4 * rg + 2] * inv,
                     o[r][cc][4 * rg + 3] * inv};
          store4(orow + d0, TypeOps<T>::from_f32(x));
        }
      }
    const int64_t ridx = (((int64_t)b * a.S + s) * H + h) * N + myq;
    if (a.lse && g == 0) a.lse[ridx] = m[r] + __log2f(ltot) * (1.0f / LOG2E);  // natural-log lse
    if (a.row_max && g == 0) a.row_max[ridx] = mx[r];
  }
}

template <typename T, int PREC, bool HAS_BIAS>
int launch_bias(const gnn_triattn_args& a, hipStream_t stream) {
  const int64_t nqb = (a.N + QB - 1) / QB;
  const int64_t nblk = nqb * a.H * ((a.S + R - 1) / R) * a.B;
  dim3 grid((uint32_t)nblk), block(NTHREADS);
  if (a.D <= 32)
    hipLaunchKernelGGL((triattn_fwd_kernel<T, PREC, 32, HAS_BIAS>), grid, block, 0, stream, a);
  else if (a.D <= 64)
    hipLaunchKernelGGL((triattn_fwd_kernel<T, PREC, 64, HAS_BIAS>), grid, block, 0, stream, a);
  else if (a.D <= 128)
    hipLaunchKernelGGL((triattn_fwd_kernel<T, PREC, 128, HAS_BIAS>), grid, block, 0, stream, a);
  else if constexpr (sizeof(T) == 2)
    hipLaunchKernelGGL((triattn_fwd_kernel<T, PREC, 256, HAS_BIAS>), grid, block, 0, stream, a);
  return (int)hipGetLastError();
}

template <typename T, int PREC>
int launch_dp(const gnn_triattn_args& a, hipStream_t stream) {
  return a.bias ? launch_bias<T, PREC, true>(a, stream) : launch_bias<T, PREC, false>(a, stream);
}

}  // namespace

int triattn_fwd(const gnn_triattn_args& a, hipStream_t stream) {
  if (a.N > (int64_t)MAX_TILES * KT)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention: N_res > 32768 is not supported");
  if (a.D > 256)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention: head dim > 256 is not supported");
  if (a.D > 128 && a.dtype == GNN_F32)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention: fp32 head dim > 128 is not supported");
  const int64_t nqb = (a.N + QB - 1) / QB;
  if (nqb * a.H * ((a.S + R - 1) / R) * a.B >= (int64_t)1 << 31)
    return set_error(GNN_ERR_UNSUPPORTED, "triangle_attention: grid too large");
  if (triattn_row_applicable(a)) return triattn_row_fwd(a, stream);
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
