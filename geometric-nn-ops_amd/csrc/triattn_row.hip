// Triangle attention forward for gfx950, row-resident variant: 16-bit inputs, head dim
// <= 32, N_res <= ROW_MAX_N.
//
// Same mathematics as the tiled kernel (triattn_fwd.hip) and the reference forward
// (geometric_nn_ops_torch/triangle/_kernels/triangle_attention.py:48-365, torch form
// geometric_nn_ops_torch/triangle/_reference/triangle_attention.py:11-44):
//   o[b,s,i,h,:] = sum_j softmax_j(l_ij) v[b,s,j,h,:],
//   l_ij = bf16(q * scale) . k_j + bias[b,h,i,j] + mask_bias[b,s,j].
//
// What changes is the schedule. At D = 32 one (b, s, h) row of K and V is N * 128 bytes
// (64 KB at N = 512), so a workgroup stages the WHOLE row of K and V in LDS once and its
// waves then sweep every key tile with no barrier at all:
//   * one workgroup per (b, s, h); its NW waves take the row's 32-query blocks round robin
//     (8 waves while two rows fit a CU's 160 KB of LDS, 16 once a row needs more than 80 KB,
//     N > 576, so that a CU still runs 4 waves per SIMD);
//   * K rows are 64 bytes with the four 16-byte chunks XOR-swizzled by (key / 4) % 4, so the
//     32-lane fragment reads of QK^T hit 16 distinct bank groups; V keeps [key][d] rows for
//     the ds_read_b64_tr_b16 V^T fragments of PV (a 64-byte pitch puts the four row windows
//     of one read pass on disjoint banks);
//   * K and V arrive by global_load_lds (global -> LDS without registers) when D = 32;
//   * the pair-bias fragments of tile t+1 are requested from global memory (L2: the plane
//     bias[b, h] is shared by every N_seq row) while tile t is computed;
//   * the pair maximum of the online softmax uses v_permlane32_swap (no LDS round trip), and
//     rows without a masked key run their tiles in order with arithmetic liveness, so the
//     key loop reads nothing from LDS but K and V;
//   * logical workgroup order (b, head pair, s, head in pair), remapped so each XCD walks a
//     contiguous range: the two heads of a pair share the 128-byte lines of the K and V rows
//     and an XCD's L2 holds just their two bias planes (248 MB fetched from beyond L2 per
//     launch at N = 512 against 309 MB with all four heads fastest). Odd H falls back to heads
//     fastest (when the planes fit the L2 together) or rows fastest.
// Measured alternatives not kept: 4 waves per workgroup (the staging then is not amortised),
// software pipelining the QK^T of the next tile (or 32-key half tile) ahead of the softmax
// (the extra score registers cost occupancy and it measured slower), and a persistent form
// (16 waves per CU streaming consecutive rows through two LDS buffers, the next row's K / V
// DMA issued during the current row's key loop: 20% slower at N = 512, its 16 waves meeting
// at a barrier every row), and unconditional buffer stores for o and lse (so that the wait for
// the next query block's q, requested during the sweep, would not cover them: the offsets
// spilled 4 registers at the 128-register cap, 157 against 148 us).
// Per tile: the transposed score tile S^T = K Q'^T on 32x32x16 MFMA, the pair bias added by
// MFMA against an identity fragment, and, on tiles with a masked key or keys past N, the
// per-key mask term (0 / mask_value / -inf from a per-row table in LDS) added by one more
// MFMA per 32-key half (a rank-1 product: the term in column 0 of A times ones in row 0 of B),
// so masking costs no per-score VALU work. The softmax is evaluated against a reference
// maximum m taken from the row's first tile only: p = exp2((s - m) log2 e) may then exceed 1
// on later tiles, which costs nothing in precision (bf16 / fp32 are relative) and removes the
// per-tile maximum reduction. A query block whose row sum ends above what the type holds
// (2^64 for bf16, 65504 for fp16: p or the accumulators could have overflowed) is
// recomputed with the per-tile maximum and lazy rescale (threshold 8 ln 2); callers asking
// for the exact row maximum have every tile's maximum reduced on the same fast sweep. exp2
// with the folded FMA, row sums of the fp32 probabilities before they are rounded for the PV
// product (as the reference's tl.sum(P_block, 1); v_add_f32, which issues alongside other
// waves' MFMAs where v_dot2 would hold the matrix pipe), and rows whose keys are all masked
// reproducing mean(v) (the sentinel swamps the logits; subtract first) are as in the tiled
// kernel, which gives the same results to rounding.
#include <algorithm>
#include <mutex>

#include "gnn_common.hpp"
#include "gnn_internal.hpp"

namespace gnn {

namespace {

constexpr int KT = 64;                 // keys per tile
constexpr int ROW_BYTES = 64;          // one key row of K or V: 32 x 16-bit
constexpr int TILE_BYTES = KT * ROW_BYTES;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_THRESHOLD = 8.0f / LOG2E;

#ifndef GNN_ROW_WAVES_PER_SIMD  // occupancy the register allocation is held to (128 VGPRs at 4)
#define GNN_ROW_WAVES_PER_SIMD 4
#endif
#ifndef GNN_ROW_SETPRIO
#define GNN_ROW_SETPRIO 1
#endif
#ifndef GNN_ROW_MAX_N
#define GNN_ROW_MAX_N 1024
#endif
#ifndef GNN_ROW_KPREFETCH  // next tile's K fragments read from LDS during the current softmax
#define GNN_ROW_KPREFETCH 0   // measured slower: the extra live fragments spill at 128 VGPRs
#endif
#ifndef GNN_ROW_VPREFETCH  // a 32-key half's V^T fragments read before its exponentials
#define GNN_ROW_VPREFETCH 0   // measured neutral
#endif
#ifndef GNN_ROW_QPREFETCH  // 1: a wave's first q requested with the K / V staging, and (no-bias
#define GNN_ROW_QPREFETCH 1   // kernel) the next block's q during the current sweep; 2: that also
#endif                        // with bias (spills at 128 VGPRs); 0: each q loaded where it is used
#ifndef GNN_ROW_STAGGER  // the first workgroups run half a row (the other halves run last)
#define GNN_ROW_STAGGER 1
#endif
#ifndef GNN_ROW_HEADS_FIRST_BYTES
#define GNN_ROW_HEADS_FIRST_BYTES (8 << 20)
#endif
constexpr int64_t ROW_HEADS_FIRST_BYTES = GNN_ROW_HEADS_FIRST_BYTES;
#ifndef GNN_ROW_HEAD_PAIRS
#define GNN_ROW_HEAD_PAIRS 1
#endif
constexpr bool ROW_HEAD_PAIRS = GNN_ROW_HEAD_PAIRS;
// waves of a workgroup: 8 while two workgroups fit the CU's LDS, else 16
constexpr size_t ROW_TWO_PER_CU_BYTES = 80 * 1024;
// 1: 12-wave workgroups (3 per SIMD) for rows of 12 k query blocks, so that no wave idles in
// a half-empty second round (N = 768: 24 blocks on 16 waves). Measured slower: 462 against
// 434 us at C4 (N = 768, ragged), 494 against 470 us at N = 768 without a mask; the 16 waves
// keep 4 per SIMD through the first round, which outweighs the idle half of the second.
#ifndef GNN_ROW_W12
#define GNN_ROW_W12 0
#endif
constexpr int ROW_MAX_TILES = (GNN_ROW_MAX_N + KT - 1) / KT;

struct RowHdr {
  uint64_t tile_live[ROW_MAX_TILES];  // bit j: key t*64+j is < N and unmasked
  uint16_t tile_list[ROW_MAX_TILES];  // tiles to run (all of them when the row is dead)
  int nrun;
  int dead;  // the row has no live key
  int full;  // every key < N is live (no masked key): tiles run in order, liveness is arithmetic
};
constexpr int HDR_BYTES = (int)((sizeof(RowHdr) + 255) / 256 * 256);
// per-key additive mask term of the row, one 16-bit value per key of every tile
__host__ __device__ constexpr int mask_table_bytes(int ntiles) { return (ntiles * KT * 2 + 255) / 256 * 256; }

size_t row_smem_bytes(int64_t N) {
  const int ntiles = (int)((N + KT - 1) / KT);
  return HDR_BYTES + mask_table_bytes(ntiles) + 2 * (size_t)ntiles * TILE_BYTES;
}

// Query blocks whose row sum ends above this are recomputed with the per-tile maximum. A
// lane's row sum bounds every probability it rounded for the PV product, so the limit is what
// the MFMA type and the fp32 accumulators hold: fp16 rounds p above 65504 to inf (a logit
// ln 65504 = 11.1 above the first tile's maximum already does), bf16 keeps 2^64 finite with
// room for the products with v.
template <typename T> struct FastLimit { static constexpr float value = 18446744073709551616.0f; };  // 2^64
template <> struct FastLimit<f16> { static constexpr float value = 65504.0f; };

template <typename T> struct BiasFragR {
  typename TypeOps<T>::V8 f[2][2];  // f[sub][t] = bias[q][tile*64 + sub*32 + 16t + 8g + 0..7]
};

// The pair bias in fragment order. bias[b, h] is shared by every N_seq row, so a launch
// reads it S times; in the caller's row-major layout one 16-byte fragment load per lane
// touches 32 query rows (32 cache lines for 1 KB) and those loads are bound by the L1's
// line rate. A pre-pass writes each (b, h, 32-query block, 64-key tile) as 4 KB in the
// order the fragments are consumed: fragment f = 2 sub + t of lane l at byte
// 1024 f + 16 l. Every fragment load is then one contiguous 1 KB range, and queries or keys
// past N hold zeros (the identity MFMA multiplies every loaded value, so padding must be
// finite).
constexpr int BIAS_TILE_ELEMS = 2048;  // 4 KB of 16-bit values per (query block, key tile)

int64_t bias_tile_count(int64_t B, int64_t H, int64_t N) {
  const int64_t nqb = (N + 31) / 32, ntiles = (N + KT - 1) / KT;
  return B * H * nqb * ntiles;
}

template <typename T>
__device__ __forceinline__ void load_bias_tile(BiasFragR<T>& bf, const T* tile) {
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int t = 0; t < 2; ++t) bf.f[sub][t] = load8_global(tile + (2 * sub + t) * 512);
}

// One thread per 16-byte chunk of the caller's bias, taken in row-major order within each
// 32 x 64 tile (8 consecutive threads read one 128-byte query row) and written to its slot in
// fragment order: chunk c = key / 8 of query row r goes to fragment f = 2 (c / 4) + (c / 2) % 2,
// lane r + 32 (c % 2). Tile id ((b H + h) nqb + query block) ntiles + key tile. Any strides;
// 16-byte loads where the row chunk is unit-stride, aligned and inside N.
template <typename T>
__global__ __launch_bounds__(256) void bias_tiles_kernel(const gnn_triattn_args a, T* tiles, int64_t nchunks) {
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= nchunks) return;
  const int N = (int)a.N, H = (int)a.H;
  const int nqb = (N + 31) / 32, ntiles = (N + KT - 1) / KT;
  const int i = (int)(id & 255), r = i >> 3, c = i & 7;
  int64_t rest = id >> 8;
  const int t = (int)(rest % ntiles);
  rest /= ntiles;
  const int qb = (int)(rest % nqb);
  rest /= nqb;
  const int h = (int)(rest % H);
  const int64_t b = rest / H;
  const int q = qb * 32 + r, key0 = t * KT + 8 * c;
  typename TypeOps<T>::V8 v = zero8<T>();
  if (q < N) {
    const T* p = (const T*)a.bias + b * a.bias_stride[0] + h * a.bias_stride[1] + (int64_t)q * a.bias_stride[2] +
                 (int64_t)key0 * a.bias_stride[3];
    if (a.bias_stride[3] == 1 && key0 + 8 <= N && ((uintptr_t)p & 15) == 0) {
      v = load8(p);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (key0 + e < N) v[e] = p[(int64_t)e * a.bias_stride[3]];
    }
  }
  const int f = 2 * (c >> 2) + ((c >> 1) & 1), lane = r + 32 * (c & 1);
  store8(tiles + (((id >> 8) * 4 + f) * 64 + lane) * 8, v);
}

// acc + the sum of 8 fp32 probabilities (a pairwise tree, so the add chain per tile is short)
__device__ __forceinline__ float rowsum_add_r(const f32x8& x, float acc) {
  return acc + (((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7])));
}

// Maxima of scores, which are finite or -inf (never NaN): v_max3_f32 / v_max_f32 written
// directly, because fmaxf's NaN rules make the compiler quiet each operand first (an extra
// v_max_f32 x, x, x per operand in the reduction tree).
__device__ __forceinline__ float max3_nn(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max_nn(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// The compiler places the wait states an MFMA result needs before a VALU instruction reads it
// (12 for a 32x32x16 MFMA) only in front of instructions it generates, not in front of inline
// assembly. max3_nn / max_nn read the score accumulators straight after the QK^T MFMAs, so
// this fence comes first: tied to the accumulators (it is placed after the MFMAs that write
// them), it supplies 16 wait states. Without it the maxima sometimes saw accumulators still
// being written, and the results changed from call to call in their last bits.
__device__ __forceinline__ void mfma_result_fence(f32x16& a, f32x16& b) {
  asm volatile("s_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b));
}

// max / sum over the lane pair (l, l ^ 32) with gfx950's v_permlane32_swap (no LDS trip)
__device__ __forceinline__ float pair_max_swap(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_nn(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum_swap(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V4 tr_read4_r(const unsigned char* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(__attribute__((address_space(3))) const unsigned char*)p);
  return __builtin_bit_cast(typename TypeOps<T>::V4, v);
}

// WMAX: the caller asked for the exact row maximum (a separate instantiation, so that the
// common one carries no maximum tracking in its fast sweep: it would spill at 128 VGPRs)
template <typename T, bool HAS_BIAS, int NW, bool WMAX>
__global__ __launch_bounds__(NW * 64, GNN_ROW_WAVES_PER_SIMD) void triattn_row_kernel(const gnn_triattn_args a) {
  constexpr int NT = NW * 64;
  constexpr bool QPF_SWEEP = GNN_ROW_QPREFETCH && (GNN_ROW_QPREFETCH == 2 || !HAS_BIAS);
  typedef typename TypeOps<T>::V8 V8;
  typedef typename TypeOps<T>::V4 V4;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ __align__(256) unsigned char smem_raw[];
  RowHdr& hdr = *reinterpret_cast<RowHdr*>(smem_raw);

  const int N = (int)a.N;
  const int H = (int)a.H;
  const int D = (int)a.D;
  const int S = (int)a.S;
  const int ntiles = (N + KT - 1) / KT;
  uint16_t* mbt = reinterpret_cast<uint16_t*>(smem_raw + HDR_BYTES);
  unsigned char* ks = smem_raw + HDR_BYTES + mask_table_bytes(ntiles);
  unsigned char* vs = ks + ntiles * TILE_BYTES;

  // Logical order: heads fastest when all H bias planes of a batch fit one XCD's L2
  // together (the XCD then reads whole 4-head key rows of K and V), rows fastest otherwise
  // (an XCD then keeps a single bias plane).
  // Workgroups [0, nsplit) run the first half of their row's query blocks and workgroups
  // [nrows, nrows + nsplit) the second half of the same rows, so that the first workgroups
  // end half a row early and the two workgroups of a CU stage their rows at different times.
  const uint32_t nrows = (uint32_t)(a.B * a.S * a.H);
  uint32_t bid = blockIdx.x;
  int qhalf = 0;  // 0: every query block, 1: the first half, 2: the second half
  if (gridDim.x > nrows) {
    if (bid < gridDim.x - nrows) qhalf = 1;
    else if (bid >= nrows) { bid -= nrows; qhalf = 2; }
  }
  const uint32_t w = xcd_remap(bid, nrows);
  int s, h;
  if (ROW_HEAD_PAIRS && H % 2 == 0) {
    // head pairs fastest: the two heads of a pair share the 128-byte lines of K and V rows
    // (D = 32, 16-bit), and an XCD keeps only their two bias planes
    const uint32_t hi = w & 1u, rest = w >> 1;
    s = (int)(rest % (uint32_t)S);
    h = 2 * (int)((rest / (uint32_t)S) % (uint32_t)(H / 2)) + (int)hi;
  } else if (a.H * a.N * a.N * (int64_t)sizeof(T) <= ROW_HEADS_FIRST_BYTES) {
    h = (int)(w % (uint32_t)H);
    s = (int)((w / (uint32_t)H) % (uint32_t)S);
  } else {
    s = (int)(w % (uint32_t)S);
    h = (int)((w / (uint32_t)S) % (uint32_t)H);
  }
  const int b = (int)(w / ((uint32_t)S * H));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int l32 = lane & 31;
  const int g = lane >> 5;

  // q of query block qb for this lane, unconditionally loaded (row clamped to N - 1, columns
  // past D read from column 0 and zeroed when used)
  const int nqb = (N + 31) / 32;
  const int qlo = qhalf == 2 ? nqb / 2 : 0, qhi = qhalf == 1 ? nqb / 2 : nqb;
  const int q0 = qlo + wave;  // this wave's first query block
  const T* qrow = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3];
  auto load_q = [&](typename TypeOps<T>::V8 (&qr)[2], int qb) {
    const T* qp = qrow + (int64_t)min(qb * 32 + l32, N - 1) * a.q_stride[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int d0 = 16 * t + 8 * g;
      qr[t] = load8(qp + (d0 < D ? d0 : 0));
    }
  };
  typename TypeOps<T>::V8 qraw[2];

  const int64_t ksn = a.k_stride[2], vsn = a.v_stride[2];
  const T* kp = (const T*)a.k + b * a.k_stride[0] + s * a.k_stride[1] + h * a.k_stride[3];
  const T* vp = (const T*)a.v + b * a.v_stride[0] + s * a.v_stride[1] + h * a.v_stride[3];

  // ---- stage the row's K (swizzled) and V into LDS.
  if (D == 32) {
    // global_load_lds_dwordx4: one instruction moves 16 key rows (1 KB) straight into LDS,
    // lane l filling bytes 16 l .. 16 l + 15, i.e. row l / 4, physical chunk l % 4. For K that
    // slot holds logical chunk (l % 4) ^ ((row / 4) % 4), and (row / 4) % 4 = (l / 16) % 4
    // because blocks start at multiples of 16 rows. Rows past N repeat row N - 1: finite
    // values whose scores are masked to -inf (p = 0).
    const int lrow = lane >> 2, lch = lane & 3;
    const int kch = lch ^ ((lane >> 4) & 3);
    const int nblk16 = ntiles * (KT / 16);
    for (int q = wave; q < nblk16; q += NW) {
      const int r = min(16 * q + lrow, N - 1);
      __builtin_amdgcn_global_load_lds((const void*)(kp + (int64_t)r * ksn + 8 * kch),
                                       (__attribute__((address_space(3))) void*)(ks + q * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vp + (int64_t)r * vsn + 8 * lch),
                                       (__attribute__((address_space(3))) void*)(vs + q * 1024), 16, 0, 0);
    }
    // the wave's first query block's q, behind its staging so that it lands with it
    if (GNN_ROW_QPREFETCH && q0 < qhi) load_q(qraw, q0);
  } else {
    // D < 32: through registers, so that columns D .. 31 are zero. Chunk c = key c / 4,
    // columns 8 (c % 4) .. + 7; rows past N are zero.
    constexpr int U = 4;
    const int nchunks = ntiles * KT * 4;
    for (int base = 0; base < nchunks; base += NT * U) {
      V8 kr[U], vr[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = base + u * NT + tid;
        const int key = c >> 2, d0 = (c & 3) * 8;
        if (c < nchunks && key < N && d0 < D) {
          kr[u] = load8(kp + (int64_t)key * ksn + d0);
          vr[u] = load8(vp + (int64_t)key * vsn + d0);
        } else {
          kr[u] = zero8<T>();
          vr[u] = zero8<T>();
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = base + u * NT + tid;
        if (c < nchunks) {
          const int key = c >> 2, cc = c & 3;
          store8((T*)(ks + key * ROW_BYTES + 16 * (cc ^ ((key >> 2) & 3))), kr[u]);
          store8((T*)(vs + key * ROW_BYTES + 16 * cc), vr[u]);
        }
      }
    }
    if (GNN_ROW_QPREFETCH && q0 < qhi) load_q(qraw, q0);
  }

  // ---- key liveness of the row, the tiles to run and the per-key mask term (wave 0):
  // 0 for a kept key, mask_value for a masked one, -inf past N.
  if (wave == 0) {
    const uint16_t mterm = __builtin_bit_cast(uint16_t, TypeOps<T>::from_f32(a.mask_value));
    const uint16_t ninf = __builtin_bit_cast(uint16_t, TypeOps<T>::from_f32(-INFINITY));
    int n = 0;
    bool full = true;
    for (int t = 0; t < ntiles; ++t) {
      const int key = t * KT + lane;
      const bool valid = key < N;
      bool live = valid;
      if (live && a.mask) live = a.mask[b * a.mask_stride[0] + s * a.mask_stride[1] + (int64_t)key * a.mask_stride[2]] != 0;
      mbt[key] = !valid ? ninf : (live ? (uint16_t)0 : mterm);
      const uint64_t bits = __ballot(live);
      full &= bits == __ballot(valid);
      if (lane == 0) {
        hdr.tile_live[t] = bits;
        if (bits != 0) hdr.tile_list[n] = (uint16_t)t;
      }
      n += bits != 0;
    }
    const bool dead = n == 0;
    if (dead)
      for (int t = lane; t < ntiles; t += 64) hdr.tile_list[t] = (uint16_t)t;
    if (lane == 0) {
      hdr.nrun = dead ? ntiles : n;
      hdr.dead = dead;
      hdr.full = full;
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): this wave's LDS DMA has landed
  __syncthreads();
  const int nrun = hdr.nrun;
  const bool dead = hdr.dead != 0;
  const bool full = hdr.full != 0;

  // identity A-fragments for the bias MFMA (element e of lane group g in step t is key
  // 16t + 8g + e of the 32-key sub-tile; row l32 holds a 1 there iff l32 is that key)
  V8 idf[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) idf[t][e] = TypeOps<T>::from_f32(l32 == 16 * t + 8 * g + e ? 1.f : 0.f);
  const uint32_t one_bits = __builtin_bit_cast(uint16_t, TypeOps<T>::from_f32(1.f));

  // per-lane LDS offsets: K fragment of k-step kk for key row l32 of a 32-key sub-tile
  // (the swizzle term (key / 4) % 4 only depends on l32), and the V^T transposed-read base.
  int koff[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) koff[kk] = l32 * ROW_BYTES + 16 * ((2 * kk + g) ^ ((l32 >> 2) & 3));
  const int tr_r = lane & 15;
  int tr_off = ((tr_r >> 2) * 32 + 16 * ((lane >> 4) & 1) + 4 * (tr_r & 3)) * 2 + 4 * g * ROW_BYTES;

  // exact row maxima are only tracked for callers that ask for them
  constexpr bool want_max = WMAX;
  for (int qblk = q0; qblk < qhi; qblk += NW) {
    // The first tiles' LDS reads are the same for every query block; keeping the compiler
    // from hoisting them out of this loop keeps their registers free for the key loop.
    asm volatile("" : "+v"(koff[0]), "+v"(koff[1]), "+v"(tr_off));
    const int myq = qblk * 32 + l32;
    const bool qok = myq < N;
    V8 qf[2];
    if (GNN_ROW_QPREFETCH) {
      // later blocks: requested during the previous block's sweep (no-bias kernel, which has
      // the registers to spare) or here
      if (!QPF_SWEEP && qblk != q0) load_q(qraw, qblk);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int d0 = 16 * t + 8 * g;
        f32x8 x = TypeOps<T>::to_f32(qraw[t]);
        qf[t] = (qok && d0 < D) ? TypeOps<T>::from_f32(x * a.scale) : zero8<T>();
      }
    } else {
      const T* qp = (const T*)a.q + b * a.q_stride[0] + s * a.q_stride[1] + h * a.q_stride[3] +
                    (int64_t)(qok ? myq : 0) * a.q_stride[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int d0 = 16 * t + 8 * g;
        if (qok && d0 < D) {
          f32x8 x = TypeOps<T>::to_f32(load8(qp + d0));
          qf[t] = TypeOps<T>::from_f32(x * a.scale);
        } else {
          qf[t] = zero8<T>();
        }
      }
    }
    // this block's bias tiles (fragment order, see bias_tiles_kernel) and this lane's chunk
    const T* btile = HAS_BIAS ? (const T*)a.workspace + (((int64_t)b * H + h) * nqb + qblk) * ntiles * BIAS_TILE_ELEMS + lane * 8
                              : nullptr;
    f32x16 o;
    float m, lsum, mx;
    BiasFragR<T> bb;
    // the next block's q, requested after this block's first bias tile (so that waiting for
    // that tile does not wait for it) and in flight during the sweep
    bool qnext_sent = false;
    auto prefetch_q = [&]() {
      if (GNN_ROW_QPREFETCH && QPF_SWEEP && !qnext_sent && qblk + NW < qhi) load_q(qraw, qblk + NW);
      qnext_sent = true;
    };

    // S^T (+ bias, + key mask term on partial tiles) of tile t into acc: acc[sub][i] is key
    // t*64 + sub*32 + 8*(i/4) + 4g + i%4.
    // K fragments of tile t (k-step kk of 32-key half sub)
    auto load_k = [&](V8 (&kf)[2][2], int t) {
      const unsigned char* kt = ks + t * TILE_BYTES;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) kf[kk][sub] = load8((const T*)(kt + sub * 32 * ROW_BYTES + koff[kk]));
    };
    V8 kf[2][2];
    auto qk = [&](f32x16 (&acc)[2], int t, bool partial) {
#if !GNN_ROW_KPREFETCH
      load_k(kf, t);
#endif
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[sub][i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) Mma<T, PREC_NATIVE>::step(acc[sub], kf[kk][sub], qf[kk]);
      if constexpr (HAS_BIAS) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int sub = 0; sub < 2; ++sub) Mma<T, PREC_NATIVE>::step(acc[sub], idf[t2], bb.f[sub][t2]);
      }
      if (partial) {
        // A[key][0] = the key's mask term (lane group 0), B[0][q] = 1: adds the term to every
        // query of the key row; all other products are 0 * 0 (or 0 * 1).
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          const uint32_t term = mbt[t * KT + sub * 32 + l32];
          const u32x4 av = {g ? 0u : term, 0u, 0u, 0u};
          const u32x4 bv = {one_bits, 0u, 0u, 0u};
          Mma<T, PREC_NATIVE>::step(acc[sub], __builtin_bit_cast(V8, av), __builtin_bit_cast(V8, bv));
        }
      }
    };

    // online softmax and O^T += V^T P^T for the scores of tile t. `first`: the row's first
    // tile sets the reference maximum; `per_tile`: every tile's maximum is taken and the
    // accumulators rescaled when it grows past the threshold; otherwise, with `want_max`, each
    // tile's maximum only updates the exact row maximum (the reference maximum stays).
    auto softmax_pv = [&](f32x16 (&sc)[2], int t, bool first, bool per_tile) {
      if (first || per_tile || want_max) {
        mfma_result_fence(sc[0], sc[1]);
        float m0 = max3_nn(sc[0][0], sc[0][1], sc[0][2]), m1 = max3_nn(sc[1][0], sc[1][1], sc[1][2]);
#pragma unroll
        for (int i = 3; i < 15; i += 2) {
          m0 = max3_nn(m0, sc[0][i], sc[0][i + 1]);
          m1 = max3_nn(m1, sc[1][i], sc[1][i + 1]);
        }
        const float mh = max3_nn(m0, max_nn(sc[0][15], sc[1][15]), m1);
        const float mt = pair_max_swap(mh);
        if (first) {
          m = mt;  // o and the row sum are still zero
          mx = mt;
        } else {
          mx = max_nn(mx, mt);
          if (per_tile && __any(mt > m + RESCALE_THRESHOLD)) {
            const float mnew = fmaxf(m, mt);
            const float alpha = fast_exp2((m - mnew) * LOG2E);
            m = mnew;
            lsum *= alpha;
#pragma unroll
            for (int i = 0; i < 16; ++i) o[i] *= alpha;
          }
        }
      }
      const float nm = -m * LOG2E;
      // per 32-key half: exponentiate, round to the MFMA type, accumulate the row sum and
      // O^T += V^T P^T. Fragment element e of k-step kk of half sub is key
      // sub*32 + 16kk + 8(e/4) + 4g + e%4 in both operands.
      const unsigned char* vt = vs + t * TILE_BYTES;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        V8 vf[2];
        auto load_v = [&](int kk) {
          const unsigned char* vb = vt + (sub * 32 + 16 * kk) * ROW_BYTES + tr_off;
          const V4 lo = tr_read4_r<T>(vb);
          const V4 hi = tr_read4_r<T>(vb + 8 * ROW_BYTES);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vf[kk][e] = lo[e];
            vf[kk][e + 4] = hi[e];
          }
        };
        if (GNN_ROW_VPREFETCH) {
          load_v(0);
          load_v(1);
        }
        if (!dead) {
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[sub][i] = fast_exp2(__builtin_fmaf(sc[sub][i], LOG2E, nm));
        } else {  // m is the collapsed sentinel: subtract first so s - m is exact
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[sub][i] = fast_exp2((sc[sub][i] - m) * LOG2E);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          f32x8 x = {sc[sub][8 * kk + 0], sc[sub][8 * kk + 1], sc[sub][8 * kk + 2], sc[sub][8 * kk + 3],
                     sc[sub][8 * kk + 4], sc[sub][8 * kk + 5], sc[sub][8 * kk + 6], sc[sub][8 * kk + 7]};
          const V8 pf = TypeOps<T>::from_f32(x);
          lsum = rowsum_add_r(x, lsum);
          if (!GNN_ROW_VPREFETCH) load_v(kk);
          Mma<T, PREC_NATIVE>::step(o, vf[kk], pf);
        }
      }
    };

#if GNN_ROW_SETPRIO
#define ROW_PRIO_HI() __builtin_amdgcn_s_setprio(1)
#define ROW_PRIO_LO() __builtin_amdgcn_s_setprio(0)
#else
#define ROW_PRIO_HI()
#define ROW_PRIO_LO()
#endif
    // every tile of the row, with the reference maximum from the first tile, or (per_tile)
    // with each tile's maximum and lazy rescale
    auto sweep = [&](bool per_tile) {
#pragma unroll
      for (int i = 0; i < 16; ++i) o[i] = 0.f;
      lsum = 0.f;
      m = -INFINITY;
      mx = -INFINITY;
      if (full) {
        // no masked key: tiles in order; only the last one can hold keys past N
        const bool tail = N % KT != 0;
        if constexpr (HAS_BIAS) load_bias_tile<T>(bb, btile);
        prefetch_q();
        if (GNN_ROW_KPREFETCH) load_k(kf, 0);
        for (int t = 0; t < ntiles; ++t) {
          f32x16 sc[2];
          ROW_PRIO_HI();
          qk(sc, t, tail && t == ntiles - 1);
          ROW_PRIO_LO();
          if (GNN_ROW_KPREFETCH && t + 1 < ntiles) load_k(kf, t + 1);  // in flight during the softmax
          if (HAS_BIAS && t + 1 < ntiles) load_bias_tile<T>(bb, btile + (t + 1) * BIAS_TILE_ELEMS);
          softmax_pv(sc, t, t == 0, per_tile);
        }
      } else {
        if constexpr (HAS_BIAS) load_bias_tile<T>(bb, btile + hdr.tile_list[0] * BIAS_TILE_ELEMS);
        prefetch_q();
        if (GNN_ROW_KPREFETCH) load_k(kf, hdr.tile_list[0]);
        for (int it = 0; it < nrun; ++it) {
          const int t = hdr.tile_list[it];
          f32x16 sc[2];
          ROW_PRIO_HI();
          qk(sc, t, hdr.tile_live[t] != ~0ull);
          ROW_PRIO_LO();
          if (GNN_ROW_KPREFETCH && it + 1 < nrun) load_k(kf, hdr.tile_list[it + 1]);
          if (HAS_BIAS && it + 1 < nrun) load_bias_tile<T>(bb, btile + hdr.tile_list[it + 1] * BIAS_TILE_ELEMS);
          softmax_pv(sc, t, it == 0, per_tile);
        }
      }
    };
    // A block whose row sum exceeds FastLimit anywhere (p or the accumulators may have
    // overflowed) runs again with per-tile maxima.
    sweep(false);
    if (__any(!(lsum <= FastLimit<T>::value))) sweep(true);

    // ---- normalise and store. o[i] is O[myq][8*(i/4) + 4g + i%4].
    const float ltot = pair_sum_swap(lsum);
    if (qok) {
      const float inv = 1.0f / ltot;
      T* orow = (T*)a.o + b * a.o_stride[0] + s * a.o_stride[1] + h * a.o_stride[3] + (int64_t)myq * a.o_stride[2];
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int d0 = 8 * rg + 4 * g;
        if (d0 < D) {
          f32x4 x = {o[4 * rg] * inv, o[4 * rg + 1] * inv, o[4 * rg + 2] * inv, o[4 * rg + 3] * inv};
          store4(orow + d0, TypeOps<T>::from_f32(x));
        }
      }
      const int64_t ridx = (((int64_t)b * a.S + s) * H + h) * N + myq;
      if (a.lse && g == 0) a.lse[ridx] = m + __log2f(ltot) * (1.0f / LOG2E);
      if (want_max && g == 0) a.row_max[ridx] = mx;
    }
  }
}

template <typename T, bool HAS_BIAS, int NW, bool WMAX>
int launch_row_nw(const gnn_triattn_args& a, hipStream_t stream, size_t smem) {
  const void* fn = (const void*)triattn_row_kernel<T, HAS_BIAS, NW, WMAX>;
  if (smem > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  const int64_t nblk = a.B * a.S * a.H;
  // split rows (first halves first, second halves last): as many as one workgroup per CU,
  // when two workgroups share a CU and a row has at least two query blocks per wave
  int64_t nsplit = 0;
  if (GNN_ROW_STAGGER && NW == 8 && (a.N + 31) / 32 >= 2 * NW) {
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      nsplit = std::min<int64_t>(ncu, nblk);
  }
  hipLaunchKernelGGL((triattn_row_kernel<T, HAS_BIAS, NW, WMAX>), dim3((uint32_t)(nblk + nsplit)), dim3(NW * 64),
                     smem, stream, a);
  return (int)hipGetLastError();
}

template <typename T, bool HAS_BIAS>
int launch_row(const gnn_triattn_args& a, hipStream_t stream) {
  if (HAS_BIAS) {
    const int64_t nchunks = bias_tile_count(a.B, a.H, a.N) * 256;
    hipLaunchKernelGGL((bias_tiles_kernel<T>), dim3((uint32_t)((nchunks + 255) / 256)), dim3(256), 0, stream, a,
                       (T*)a.workspace, nchunks);
  }
  const size_t smem = row_smem_bytes(a.N);
  // one workgroup per CU: 16 waves (12 with GNN_ROW_W12 where that spreads the row's 32-query
  // blocks evenly)
  const int64_t nqb = (a.N + 31) / 32;
  const bool w12 = GNN_ROW_W12 && nqb % 12 == 0 && nqb % 16 != 0;
  if (a.row_max) {
    if (smem > ROW_TWO_PER_CU_BYTES)
      return w12 ? launch_row_nw<T, HAS_BIAS, 12, true>(a, stream, smem)
                 : launch_row_nw<T, HAS_BIAS, 16, true>(a, stream, smem);
    return launch_row_nw<T, HAS_BIAS, 8, true>(a, stream, smem);
  }
  if (smem > ROW_TWO_PER_CU_BYTES)
    return w12 ? launch_row_nw<T, HAS_BIAS, 12, false>(a, stream, smem)
               : launch_row_nw<T, HAS_BIAS, 16, false>(a, stream, smem);
  return launch_row_nw<T, HAS_BIAS, 8, false>(a, stream, smem);
}

}  // namespace

size_t triattn_row_workspace_bytes(const gnn_triattn_args& a) {
  return a.bias ? (size_t)bias_tile_count(a.B, a.H, a.N) * BIAS_TILE_ELEMS * 2 : 0;
}

bool triattn_row_applicable(const gnn_triattn_args& a) {
  return (a.dtype == GNN_BF16 || a.dtype == GNN_F16) && a.D <= 32 && a.N <= GNN_ROW_MAX_N && a.N >= 1 &&
         a.B * a.S * a.H < ((int64_t)1 << 31);
}

int triattn_row_fwd(const gnn_triattn_args& a, hipStream_t stream) {
  if (a.dtype == GNN_BF16) return a.bias ? launch_row<bf16, true>(a, stream) : launch_row<bf16, false>(a, stream);
  return a.bias ? launch_row<f16, true>(a, stream) : launch_row<f16, false>(a, stream);
}

// ---- allocation-free forward: the bias tiles go to a static device array of the library.
// Each device that loads the library holds its own copy of `scratch` until the process ends.
// In host code the array's name is not a device address: the address is taken once per
// device with hipGetSymbolAddress (with that device current) and only that pointer is passed
// to kernels. Calls on one device share the array, so calls that overlap on one device race;
// the pre-pass rewrites every byte a call reads, so no state needs clearing between calls.
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[MAX_DEVICES];
}  // namespace

int triattn_fwd_noalloc(const gnn_triattn_args& a, hipStream_t stream) {
  const size_t need = triattn_row_applicable(a) ? triattn_row_workspace_bytes(a) : 0;
  if (need > NOALLOC_SCRATCH_BYTES)
    return set_error(GNN_ERR_UNSUPPORTED,
                     "triangle_attention (no-alloc): the pair bias in fragment order needs more than the 16 MiB "
                     "static scratch (B * H * ceil(N/32) * ceil(N/64) * 4 KB); use gnn_triattn_fwd with a workspace");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return set_error(GNN_ERR_ARG, "triangle_attention (no-alloc): no current HIP device");
  void* ptr;
  {
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
      void* p = nullptr;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return set_error(GNN_ERR_ARG, "triangle_attention (no-alloc): hipGetSymbolAddress(scratch) failed");
      scratch_ptr[dev] = p;
    }
    ptr = scratch_ptr[dev];
  }
  gnn_triattn_args b = a;
  b.workspace = ptr;
  b.workspace_bytes = NOALLOC_SCRATCH_BYTES;
  return triattn_fwd(b, stream);
}

}  // namespace gnn
