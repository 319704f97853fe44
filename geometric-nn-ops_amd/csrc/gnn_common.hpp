// Shared device helpers for the gfx950 (CDNA4) triangle kernels.
//
// Every matrix product in this library is issued as 32x32 output tiles on the
// 32x32xK MFMA units. The common currency is a "fragment": for one K=16 step of a
// 32x32 tile, lane l holds 8 consecutive-k elements of row (l % 32) of its operand,
// lane group g = l / 32 holding k = 8g .. 8g+7. A and B fragments use the same
// (lane group, element) -> k assignment, so the product is correct for whichever
// concrete k order the hardware uses inside one instruction, and callers may map
// logical k indices onto (g, element) any way they like as long as A and B agree.
//
// The 32x32 fp32 accumulator (16 VGPRs) holds, in lane l and register r,
//   row = 8 * (r / 4) + 4 * (l / 32) + (r % 4),   col = l % 32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gnn {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

enum Prec { PREC_NATIVE = 0, PREC_IEEE = 1, PREC_BF16X3 = 2 };

// ---- element-type traits ------------------------------------------------------------
template <typename T> struct TypeOps;

template <> struct TypeOps<bf16> {
  typedef bf16x8 V8;
  typedef bf16x4 V4;
  static __device__ __forceinline__ V8 from_f32(const f32x8& x) {
    return __builtin_convertvector(x, bf16x8);
  }
  static __device__ __forceinline__ V4 from_f32(const f32x4& x) {
    return __builtin_convertvector(x, bf16x4);
  }
  static __device__ __forceinline__ f32x8 to_f32(const V8& x) {
    return __builtin_convertvector(x, f32x8);
  }
  static __device__ __forceinline__ f32x4 to_f32(const V4& x) {
    return __builtin_convertvector(x, f32x4);
  }
  static __device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
  static __device__ __forceinline__ bf16 from_f32(float x) { return (bf16)x; }
};

template <> struct TypeOps<f16> {
  typedef f16x8 V8;
  typedef f16x4 V4;
  static __device__ __forceinline__ V8 from_f32(const f32x8& x) {
    return __builtin_convertvector(x, f16x8);
  }
  static __device__ __forceinline__ V4 from_f32(const f32x4& x) {
    return __builtin_convertvector(x, f16x4);
  }
  static __device__ __forceinline__ f32x8 to_f32(const V8& x) {
    return __builtin_convertvector(x, f32x8);
  }
  static __device__ __forceinline__ f32x4 to_f32(const V4& x) {
    return __builtin_convertvector(x, f32x4);
  }
  static __device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
  static __device__ __forceinline__ f16 from_f32(float x) { return (f16)x; }
};

template <> struct TypeOps<float> {
  typedef f32x8 V8;
  typedef f32x4 V4;
  static __device__ __forceinline__ V8 from_f32(const f32x8& x) { return x; }
  static __device__ __forceinline__ V4 from_f32(const f32x4& x) { return x; }
  static __device__ __forceinline__ f32x8 to_f32(const V8& x) { return x; }
  static __device__ __forceinline__ f32x4 to_f32(const V4& x) { return x; }
  static __device__ __forceinline__ float to_f32(float x) { return x; }
  static __device__ __forceinline__ float from_f32(float x) { return x; }
};

// ---- vector memory access ---------------------------------------------------------------
// 8 consecutive elements (16 B for 16-bit types, 32 B for fp32). Pointer must be aligned
// to the vector size (the host checks base pointers and strides).
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 load8(const T* p) {
  return *reinterpret_cast<const typename TypeOps<T>::V8*>(p);
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const typename TypeOps<T>::V8& v) {
  *reinterpret_cast<typename TypeOps<T>::V8*>(p) = v;
}
// load8 through a global-address-space pointer: a global_load counts only in vmcnt, where a
// flat_load (what the compiler emits when it cannot prove a pointer global) counts in lgkmcnt
// too, so that every later wait for an LDS read would also wait for it.
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 load8_global(const T* p) {
  typedef typename TypeOps<T>::V8 V8;
  return *(const __attribute__((address_space(1))) V8*)(p);
}
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V4 load4(const T* p) {
  return *reinterpret_cast<const typename TypeOps<T>::V4*>(p);
}
template <typename T>
__device__ __forceinline__ void store4(T* p, const typename TypeOps<T>::V4& v) {
  *reinterpret_cast<typename TypeOps<T>::V4*>(p) = v;
}
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 zero8() {
  return TypeOps<T>::from_f32(f32x8{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f});
}

// 8 bias values from key `key` on, with the ones at keys >= N replaced by zero: the
// identity-fragment MFMA that adds the bias multiplies every loaded value (0 * x for the
// other keys), so padding past N must not hold a NaN or an infinity.
template <typename T>
__device__ __forceinline__ typename TypeOps<T>::V8 load8_bias_tail(const T* row, int key, int N) {
  if (key >= N) return zero8<T>();
  typename TypeOps<T>::V8 x = load8(row + key);
  if (key + 8 > N) {
    const T zero = TypeOps<T>::from_f32(0.f);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (key + e >= N) x[e] = zero;
  }
  return x;
}

// ---- raw buffer stores (gfx9 family) ------------------------------------------------------
// A buffer store whose byte offset lies at or past its resource's range is dropped by the
// hardware. A kernel can then issue its stores unconditionally (no store inside a branch)
// and still skip lanes: such lanes carry BUFFER_OOB (the range stays below 2^31 bytes). This
// matters for the compiler's memory-counter waits (vmcnt counts loads and stores in issue
// order): at the join after a branch holding a store it takes the count of the path without
// the store, so a later wait for a load issued before that store also waits for the store.
constexpr uint32_t BUFFER_RSRC_WORD3 = 0x00020000;  // raw, unswizzled buffer
constexpr uint32_t BUFFER_OOB = 0x80000000u;
// base and range_bytes must be the same for every lane of the wave. They pass through
// readfirstlane: where the compiler keeps them in vector registers (tile coordinates it
// cannot prove uniform) it would otherwise wrap every store in a loop over the lanes'
// distinct descriptors (readfirstlane, compare, exec mask, branch back).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int range_bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  void* u = (void*)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, __builtin_amdgcn_readfirstlane(range_bytes),
                                           BUFFER_RSRC_WORD3);
}
template <typename V>
__device__ __forceinline__ void buffer_store(const V& v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  static_assert(sizeof(V) == 4 || sizeof(V) == 8 || sizeof(V) == 16, "buffer_store: 4, 8 or 16 bytes");
  if constexpr (sizeof(V) == 16)
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, off, 0, 0);
  else if constexpr (sizeof(V) == 8)
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, off, 0, 0);
  else
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}

// ---- 32x32 tile, one K=16 step ----------------------------------------------------------
// acc[row, col] += sum_k A[row, k] * B[k, col] over the 16 k of this step, with both
// operands given as fragments (see the file comment).
template <typename T, int PREC> struct Mma;

template <> struct Mma<bf16, PREC_NATIVE> {
  static __device__ __forceinline__ void step(f32x16& acc, const bf16x8& a, const bf16x8& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
  }
};

template <> struct Mma<f16, PREC_NATIVE> {
  static __device__ __forceinline__ void step(f32x16& acc, const f16x8& a, const f16x8& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  }
};

// Full fp32: eight K=2 fp32 MFMAs; instruction e consumes element e of both fragments.
template <> struct Mma<float, PREC_IEEE> {
  static __device__ __forceinline__ void step(f32x16& acc, const f32x8& a, const f32x8& b) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], acc, 0, 0, 0);
  }
};

// bf16x3 emulation of an fp32 product: x = hi + lo with hi = bf16(x), lo = bf16(x - hi);
// a*b ~= hi_a*hi_b + hi_a*lo_b + lo_a*hi_b (the lo*lo term is dropped), accumulated in fp32.
// hi widens back to fp32 from its packed pairs (element 2i in the low half of dword i: a
// shift, element 2i + 1 in the high half: a mask), one instruction per element; converting
// each element of x again for it costs two.
__device__ __forceinline__ void split_bf16(const f32x8& x, bf16x8& hi, bf16x8& lo) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  hi = __builtin_convertvector(x, bf16x8);
  const u32x4_t hp = __builtin_bit_cast(u32x4_t, hi);
  f32x8 back;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    back[2 * i] = __uint_as_float(hp[i] << 16);
    back[2 * i + 1] = __uint_as_float(hp[i] & 0xffff0000u);
  }
  lo = __builtin_convertvector(x - back, bf16x8);
}

template <> struct Mma<float, PREC_BF16X3> {
  static __device__ __forceinline__ void step(f32x16& acc, const f32x8& a, const f32x8& b) {
    bf16x8 ah, al, bh, bl;
    split_bf16(a, ah, al);
    split_bf16(b, bh, bl);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc, 0, 0, 0);
  }
};

// ---- misc -------------------------------------------------------------------------------
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Reductions over the lane pair (l, l ^ 32).
__device__ __forceinline__ float pair_max(float x) { return fmaxf(x, __shfl_xor(x, 32)); }
__device__ __forceinline__ float pair_sum(float x) { return x + __shfl_xor(x, 32); }

__device__ __forceinline__ float sigmoidf_fast(float x) {
  return 1.0f / (1.0f + fast_exp2(-x * 1.4426950408889634f));
}

// MI355X dispatches consecutive workgroup ids round-robin over its 8 XCDs, each with a
// private L2. Remap so that the workgroups resident on one XCD take a contiguous range
// of the logical work order (a bijection for any grid size).
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t nblk) {
  constexpr uint32_t NXCD = 8;
  const uint32_t xcd = bid % NXCD;
  const uint32_t idx = bid / NXCD;
  const uint32_t per = (nblk + NXCD - 1) / NXCD;  // blocks on the fuller XCDs
  uint32_t tall = nblk % NXCD;
  if (tall == 0) tall = NXCD;
  if (xcd < tall) return xcd * per + idx;
  return tall * per + (xcd - tall) * (per - 1) + idx;
}

}  // namespace gnn
