// Register-level building blocks shared by the decode kernels (gfx950).
#pragma once

#include "qgemm_common.h"

namespace hsq {

// No inline asm anywhere near the MFMAs: the compiler's MFMA hazard handling
// does not see through it (an empty asm on accumulators produced stale
// results on gfx950).  (x & mask) | magic with mask/magic in VGPRs compiles
// to a single v_and_or_b32.
__device__ __forceinline__ uint32_t insert_nibbles(uint32_t mask, uint32_t src, uint32_t magic) {
  return (src & mask) | magic;
}

// Eight nibbles of one word -> eight bf16 128+q in the order
// [q0, q4, q1, q5, q2, q6, q3, q7]: a shift and one v_and_or_b32 per output
// dword, with mask 0x000F000F and magic 0x43004300 (bf16 128.0 in both
// halves; 128+q is exact).  The A operand must use the same order
// (permute_x).
__device__ __forceinline__ bf16x8_t int4_operand(uint32_t w, uint32_t nib_mask, uint32_t magic) {
  u32x4_t p;
  p[0] = insert_nibbles(nib_mask, w, magic);
  p[1] = insert_nibbles(nib_mask, w >> 4, magic);
  p[2] = insert_nibbles(nib_mask, w >> 8, magic);
  p[3] = insert_nibbles(nib_mask, w >> 12, magic);
  return __builtin_bit_cast(bf16x8_t, p);
}

// int4_operand of two words at once: each right shift is one 64-bit shift
// of the pair (w1:w0).  The bits of w1 that the shift moves into the low
// word land at bit 20 or above, outside the nibble mask of every position
// they reach.
__device__ __forceinline__ void int4_operand2(uint32_t w0, uint32_t w1, uint32_t nib_mask, uint32_t magic,
                                              bf16x8_t& b0, bf16x8_t& b1) {
  const uint64_t v = (static_cast<uint64_t>(w1) << 32) | w0;
  u32x4_t p0, p1;
  p0[0] = insert_nibbles(nib_mask, w0, magic);
  p1[0] = insert_nibbles(nib_mask, w1, magic);
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    const uint64_t t = v >> (4 * i);
    p0[i] = insert_nibbles(nib_mask, static_cast<uint32_t>(t), magic);
    p1[i] = insert_nibbles(nib_mask, static_cast<uint32_t>(t >> 32), magic);
  }
  b0 = __builtin_bit_cast(bf16x8_t, p0);
  b1 = __builtin_bit_cast(bf16x8_t, p1);
}

// bf16 (x0..x7) -> (x0, x4, x1, x5, x2, x6, x3, x7), matching int4_operand.
__device__ __forceinline__ u32x4_t permute_x(u32x4_t d) {
  u32x4_t e;
  e[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
  e[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
  e[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
  e[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
  return e;
}

// Eight E4M3FN bytes -> eight bf16, exactly (every E4M3FN value is a bf16
// value), in memory order.
__device__ __forceinline__ bf16x8_t fp8_operand(uint32_t d0, uint32_t d1) {
  u32x4_t p;
  p[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
  p[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
  p[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
  p[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
  return __builtin_bit_cast(bf16x8_t, p);
}

// B bytes moved as one vector access (B = 4, 8, 16, 32): a native vector
// type, so copies stay in registers.
template <int B>
struct VecT;
template <>
struct VecT<2> {
  typedef uint16_t type;
};
template <>
struct VecT<4> {
  typedef uint32_t type __attribute__((ext_vector_type(1)));
};
template <>
struct VecT<8> {
  typedef uint32_t type __attribute__((ext_vector_type(2)));
};
template <>
struct VecT<16> {
  typedef uint32_t type __attribute__((ext_vector_type(4)));
};
template <>
struct VecT<32> {
  typedef uint32_t type __attribute__((ext_vector_type(8)));
};
template <int B>
using Blob = typename VecT<B>::type;

// Raw buffer access: a resource descriptor in SGPRs covering `bytes` bytes
// from p (the host refuses calls with an operand of 2^31 bytes or more:
// extents_ok in qgemm_capi.hip), a per-lane 32-bit
// offset and a uniform 32-bit offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

// soff is uniform by construction; readfirstlane states it, so the compiler
// never wraps the load in a per-lane loop.  AUX is the cache-policy operand
// (kNonTemporal: data read once, streamed past the caches it would evict).
constexpr int kNonTemporal = 2;

template <typename V, int AUX = 0>
__device__ __forceinline__ V bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff_in) {
  const uint32_t soff = __builtin_amdgcn_readfirstlane(soff_in);
  if constexpr (sizeof(V) == 16) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
  } else if constexpr (sizeof(V) == 8) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, AUX));
  } else if constexpr (sizeof(V) == 4) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, AUX));
  } else {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, AUX));
  }
}

// Copy nrows rows of row_bytes bytes (source row stride src_stride bytes)
// into dense LDS rows, V bytes per access, eight loads in flight per thread.
template <int V, int THREADS>
__device__ __forceinline__ void stage_copy(uint8_t* dst, const uint8_t* src, int nrows, int row_bytes,
                                           int64_t src_stride, int tid) {
  using T = Blob<V>;
  const int upr = row_bytes / V;
  const int total = nrows * upr;
  for (int base = tid; base < total; base += 8 * THREADS) {
    T v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int i = base + j * THREADS;
      i = i < total ? i : total - 1;
      const int r = i / upr, u = i - r * upr;
      v[j] = *reinterpret_cast<const T*>(src + r * src_stride + static_cast<int64_t>(u) * V);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = base + j * THREADS;
      if (i < total) *reinterpret_cast<T*>(dst + static_cast<int64_t>(i) * V) = v[j];
    }
  }
}

template <int THREADS>
__device__ __forceinline__ void stage_copy_any(uint8_t* dst, const uint8_t* src, int nrows, int row_bytes,
                                               int64_t src_stride, int tid) {
  const uint64_t al = reinterpret_cast<uintptr_t>(src) | static_cast<uint64_t>(row_bytes) |
                      static_cast<uint64_t>(src_stride);
  if ((al & 15) == 0) return stage_copy<16, THREADS>(dst, src, nrows, row_bytes, src_stride, tid);
  if ((al & 7) == 0) return stage_copy<8, THREADS>(dst, src, nrows, row_bytes, src_stride, tid);
  if ((al & 3) == 0) return stage_copy<4, THREADS>(dst, src, nrows, row_bytes, src_stride, tid);
  stage_copy<2, THREADS>(dst, src, nrows, row_bytes, src_stride, tid);
}

}  // namespace hsq
