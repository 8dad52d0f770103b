// Shared device helpers for the quantized weight-only GEMMs (gfx950 / CDNA4).
//
// Both weight formats compute Y[M,N] = X[M,K] . W[N,K]^T with bf16 X and Y and
// fp32 accumulation, like hydraserve/kernels/awq.py:82-142 and
// hydraserve/kernels/fp8.py:104-168, but the work decomposition is our own:
//
//   * a "unit" is (output tile, K chunk); units are numbered tile-major, so a
//     contiguous range of units walks K inside one tile before moving on;
//   * a persistent grid of P workgroups takes equal contiguous unit ranges
//     (stream-K).  A workgroup whose range covers a whole tile stores bf16
//     directly.  Tiles cut by a range boundary are finished by the last
//     contributor to arrive: every contributor writes an fp32 partial into its
//     own slot, bumps the tile's counter, and the last one sums the slots in
//     workgroup order (deterministic) and stores bf16.  The last one also
//     resets the counter, so the workspace stays zeroed between calls.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace hsq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

enum WeightKind { W_INT4 = 0, W_FP8 = 1 };
enum ScaleDtype { SCALE_BF16 = 0, SCALE_F16 = 1, SCALE_F32 = 2 };

struct GemmArgs {
  const uint16_t* x;  // bf16 activations [M, K], row stride ldx (elements)
  int64_t ldx;
  const void* w;      // INT4: int32 words [N, ceil(K/8)]; FP8: bytes [N, K]
  int64_t ldw;        // row stride in words (INT4) or bytes (FP8)
  const void* scale;  // INT4: [N, G128]; FP8: [ceil(N/128), ceil(K/128)]
  int64_t lds;        // row stride of scale (elements)
  int sdt;            // ScaleDtype
  const int32_t* zero;  // INT4 zero points [ceil(N/8), G128], row stride ldz
  int64_t ldz;
  uint16_t* y;        // bf16 output [M, N], row stride ldy
  int64_t ldy;
  int M, N, K;
  int G;              // stream-K steps per tile (decode: batches of NB chunks)
  int NB;             // decode: K chunks per stream-K step
  int T;              // output tiles
  int TM;             // tiles along M (prefill only; decode uses 1)
  int64_t U;          // stream-K steps = T * G
  int P;              // persistent workgroups (P <= U)
  int* counters;      // [T] arrival counters, zero between calls
  float* partials;    // [P][2][slot] fp32 partial tiles
  int xvec;           // X base and row stride allow 16-byte loads
  int wvec;           // W base and row stride allow 16-byte loads
  int tune;           // kernel-specific experiment bits (0 = defaults)
  int silu_mul;       // 1: W rows interleave gate and up in 16-row blocks and
                      // y [M, N/2] receives silu(gate) * up
  const void* wtiles;  // optional load-time copy of W in 16-row tiles (read by
                       // the tiled decode kernel only; layout in qgemm_tiled.hip)
  int tpw;            // tiled decode kernel: 16-row tiles per workgroup
  int splits;         // tiled decode kernel: K ranges per tile group
  int cps;            // tiled decode kernel: 128-wide K chunks per K range
};

// Row partitions of the row-partitioned decode kernels: rows [*r0, *r1) of
// workgroup p of a.P.  An even split of the N rows, or with the fused
// SiLU-and-mul epilogue (a.silu_mul, N a multiple of 32) an even split of the
// N/32 gate/up block pairs, so both blocks of a pair land in one workgroup.
__host__ __device__ inline void row_partition(const GemmArgs& a, int p, int* r0, int* r1) {
  if (a.silu_mul) {
    const int64_t np = a.N / 32;
    *r0 = 32 * static_cast<int>(p * np / a.P);
    *r1 = 32 * static_cast<int>((p + 1) * np / a.P);
  } else {
    *r0 = static_cast<int>(static_cast<int64_t>(p) * a.N / a.P);
    *r1 = static_cast<int>(static_cast<int64_t>(p + 1) * a.N / a.P);
  }
}

// The largest partition row_partition gives with P workgroups.
__host__ __device__ inline int row_partition_max(const GemmArgs& a, int P) {
  return a.silu_mul ? 32 * static_cast<int>((a.N / 32 + P - 1) / P) : (a.N + P - 1) / P;
}

template <int SDT>
__device__ __forceinline__ float load_scale(const void* p, int64_t idx) {
  // idx is in elements of the scale dtype
  if constexpr (SDT == SCALE_F32) {
    return reinterpret_cast<const float*>(p)[idx];
  } else {
    const uint32_t h = reinterpret_cast<const uint16_t*>(p)[idx];
    if constexpr (SDT == SCALE_BF16) return __uint_as_float(h << 16);
    return __half2float(__ushort_as_half(static_cast<unsigned short>(h)));
  }
}

__device__ __forceinline__ float load_scale_rt(const void* p, int64_t idx, int dt) {
  if (dt == SCALE_F32) return load_scale<SCALE_F32>(p, idx);
  if (dt == SCALE_BF16) return load_scale<SCALE_BF16>(p, idx);
  return load_scale<SCALE_F16>(p, idx);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Two floats -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// x & m, hidden from the optimizer so that byte extraction of the result
// stays v_cvt_f32_ubyte{0..3} (one op per nibble) instead of being folded into
// v_bfe_u32 + convert (two ops per nibble).
__device__ __forceinline__ uint32_t opaque_and(uint32_t x, uint32_t m) {
  uint32_t r;
  asm volatile("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(m));
  return r;
}

// ---- stream-K bookkeeping -------------------------------------------------
__device__ __forceinline__ int64_t unit_begin(int p, int64_t U, int P) {
  return (static_cast<int64_t>(p) * U) / P;
}

// Workgroup whose unit range holds unit u.
__device__ __forceinline__ int unit_owner(int64_t u, int64_t U, int P) {
  int p = static_cast<int>((u * P) / U);
  if (p > P - 1) p = P - 1;
  while (p + 1 < P && unit_begin(p + 1, U, P) <= u) ++p;
  while (p > 0 && unit_begin(p, U, P) > u) --p;
  return p;
}

// Slot of workgroup p's partial for tile t: 0 if t is p's first tile, else 1.
__device__ __forceinline__ int partial_slot(int p, int t, int G, int64_t U, int P) {
  return (unit_begin(p, U, P) / G == t) ? 0 : 1;
}

// Partial tiles cross workgroups that may run on different XCDs, whose L2s are
// not coherent with each other.  Instead of agent-scope release/acquire
// fences (which write back and invalidate the whole L2), partials are written
// and read with the cache policy of agent-scope atomics (sc1: write-through on
// stores, coherent on loads; see store_partial4 / load_partial4 below), and
// the arrival counter is an agent-scope atomic.

// Count this workgroup's arrival at tile t once every thread's partial stores
// are acknowledged; true in every thread of the workgroup that arrived last.
__device__ __forceinline__ bool arrive_last(int* counters, int t, int contributors, int* lds_flag) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): every partial store acknowledged
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(&counters[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = (old == contributors - 1);
  }
  __syncthreads();
  return *lds_flag != 0;
}

// Partial tiles as 16-byte buffer accesses carrying the cache policy the
// compiler gives agent-scope atomic loads and stores (sc1): as coherent
// across XCDs as 4-byte atomics, but not ordered one after another, so a
// settle keeps all of its loads in flight at once (atomic loads are issued
// one round trip at a time, ~1 us each).
constexpr int kAgentCoherent = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(float* partials) {
  return __builtin_amdgcn_make_buffer_rsrc(partials, static_cast<short>(0), 0x7FFFFFFF, 0x00020000);
}

__device__ __forceinline__ void store_partial4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, byte_off, 0, kAgentCoherent);
}

__device__ __forceinline__ f32x4_t load_partial4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kAgentCoherent));
}

__device__ __forceinline__ void reset_counter(int* counters, int t) {
  if (threadIdx.x == 0) __hip_atomic_store(&counters[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// (tile, chunk) position of a unit, advanced without divisions.
struct Cursor {
  int t, c;
  __device__ __forceinline__ void advance(int G) {
    if (++c == G) {
      c = 0;
      ++t;
    }
  }
};

}  // namespace hsq
