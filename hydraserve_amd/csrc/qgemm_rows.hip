// Decode-regime (M <= 32) quantized weight GEMM for gfx950: row-partitioned.
//
// Replaces the Triton launches of hydraserve/kernels/awq.py:52-74
// (_awq_gemm_kernel, awq.py:82-142) and hydraserve/kernels/fp8.py:68-96
// (_fp8_gemm_kernel, fp8.py:104-168) for activations of at most 16 rows
// (MS = 1 strip) and, on wide outputs, 17..32 rows (MS = 2 strips of 16
// rows sharing every unpacked weight fragment).
//
// Work split.  Workgroup p owns the contiguous weight rows
// [p*N/P, (p+1)*N/P) -- at most 16*NBLK rows, NBLK blocks of 16 -- and its KW
// wavefronts split K into KW contiguous ranges of 128-wide chunks (one INT4
// group / one FP8 block each).  Every wavefront therefore streams its own
// disjoint slab of the weight matrix, no two workgroups ever touch the same
// output, and the only reduction is across the workgroup's wavefronts, in
// LDS, once at the end.  There is no grid-level synchronisation and no
// partial-result traffic.
//
// Per wavefront, per chunk c of its range:
//   * weights: lane (l16, h) holds 16 bytes (INT4) / 32 bytes (FP8) of row
//     16b + l16 of every block b -- one buffer load per block;
//   * A fragments: the same lane holds X[min(16s + l16, M-1)][c*128 + 32h, +32)
//     for each strip s,
//     either from a copy of X staged into LDS once (XL: when X fits) or read
//     from global memory (an L2 hit after first use) two groups ahead;
//   * weights stream through a register ring RD chunks deep: the slot of a
//     block is refilled with the same block RD chunks later right after it is
//     unpacked, so RD chunks of loads stay in flight and no loaded register
//     is ever copied;
//   * INT4: nibble q -> bf16 128+q (int4_operand), T = MFMA(X, 128+q), the
//     group sum Xg = MFMA(X, 1) once per chunk for all blocks, and
//     acc += s * (T - (128+z) * Xg);  FP8: exact E4M3FN -> bf16 and
//     acc += s * MFMA(X, W).
// Scales and zero points of the workgroup's rows (and X, for XL) are staged
// into LDS once, every thread keeping eight wide loads in flight.
#include <type_traits>

#include "qgemm_ops.h"

namespace hsq {

template <int WT, int SDT, int NBLK, int KW, int RD, bool XL, int MS>
struct RowsK {
  static constexpr int THREADS = 64 * KW;
  static constexpr int SES = SDT == SCALE_F32 ? 4 : 2;
  static constexpr int CB = WT == W_INT4 ? 64 : 128;  // bytes of a weight row per chunk
  static constexpr int LPB = WT == W_INT4 ? 1 : 2;    // 16-byte loads per block per chunk

  struct WSlot {
    u32x4_t q[NBLK][LPB];
  };
  struct ASlot {
    u32x4_t a[MS][4];
  };

  // LDS: [front] the reduction area ([KW][NBLK][64 lanes] f32x4), which for
  // XL also holds X first (M rows of 2K+32 bytes; the padding spreads the
  // rows over the banks); then zero points (INT4: rows r0>>3 .. (r1-1)>>3,
  // GC words each); then scales (INT4: one row per weight row; FP8: one row
  // per 128-row block), GC entries each.
  static __host__ __device__ int red_bytes() { return KW * NBLK * MS * 64 * 16; }
  static __host__ __device__ int x_stride(int K) { return 2 * K + 32; }
  static __host__ __device__ size_t front_bytes(int M, int K) {
    const size_t x = XL ? static_cast<size_t>(M) * x_stride(K) : 0;
    const size_t r = red_bytes();
    return (x > r ? x : r + 0) / 16 * 16 + 16;
  }
  static __host__ __device__ int zrows_max() { return WT == W_INT4 ? NBLK * 2 + 2 : 0; }
  static __host__ __device__ int srows_max() { return WT == W_INT4 ? 16 * NBLK : 3; }
  static __host__ __device__ size_t lds_bytes(int M, int K) {
    const int GC = K / 128;
    const size_t z = static_cast<size_t>(zrows_max()) * GC * 4;
    const size_t s = (static_cast<size_t>(srows_max()) * GC * SES + 3) / 4 * 4;
    return front_bytes(M, K) + z + s;
  }

  static __device__ __forceinline__ float scale_from_lds(const uint8_t* p) {
    if constexpr (SDT == SCALE_F32) {
      return *reinterpret_cast<const float*>(p);
    } else {
      const uint32_t h16 = *reinterpret_cast<const uint16_t*>(p);
      if constexpr (SDT == SCALE_BF16) return __uint_as_float(h16 << 16);
      return __half2float(__ushort_as_half(static_cast<unsigned short>(h16)));
    }
  }
};

// a.P = workgroups (row partitions); a.T = chunks per row (K / 128).
template <int WT, int SDT, int NBLK, int KW, int RD, bool XL, int MS>
__global__ __launch_bounds__(64 * KW) void qgemm_rows_kernel(GemmArgs a) {
  using D = RowsK<WT, SDT, NBLK, KW, RD, XL, MS>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int GC = a.T;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(tid >> 6));
  const int lane = tid & 63, l16 = lane & 15, h = lane >> 4;
  const int p = blockIdx.x;
  int r0, r1;
  row_partition(a, p, &r0, &r1);
  if (r0 >= r1) return;
  const int nr = r1 - r0;

  float* red = reinterpret_cast<float*>(smem);
  uint8_t* xl = smem;
  const int xst = D::x_stride(a.K);
  const size_t front = D::front_bytes(a.M, a.K);
  uint32_t* zl = reinterpret_cast<uint32_t*>(smem + front);
  uint8_t* sl = smem + front + static_cast<size_t>(D::zrows_max()) * GC * 4;
  const int z0 = r0 >> 3, zn = ((r1 - 1) >> 3) - z0 + 1;
  const int b0 = r0 >> 7, bn = ((r1 - 1) >> 7) - b0 + 1;

  // ---- per-lane constants ------------------------------------------------------
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(
      a.w, static_cast<int64_t>(a.N - 1) * (WT == W_INT4 ? a.ldw * 4 : a.ldw) + (WT == W_INT4 ? a.K / 2 : a.K));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (static_cast<int64_t>(a.M - 1) * a.ldx + a.K) * 2);
  const int rb = static_cast<int>(WT == W_INT4 ? a.ldw * 4 : a.ldw);  // bytes per weight row
  uint32_t woff[NBLK];
  uint32_t soff[NBLK];  // LDS byte offset of the lane's scale row (chunk 0)
  uint32_t zoff[NBLK];  // LDS word offset of the lane's zero-point row (chunk 0)
  uint32_t zsh[NBLK];
#pragma unroll
  for (int b = 0; b < NBLK; ++b) {
    int rl = 16 * b + l16;  // row within the partition, clamped to it
    rl = rl < nr ? rl : nr - 1;
    const int row = r0 + rl;
    woff[b] = static_cast<uint32_t>(row * rb) + (WT == W_INT4 ? 16u : 32u) * h;
    if constexpr (WT == W_INT4) {
      soff[b] = static_cast<uint32_t>(rl * GC * D::SES);
      zoff[b] = static_cast<uint32_t>(((row >> 3) - z0) * GC);
      zsh[b] = 4u * static_cast<uint32_t>(row & 7);
    } else {
      soff[b] = static_cast<uint32_t>(((row >> 7) - b0) * GC * D::SES);
      zoff[b] = 0;
      zsh[b] = 0;
    }
  }
  // Activation row of the lane in strip s (rows past M repeat row M-1).
  uint32_t xoff[MS], xloff[MS];
#pragma unroll
  for (int s = 0; s < MS; ++s) {
    const int xm = 16 * s + l16 < a.M ? 16 * s + l16 : a.M - 1;
    xoff[s] = static_cast<uint32_t>(xm * static_cast<int>(a.ldx) * 2) + 64u * h;
    xloff[s] = static_cast<uint32_t>(xm * xst) + 64u * h;
  }

  const uint32_t nib_mask = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t magic = opaque_and(0x43004300u, 0xFFFFFFFFu);
  const uint32_t one2 = opaque_and(0x3F803F80u, 0xFFFFFFFFu);
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{one2, one2, one2, one2});

  // ---- the wavefront's K range -------------------------------------------------
  const int cs = wave * GC / KW, ce = (wave + 1) * GC / KW;
  const int n = ce - cs;  // >= 1: the host requires K / 128 >= KW

  // Chunk i of the wavefront's range, clamped to its last chunk.
  auto chunk_of = [&](int i) __attribute__((always_inline)) { return cs + (i < n ? i : n - 1); };
  auto load_w = [&](u32x4_t (&q)[D::LPB], int b, int i) __attribute__((always_inline)) {
    const uint32_t so = static_cast<uint32_t>(chunk_of(i) * D::CB);
#pragma unroll
    for (int e = 0; e < D::LPB; ++e) q[e] = bload<u32x4_t>(rw, woff[b] + 16u * e, so);
  };
  auto load_a = [&](typename D::ASlot& as, int i) __attribute__((always_inline)) {
    const uint32_t xs = static_cast<uint32_t>(chunk_of(i) * 256);
#pragma unroll
    for (int s = 0; s < MS; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) as.a[s][j] = bload<u32x4_t>(rx, xoff[s] + 16u * j, xs);
  };

  // Weights: a ring of RD chunks (slot r = chunk % RD), refilled block by
  // block right after each block is unpacked.  Without XL, A fragments come
  // in two groups of RD chunks; group g+1 is requested at the start of group
  // g, ahead of every weight load it pairs with, because the memory counter
  // completes loads in issue order (waiting for an A fragment issued after
  // its weights would wait for all of them at once).
  typename D::WSlot wring[RD];
  typename D::ASlot abuf[XL ? 1 : 2][RD];
  if constexpr (!XL) {
#pragma unroll
    for (int r = 0; r < RD; ++r) load_a(abuf[0][r], r);
  }
#pragma unroll
  for (int r = 0; r < RD; ++r)
#pragma unroll
    for (int b = 0; b < NBLK; ++b) load_w(wring[r].q[b], b, r);

  // ---- stage scales / zero points (and X) while the first weights land ---------
  if constexpr (WT == W_INT4) {
    stage_copy_any<D::THREADS>(sl, reinterpret_cast<const uint8_t*>(a.scale) + static_cast<int64_t>(r0) * a.lds * D::SES,
                               nr, GC * D::SES, a.lds * D::SES, tid);
    stage_copy_any<D::THREADS>(reinterpret_cast<uint8_t*>(zl),
                               reinterpret_cast<const uint8_t*>(a.zero) + static_cast<int64_t>(z0) * a.ldz * 4, zn,
                               GC * 4, a.ldz * 4, tid);
  } else {
    stage_copy_any<D::THREADS>(sl, reinterpret_cast<const uint8_t*>(a.scale) + static_cast<int64_t>(b0) * a.lds * D::SES,
                               bn, GC * D::SES, a.lds * D::SES, tid);
  }
  if constexpr (XL) {
    // X rows, 16 bytes per access (INT4: permuted to int4_operand's order).
    const int upr = a.K / 8;
    const int total = a.M * upr;
    for (int base = tid; base < total; base += 8 * D::THREADS) {
      u32x4_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int i = base + j * D::THREADS;
        i = i < total ? i : total - 1;
        const int m = i / upr, u = i - m * upr;
        v[j] = bload<u32x4_t>(rx, static_cast<uint32_t>(m * static_cast<int>(a.ldx) * 2 + u * 16), 0u);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = base + j * D::THREADS;
        if (i < total) {
          const int m = i / upr, u = i - m * upr;
          u32x4_t w = v[j];
          if constexpr (WT == W_INT4) w = permute_x(w);
          *reinterpret_cast<u32x4_t*>(xl + m * xst + u * 16) = w;
        }
      }
    }
  }
  __syncthreads();

  f32x4_t acc[NBLK][MS];
#pragma unroll
  for (int b = 0; b < NBLK; ++b)
#pragma unroll
    for (int s = 0; s < MS; ++s) acc[b][s] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One group of RD chunks starting at chunk i0 (A fragments in abuf[G]
  // without XL).
  auto group = [&](auto gsel, int i0) __attribute__((always_inline)) {
    constexpr int G = decltype(gsel)::value;
    if constexpr (!XL) {
#pragma unroll
      for (int r = 0; r < RD; ++r) load_a(abuf[G ^ 1][r], i0 + RD + r);
    }
#pragma unroll
    for (int r = 0; r < RD; ++r) {
      const int i = i0 + r;
      const bool valid = i < n;
      const int c = cs + (valid ? i : n - 1);
      bf16x8_t A[MS][4];
#pragma unroll
      for (int s = 0; s < MS; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (XL) {
            A[s][j] =
                __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(xl + xloff[s] + c * 256 + 16 * j));
          } else if constexpr (WT == W_INT4) {
            A[s][j] = __builtin_bit_cast(bf16x8_t, permute_x(abuf[G][r].a[s][j]));
          } else {
            A[s][j] = __builtin_bit_cast(bf16x8_t, abuf[G][r].a[s][j]);
          }
        }
      f32x4_t xg[MS];
#pragma unroll
      for (int s = 0; s < MS; ++s) {
        xg[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if constexpr (WT == W_INT4) {
#pragma unroll
          for (int j = 0; j < 4; ++j) xg[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[s][j], ones, xg[s], 0, 0, 0);
        }
      }
      // Software pipeline over the blocks.  Region b: unpack block b, refill
      // block b-1's slot (its only reader was the previous region's unpack),
      // multiply block b, fold block b-1's products.  Nothing in a region
      // depends on another of its parts, so the scheduler interleaves them;
      // the barrier between regions keeps every refill after its slot's read.
      f32x4_t tp[MS];
#pragma unroll
      for (int s = 0; s < MS; ++s) tp[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int b = 0; b <= NBLK; ++b) {
        bf16x8_t B[4];
        if (b < NBLK) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if constexpr (WT == W_INT4) {
              B[j] = int4_operand(wring[r].q[b][0][j], nib_mask, magic);
            } else {
              B[j] = fp8_operand(wring[r].q[b][j >> 1][(j & 1) * 2], wring[r].q[b][j >> 1][(j & 1) * 2 + 1]);
            }
          }
        }
        if (b > 0) load_w(wring[r].q[b - 1], b - 1, i + RD);
        f32x4_t t[MS];
#pragma unroll
        for (int s = 0; s < MS; ++s) {
          t[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          if (b < NBLK) {
#pragma unroll
            for (int j = 0; j < 4; ++j) t[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[s][j], B[j], t[s], 0, 0, 0);
          }
        }
        if (b > 0) {
          const int bb = b - 1;
          const float sc = valid ? D::scale_from_lds(sl + soff[bb] + c * D::SES) : 0.f;
          if constexpr (WT == W_INT4) {
            const float negc = -(128.0f + static_cast<float>((zl[zoff[bb] + c] >> zsh[bb]) & 0xFu));
#pragma unroll
            for (int s = 0; s < MS; ++s)
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[bb][s][e] = fmaf(sc, fmaf(negc, xg[s][e], tp[s][e]), acc[bb][s][e]);
          } else {
#pragma unroll
            for (int s = 0; s < MS; ++s)
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[bb][s][e] = fmaf(sc, tp[s][e], acc[bb][s][e]);
          }
        }
#pragma unroll
        for (int s = 0; s < MS; ++s) tp[s] = t[s];
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  if constexpr (XL) {
    for (int i0 = 0; i0 < n; i0 += RD) group(std::integral_constant<int, 0>{}, i0);
  } else {
    for (int i0 = 0; i0 < n; i0 += 2 * RD) {
      group(std::integral_constant<int, 0>{}, i0);
      if (i0 + RD >= n) break;
      group(std::integral_constant<int, 1>{}, i0 + RD);
    }
  }

  // ---- reduce the KW partial sums of every output, in wavefront order ---------
  if constexpr (XL) __syncthreads();  // the reduction area overlays X
  // Entry (w, b, s) of the reduction area: wavefront w's sums of block b,
  // strip s.  Work item i = b * MS + s is reduced by wavefront i % KW.
#pragma unroll
  for (int b = 0; b < NBLK; ++b)
#pragma unroll
    for (int s = 0; s < MS; ++s)
      *reinterpret_cast<f32x4_t*>(red + (((wave * NBLK + b) * MS + s) * 64 + lane) * 4) = acc[b][s];
  __syncthreads();
  if (a.silu_mul) {
    // Fused SiLU-and-mul: local blocks 2q (gate rows) and 2q+1 (the matching
    // up rows) of the interleaved weight; r0 and nr are multiples of 32.  As
    // in the reference's unfused sequence (hydraserve/model/runtime.py:
    // 1202-1210, silu_and_mul at hydraserve/kernels/activation.py:66-76),
    // gate and up are rounded to bf16 first, then out = gate * sigmoid(gate)
    // * up in fp32, rounded to bf16, into y [M, N/2].
    for (int i = wave; i < (NBLK / 2) * MS; i += KW) {
      const int q = i / MS, s = i - q * MS;
      if (32 * q >= nr) continue;
      const int ig = (2 * q) * MS + s, iu = (2 * q + 1) * MS + s;
      f32x4_t g = *reinterpret_cast<const f32x4_t*>(red + (ig * 64 + lane) * 4);
      f32x4_t u = *reinterpret_cast<const f32x4_t*>(red + (iu * 64 + lane) * 4);
#pragma unroll
      for (int w = 1; w < KW; ++w) {
        const f32x4_t vg = *reinterpret_cast<const f32x4_t*>(red + ((w * NBLK * MS + ig) * 64 + lane) * 4);
        const f32x4_t vu = *reinterpret_cast<const f32x4_t*>(red + ((w * NBLK * MS + iu) * 64 + lane) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g[e] += vg[e];
          u[e] += vu[e];
        }
      }
      const int col = r0 / 2 + 16 * q + l16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * s + 4 * h + e;
        if (m < a.M) {
          const float gb = bf16_to_f32(to_bf16_bits(g[e]));
          const float ub = bf16_to_f32(to_bf16_bits(u[e]));
          const float sig = 1.0f / (1.0f + expf(-gb));
          a.y[m * a.ldy + col] = to_bf16_bits(gb * sig * ub);
        }
      }
    }
    return;
  }
  for (int i = wave; i < NBLK * MS; i += KW) {
    const int b = i / MS, s = i - b * MS;
    f32x4_t sum = *reinterpret_cast<const f32x4_t*>(red + (i * 64 + lane) * 4);
#pragma unroll
    for (int w = 1; w < KW; ++w) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(red + ((w * NBLK * MS + i) * 64 + lane) * 4);
      sum[0] += v[0];
      sum[1] += v[1];
      sum[2] += v[2];
      sum[3] += v[3];
    }
    const int rl = 16 * b + l16;
    if (rl < nr) {
      const int col = r0 + rl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * s + 4 * h + e;
        if (m < a.M) a.y[m * a.ldy + col] = to_bf16_bits(sum[e]);
      }
    }
  }
}

template <int WT, int SDT, int NBLK, int KW, int RD, bool XL, int MS>
static hipError_t launch_rows_t(const GemmArgs& a, hipStream_t stream) {
  using D = RowsK<WT, SDT, NBLK, KW, RD, XL, MS>;
  const size_t lds = D::lds_bytes(a.M, a.K);
  hipLaunchKernelGGL((qgemm_rows_kernel<WT, SDT, NBLK, KW, RD, XL, MS>), dim3(a.P), dim3(D::THREADS), lds, stream, a);
  return hipGetLastError();
}

// K split and ring depth for NBLK row blocks: 8-16 KB of weight loads in
// flight per wavefront within the register budget (FP8 chunks are twice the
// bytes of INT4 chunks; staging X in LDS frees the A-fragment registers).
// Two 16-row strips (17..32 activation rows) run only with 3+ row blocks,
// without XL, at the one-chunk ring.
struct RowsCfg {
  int nblk, kw, rd;
};

int rows_kw8 = 0;  // tuning: 1 selects 8 wavefronts (2 per SIMD) for INT4 with 5+ row blocks

static RowsCfg rows_cfg(int wt, int nblk, bool xl, int ms) {
  if (ms > 1) return {nblk, 4, 1};
  if (wt == W_INT4) {
    if (nblk <= 2) return {nblk, 8, 4};
    if (nblk <= 4) return {nblk, 4, xl ? 4 : 2};
    if (rows_kw8) return {nblk, 8, 1};
    return {nblk, 4, xl ? 2 : 1};
  }
  if (nblk <= 2) return {nblk, 8, xl ? 4 : 2};
  if (nblk <= 4) return {nblk, 4, xl ? 2 : 1};
  return {nblk, 4, 1};
}

#define HSQ_RW(NB_, KW_, RD_) \
  if (c.nblk == NB_ && c.kw == KW_ && c.rd == RD_) return launch_rows_t<WT, SDT, NB_, KW_, RD_, XL, 1>(a, stream);
#define HSQ_RW2(NB_) \
  if (c.nblk == NB_) return launch_rows_t<WT, SDT, NB_, 4, 1, false, 2>(a, stream);

template <int WT, int SDT, bool XL>
static hipError_t launch_rows_x(const GemmArgs& a, int nblk, int ms, hipStream_t stream) {
  const RowsCfg c = rows_cfg(WT, nblk, XL, ms);
  if (ms == 2) {
    if constexpr (!XL) {
      HSQ_RW2(3) HSQ_RW2(4) HSQ_RW2(5) HSQ_RW2(6) HSQ_RW2(7) HSQ_RW2(8) HSQ_RW2(9)
    }
    return hipErrorInvalidValue;
  }
  if (ms != 1) return hipErrorInvalidValue;
  if constexpr (WT == W_INT4 && XL) {
    HSQ_RW(1, 8, 4) HSQ_RW(2, 8, 4) HSQ_RW(3, 4, 4) HSQ_RW(4, 4, 4) HSQ_RW(5, 4, 2) HSQ_RW(6, 4, 2)
    HSQ_RW(7, 4, 2) HSQ_RW(8, 4, 2) HSQ_RW(9, 4, 2) HSQ_RW(10, 4, 2)
    HSQ_RW(5, 8, 1) HSQ_RW(6, 8, 1) HSQ_RW(7, 8, 1) HSQ_RW(8, 8, 1) HSQ_RW(9, 8, 1)
  } else if constexpr (WT == W_INT4) {
    HSQ_RW(1, 8, 4) HSQ_RW(2, 8, 4) HSQ_RW(3, 4, 2) HSQ_RW(4, 4, 2) HSQ_RW(5, 4, 1) HSQ_RW(6, 4, 1)
    HSQ_RW(7, 4, 1) HSQ_RW(8, 4, 1) HSQ_RW(9, 4, 1) HSQ_RW(10, 4, 1)
    HSQ_RW(5, 8, 1) HSQ_RW(6, 8, 1) HSQ_RW(7, 8, 1) HSQ_RW(8, 8, 1) HSQ_RW(9, 8, 1)
  } else if constexpr (XL) {
    HSQ_RW(1, 8, 4) HSQ_RW(2, 8, 4) HSQ_RW(3, 4, 2) HSQ_RW(4, 4, 2) HSQ_RW(5, 4, 1) HSQ_RW(6, 4, 1)
    HSQ_RW(7, 4, 1) HSQ_RW(8, 4, 1) HSQ_RW(9, 4, 1)
  } else {
    HSQ_RW(1, 8, 2) HSQ_RW(2, 8, 2) HSQ_RW(3, 4, 1) HSQ_RW(4, 4, 1) HSQ_RW(5, 4, 1) HSQ_RW(6, 4, 1)
    HSQ_RW(7, 4, 1) HSQ_RW(8, 4, 1) HSQ_RW(9, 4, 1)
  }
  return hipErrorInvalidValue;
}
#undef HSQ_RW
#undef HSQ_RW2

constexpr int kRowsMaxBlocks = 9;
constexpr int kRowsMaxBlocksSilu = 10;  // INT4 only: whole gate/up pairs per workgroup
constexpr size_t kRowsMaxLds = 160 * 1024;

size_t rows_lds_bytes(int wt, int sdt, int nblk, bool xl, int M, int K, int ms) {
  const RowsCfg c = rows_cfg(wt, nblk, xl, ms);
  const int GC = K / 128;
  const size_t red = static_cast<size_t>(c.kw) * c.nblk * ms * 64 * 16;
  const size_t x = xl ? static_cast<size_t>(M) * (2 * K + 32) : 0;
  const size_t front = (x > red ? x : red) / 16 * 16 + 16;
  const int ses = sdt == SCALE_F32 ? 4 : 2;
  const size_t z = wt == W_INT4 ? static_cast<size_t>(c.nblk * 2 + 2) * GC * 4 : 0;
  const size_t s = (static_cast<size_t>(wt == W_INT4 ? 16 * c.nblk : 3) * GC * ses + 3) / 4 * 4;
  return front + z + s;
}

// Can the row-partitioned kernel run this problem with P workgroups?  Sets
// the row-block count, whether X is staged in LDS, and the number of 16-row
// activation strips (1 up to 16 rows; 2 up to 32 rows with 3+ row blocks).
bool rows_ok(const GemmArgs& a, int wt, int P, int* nblk_out, bool* xl_out, int* ms_out, int xl_pref) {
  if (a.M < 1 || a.M > 32 || !a.xvec || !a.wvec || a.K % 128 != 0 || P < 1) return false;
  if (a.K / 128 < 8) return false;  // every wavefront of the K split (<= 8) gets at least one chunk
  const int ms = a.M > 16 ? 2 : 1;
  if (a.silu_mul && (wt != W_INT4 || a.N % 32 != 0 || ms > 1)) return false;
  const int rows = row_partition_max(a, P);
  const int nblk = (rows + 15) / 16;
  if (nblk > (a.silu_mul ? kRowsMaxBlocksSilu : kRowsMaxBlocks) || (ms > 1 && nblk < 3)) return false;
  const int64_t rb = wt == W_INT4 ? a.ldw * 4 : a.ldw;
  if (static_cast<int64_t>(a.N) * rb >= (int64_t{1} << 31)) return false;
  if ((static_cast<int64_t>(a.M) * a.ldx + a.K) * 2 >= (int64_t{1} << 31)) return false;
  bool xl = ms == 1 && xl_pref != 0 && rows_lds_bytes(wt, a.sdt, nblk, true, a.M, a.K, ms) <= kRowsMaxLds;
  if (!xl && rows_lds_bytes(wt, a.sdt, nblk, false, a.M, a.K, ms) > kRowsMaxLds) return false;
  *nblk_out = nblk;
  *xl_out = xl;
  *ms_out = ms;
  return true;
}

hipError_t launch_rows(int wt, const GemmArgs& a, int nblk, bool xl, int ms, hipStream_t stream) {
#define HSQ_RX(WT_, SDT_)                                                    \
  return xl ? launch_rows_x<WT_, SDT_, true>(a, nblk, ms, stream)           \
            : launch_rows_x<WT_, SDT_, false>(a, nblk, ms, stream);
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) HSQ_RX(W_INT4, SCALE_BF16)
    if (a.sdt == SCALE_F16) HSQ_RX(W_INT4, SCALE_F16)
    HSQ_RX(W_INT4, SCALE_F32)
  }
  if (a.sdt == SCALE_BF16) HSQ_RX(W_FP8, SCALE_BF16)
  if (a.sdt == SCALE_F16) HSQ_RX(W_FP8, SCALE_F16)
  HSQ_RX(W_FP8, SCALE_F32)
#undef HSQ_RX
}

}  // namespace hsq
