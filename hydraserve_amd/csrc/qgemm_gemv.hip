// Decode-regime quantized weight GEMM for gfx950: row-partitioned,
// block-major ("GEMV") variant for activations that fit in LDS.
//
// Replaces the Triton launches of hydraserve/kernels/awq.py:52-74
// (_awq_gemm_kernel, awq.py:82-142) and hydraserve/kernels/fp8.py:68-96
// (_fp8_gemm_kernel, fp8.py:104-168) for activations of at most 16 rows whose
// copy fits in LDS next to the workgroup's scales.
//
// Work split.  Workgroup p owns the weight rows [p*N/P, (p+1)*N/P), cut into
// blocks of 16 rows; its KW wavefronts split K into KW contiguous ranges of
// 128-wide chunks.  A wavefront walks its slab block-major: all chunks of its
// K range for block 0, then block 1, ...  Its weight loads therefore stream
// each row of a block contiguously (chunk after chunk, RD chunks in flight),
// which is the order HBM serves best, and the ring of RD chunks costs only
// RD registers-worth of one block, leaving room for several wavefronts per
// SIMD.  There is no inter-workgroup communication: the KW partial sums of
// each block meet in LDS at the end.
//
// Per step (one block x one chunk), lane (l16, h):
//   * weights: 16 bytes (INT4) / 32 bytes (FP8) of row 16b + l16 at byte
//     16h / 32h of the chunk, one buffer load per 16 bytes;
//   * A: X[min(l16, M-1)][c*128 + 32h, +32) from the LDS copy of X (INT4: in
//     int4_operand's order), and Xg (the fp32 sum of the chunk's 128 X values
//     for rows 4h..4h+3) from a table filled while X is staged;
//   * INT4: T = MFMA(X, 128+q), acc += s * (T - (128+z) * Xg);
//     FP8: acc += s * MFMA(X, W), W exact from E4M3FN.
#include "qgemm_ops.h"

namespace hsq {

template <int WT, int SDT, int KW, int RD>
struct GemvK {
  static constexpr int THREADS = 64 * KW;
  static constexpr int SES = SDT == SCALE_F32 ? 4 : 2;
  static constexpr int CB = WT == W_INT4 ? 64 : 128;  // bytes of a weight row per chunk
  static constexpr int LPB = WT == W_INT4 ? 1 : 2;    // 16-byte loads per step

  struct Slot {
    u32x4_t q[LPB];
  };

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

// LDS layout, in order (every part 16-byte aligned):
//   X    [M][2K+32 bytes]     (the padding spreads rows over the banks)
//   red  [KW][nblk][64][4]    f32 partial sums of every block
//   xg   [GC][XGR]            f32 group sums, XGR = M rounded up to 4
//   zero [zn][GC]             u32 zero-point words (INT4)
//   scl  [srows][GC]          scales (INT4: per weight row; FP8: per 128-row block)
struct GemvLds {
  size_t x, red, xg, zero, scl, total;
};

__host__ __device__ inline size_t align16(size_t v) { return (v + 15) / 16 * 16; }

__host__ __device__ inline GemvLds gemv_lds(int wt, int sdt, int kw, int M, int K, int nr_max) {
  const int GC = K / 128;
  const int nblk = (nr_max + 15) / 16;
  const int ses = sdt == SCALE_F32 ? 4 : 2;
  GemvLds l;
  l.x = 0;
  l.red = align16(static_cast<size_t>(M) * (2 * K + 32));
  l.xg = l.red + static_cast<size_t>(kw) * nblk * 64 * 16;
  l.zero = l.xg + align16(static_cast<size_t>(GC) * ((M + 3) / 4 * 4) * 4);
  const int zn = wt == W_INT4 ? nr_max / 8 + 2 : 0;
  l.scl = l.zero + align16(static_cast<size_t>(zn) * GC * 4);
  const int srows = wt == W_INT4 ? nr_max : nr_max / 128 + 2;
  l.total = l.scl + align16(static_cast<size_t>(srows) * GC * ses);
  return l;
}

// a.P = workgroups (row partitions); a.T = chunks per row (K / 128); a.G =
// the largest partition (rows), which sized the LDS layout.
template <int WT, int SDT, int KW, int RD>
__global__ __launch_bounds__(64 * KW) void qgemm_gemv_kernel(GemmArgs a) {
  using D = GemvK<WT, SDT, KW, RD>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int GC = a.T;
  const int M = a.M;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(tid >> 6));
  const int lane = tid & 63, l16 = lane & 15, h = lane >> 4;
  const int p = blockIdx.x;
  int r0, r1;
  row_partition(a, p, &r0, &r1);
  if (r0 >= r1) return;
  const int nr = r1 - r0;
  const int nblk = (nr + 15) / 16;

  const GemvLds L = gemv_lds(WT, SDT, KW, M, a.K, a.G);
  const int xst = 2 * a.K + 32;
  const int xgr = (M + 3) / 4 * 4;
  uint8_t* xl = smem + L.x;
  float* red = reinterpret_cast<float*>(smem + L.red);
  float* xgl = reinterpret_cast<float*>(smem + L.xg);
  uint32_t* zl = reinterpret_cast<uint32_t*>(smem + L.zero);
  uint8_t* sl = smem + L.scl;
  const int z0 = r0 >> 3, zn = ((r1 - 1) >> 3) - z0 + 1;
  const int b0 = r0 >> 7, bn = ((r1 - 1) >> 7) - b0 + 1;

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(
      a.w, static_cast<int64_t>(a.N - 1) * (WT == W_INT4 ? a.ldw * 4 : a.ldw) + (WT == W_INT4 ? a.K / 2 : a.K));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (static_cast<int64_t>(M - 1) * a.ldx + a.K) * 2);
  const int rb = static_cast<int>(WT == W_INT4 ? a.ldw * 4 : a.ldw);  // bytes per weight row

  // ---- the wavefront's K range and its (block, chunk) steps -------------------
  const int cs = wave * GC / KW, ce = (wave + 1) * GC / KW;
  const int n = ce - cs;  // >= 1: the host requires K / 128 >= KW
  const int total = nblk * n;

  // Load cursor (runs RD steps ahead, stops at the last step).
  int lb = 0, li = 0, lstep = 0;
  auto row_off = [&](int b) __attribute__((always_inline)) {
    int row = r0 + 16 * b + l16;
    row = row < r1 ? row : r1 - 1;
    return static_cast<uint32_t>(row * rb) + (WT == W_INT4 ? 16u : 32u) * h;
  };
  const int cstride = D::CB;
  uint32_t lwoff = row_off(0);
  auto load_step = [&](typename D::Slot& s) __attribute__((always_inline)) {
    const uint32_t so = static_cast<uint32_t>((cs + li) * cstride);
#pragma unroll
    for (int e = 0; e < D::LPB; ++e) s.q[e] = bload<u32x4_t>(rw, lwoff + 16u * e, so);
    if (lstep < total - 1) {
      ++lstep;
      if (++li == n) {
        li = 0;
        ++lb;
        lwoff = row_off(lb);
      }
    }
  };

  // ---- staging: X (16-byte units; INT4 permuted to int4_operand's order, with
  // the fp32 group sums computed on the way), scales and zero points (dword
  // units, or 16-bit when a scale row is not dword-aligned).  Every pass
  // issues all of its loads before storing; pass 0 is issued before the
  // first weight loads so waiting for it never waits for those.
  const int xupr = a.K / 8;                 // 16-byte X units per row (multiple of 16)
  const int xunits = M * xupr;
  const int64_t srow_bytes = static_cast<int64_t>(GC) * D::SES;
  const int srows = WT == W_INT4 ? nr : bn;
  const uint8_t* sbase = reinterpret_cast<const uint8_t*>(a.scale) +
                         static_cast<int64_t>(WT == W_INT4 ? r0 : b0) * a.lds * D::SES;
  const bool sdw = ((reinterpret_cast<uintptr_t>(sbase) | static_cast<uintptr_t>(srow_bytes) |
                     static_cast<uintptr_t>(a.lds * D::SES)) & 3) == 0;
  const int sv = sdw ? 4 : 2;                          // bytes per scale unit
  const int supr = static_cast<int>(srow_bytes / sv);  // scale units per row
  const int sunits = srows * supr;
  const int zunits = WT == W_INT4 ? zn * GC : 0;       // dword units
  constexpr int QX = 8, QS = 8;
  auto stage_round = [&](int round, auto issue_weights) __attribute__((always_inline)) {
    u32x4_t xv[QX];
    uint32_t svv[QS];
#pragma unroll
    for (int q = 0; q < QX; ++q) {
      int i = (round * QX + q) * D::THREADS + tid;
      i = i < xunits ? i : xunits - 1;
      const int m = i / xupr, u = i - m * xupr;
      xv[q] = bload<u32x4_t>(rx, static_cast<uint32_t>(m * static_cast<int>(a.ldx) * 2 + u * 16), 0u);
    }
#pragma unroll
    for (int q = 0; q < QS; ++q) {
      int i = (round * QS + q) * D::THREADS + tid;
      const int su = sunits + zunits;
      i = i < su ? i : su - 1;
      if (i < sunits) {
        const int r = i / supr, u = i - r * supr;
        const uint8_t* src = sbase + static_cast<int64_t>(r) * a.lds * D::SES + static_cast<int64_t>(u) * sv;
        svv[q] = sdw ? *reinterpret_cast<const uint32_t*>(src) : *reinterpret_cast<const uint16_t*>(src);
      } else {
        const int zi = i - sunits;
        const int r = zi / GC, c = zi - r * GC;
        svv[q] = static_cast<uint32_t>(a.zero[static_cast<int64_t>(z0 + r) * a.ldz + c]);
      }
    }
    issue_weights();
#pragma unroll
    for (int q = 0; q < QX; ++q) {
      const int i = (round * QX + q) * D::THREADS + tid;
      const int ic = i < xunits ? i : xunits - 1;
      const int m = ic / xupr, u = ic - m * xupr;
      u32x4_t w = xv[q];
      if constexpr (WT == W_INT4) {
        // Units u = 16c .. 16c+15 of a row sit in 16 consecutive lanes.
        float v = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v += __uint_as_float(w[e] << 16);
          v += __uint_as_float(w[e] & 0xFFFF0000u);
        }
        v += __shfl_xor(v, 8, 16);
        v += __shfl_xor(v, 4, 16);
        v += __shfl_xor(v, 2, 16);
        v += __shfl_xor(v, 1, 16);
        if (i < xunits && (u & 15) == 0) xgl[(u >> 4) * xgr + m] = v;
        w = permute_x(w);
      }
      if (i < xunits) *reinterpret_cast<u32x4_t*>(xl + m * xst + u * 16) = w;
    }
#pragma unroll
    for (int q = 0; q < QS; ++q) {
      const int i = (round * QS + q) * D::THREADS + tid;
      if (i < sunits) {
        if (sdw) {
          *reinterpret_cast<uint32_t*>(sl + static_cast<size_t>(i) * 4) = svv[q];
        } else {
          *reinterpret_cast<uint16_t*>(sl + static_cast<size_t>(i) * 2) = static_cast<uint16_t>(svv[q]);
        }
      } else if (i < sunits + zunits) {
        zl[i - sunits] = svv[q];
      }
    }
  };
  typename D::Slot ring[RD];
  const int xrounds = (xunits + QX * D::THREADS - 1) / (QX * D::THREADS);
  const int srounds = (sunits + zunits + QS * D::THREADS - 1) / (QS * D::THREADS);
  const int rounds = xrounds > srounds ? xrounds : srounds;
  stage_round(0, [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < RD; ++r) load_step(ring[r]);
  });
  for (int round = 1; round < rounds; ++round) stage_round(round, []() {});
  __syncthreads();

  const int xm = l16 < M ? l16 : M - 1;
  const uint32_t xloff = static_cast<uint32_t>(xm * xst) + 64u * h;
  const int xgh = 4 * h < xgr - 4 ? 4 * h : xgr - 4;  // rows past M read real (unused) sums
  const uint32_t nib_mask = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t magic = opaque_and(0x43004300u, 0xFFFFFFFFu);

  // Compute cursor: block cb, chunk ci; the lane's scale / zero-point offsets
  // for block cb.
  int cb = 0, ci = 0;
  uint32_t soff = 0, zoff = 0, zsh = 0;
  auto set_block = [&](int b) __attribute__((always_inline)) {
    int rl = 16 * b + l16;
    rl = rl < nr ? rl : nr - 1;
    const int row = r0 + rl;
    if constexpr (WT == W_INT4) {
      soff = static_cast<uint32_t>(rl * GC * D::SES);
      zoff = static_cast<uint32_t>(((row >> 3) - z0) * GC);
      zsh = 4u * static_cast<uint32_t>(row & 7);
    } else {
      soff = static_cast<uint32_t>(((row >> 7) - b0) * GC * D::SES);
    }
  };
  set_block(0);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};

  for (int s0 = 0; s0 < total; s0 += RD) {
#pragma unroll
    for (int r = 0; r < RD; ++r) {
      if (s0 + r < total) {
        const int c = cs + ci;
        bf16x8_t A[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          A[j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(xl + xloff + c * 256 + 16 * j));
        bf16x8_t B[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (WT == W_INT4) {
            B[j] = int4_operand(ring[r].q[0][j], nib_mask, magic);
          } else {
            B[j] = fp8_operand(ring[r].q[j >> 1][(j & 1) * 2], ring[r].q[j >> 1][(j & 1) * 2 + 1]);
          }
        }
        // The slot's last use is the unpack above: refill it RD steps ahead
        // (same registers, nothing copied).
        __builtin_amdgcn_sched_barrier(0);
        load_step(ring[r]);
        f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j], B[j], t, 0, 0, 0);
        const float sc = D::scale_from_lds(sl + soff + c * D::SES);
        if constexpr (WT == W_INT4) {
          const f32x4_t xg = *reinterpret_cast<const f32x4_t*>(xgl + c * xgr + xgh);
          const float negc = -(128.0f + static_cast<float>((zl[zoff + c] >> zsh) & 0xFu));
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] = fmaf(sc, fmaf(negc, xg[e], t[e]), acc[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] = fmaf(sc, t[e], acc[e]);
        }
        if (++ci == n) {
          *reinterpret_cast<f32x4_t*>(red + ((wave * nblk + cb) * 64 + lane) * 4) = acc;
          acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
          ci = 0;
          ++cb;
          set_block(cb < nblk ? cb : nblk - 1);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- sum the KW partials of every block in wavefront order, store bf16 ------
  __syncthreads();
  if (a.silu_mul) {
    // Fused SiLU-and-mul: local blocks 2q (gate rows) and 2q+1 (the matching
    // up rows) of the interleaved weight; r0 and nr are multiples of 32.  As
    // in the reference's unfused sequence (hydraserve/model/runtime.py:
    // 1202-1210, silu_and_mul at hydraserve/kernels/activation.py:66-76),
    // gate and up are rounded to bf16 first, then out = gate * sigmoid(gate)
    // * up in fp32, rounded to bf16, into y [M, N/2].
    for (int q = wave; 2 * q < nblk; q += KW) {
      f32x4_t g = *reinterpret_cast<const f32x4_t*>(red + ((0 * nblk + 2 * q) * 64 + lane) * 4);
      f32x4_t u = *reinterpret_cast<const f32x4_t*>(red + ((0 * nblk + 2 * q + 1) * 64 + lane) * 4);
#pragma unroll
      for (int w = 1; w < KW; ++w) {
        const f32x4_t vg = *reinterpret_cast<const f32x4_t*>(red + ((w * nblk + 2 * q) * 64 + lane) * 4);
        const f32x4_t vu = *reinterpret_cast<const f32x4_t*>(red + ((w * nblk + 2 * q + 1) * 64 + lane) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g[e] += vg[e];
          u[e] += vu[e];
        }
      }
      const int col = r0 / 2 + 16 * q + l16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 4 * h + e;
        if (m < M) {
          const float gb = bf16_to_f32(to_bf16_bits(g[e]));
          const float ub = bf16_to_f32(to_bf16_bits(u[e]));
          const float sig = 1.0f / (1.0f + expf(-gb));
          a.y[m * a.ldy + col] = to_bf16_bits(gb * sig * ub);
        }
      }
    }
    return;
  }
  for (int b = wave; b < nblk; b += KW) {
    f32x4_t s = *reinterpret_cast<const f32x4_t*>(red + ((0 * nblk + b) * 64 + lane) * 4);
#pragma unroll
    for (int w = 1; w < KW; ++w) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(red + ((w * nblk + b) * 64 + lane) * 4);
      s[0] += v[0];
      s[1] += v[1];
      s[2] += v[2];
      s[3] += v[3];
    }
    const int rl = 16 * b + l16;
    if (rl < nr) {
      const int col = r0 + rl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 4 * h + e;
        if (m < M) a.y[m * a.ldy + col] = to_bf16_bits(s[e]);
      }
    }
  }
}

template <int WT, int SDT, int KW, int RD>
static hipError_t launch_gemv_t(const GemmArgs& a, hipStream_t stream) {
  const GemvLds l = gemv_lds(WT, SDT, KW, a.M, a.K, a.G);
  hipLaunchKernelGGL((qgemm_gemv_kernel<WT, SDT, KW, RD>), dim3(a.P), dim3(64 * KW), l.total, stream, a);
  return hipGetLastError();
}

int gemv_rd = 0;  // tuning: ring depth override (4 or 8; 0 = 8)

template <int WT, int SDT>
static hipError_t launch_gemv_wt(const GemmArgs& a, int kw, hipStream_t stream) {
  const int rd = gemv_rd == 4 ? 4 : 8;
#define HSQ_GV(KW_, RD_) \
  if (kw == KW_ && rd == RD_) return launch_gemv_t<WT, SDT, KW_, RD_>(a, stream);
  HSQ_GV(4, 4) HSQ_GV(4, 8) HSQ_GV(8, 4) HSQ_GV(8, 8) HSQ_GV(16, 4) HSQ_GV(16, 8)
#undef HSQ_GV
  return hipErrorInvalidValue;
}

constexpr size_t kGemvMaxLds = 160 * 1024;

// Can the block-major kernel run this problem with P workgroups and
// kw_pref wavefronts per workgroup?
bool gemv_ok(const GemmArgs& a, int wt, int P, int kw_pref, int* kw_out, int* rows_max) {
  if (a.M < 1 || a.M > 16 || !a.xvec || !a.wvec || a.K % 128 != 0 || P < 1) return false;
  const int64_t rb = wt == W_INT4 ? a.ldw * 4 : a.ldw;
  if (static_cast<int64_t>(a.N) * rb >= (int64_t{1} << 31)) return false;
  if ((static_cast<int64_t>(a.M) * a.ldx + a.K) * 2 >= (int64_t{1} << 31)) return false;
  // Only with kw_pref wavefronts: fewer leave too few loads in flight (a
  // layout that does not fit goes to the row-partitioned kernel instead).
  if (a.silu_mul && (wt != W_INT4 || a.N % 32 != 0)) return false;
  const int nr_max = row_partition_max(a, P);
  const int kw = kw_pref;
  if (a.K / 128 < kw) return false;  // every wavefront gets at least one chunk
  if (gemv_lds(wt, a.sdt, kw, a.M, a.K, nr_max).total > kGemvMaxLds) return false;
  *kw_out = kw;
  *rows_max = nr_max;
  return true;
}

hipError_t launch_gemv(int wt, const GemmArgs& a, int kw, hipStream_t stream) {
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_gemv_wt<W_INT4, SCALE_BF16>(a, kw, stream);
    if (a.sdt == SCALE_F16) return launch_gemv_wt<W_INT4, SCALE_F16>(a, kw, stream);
    return launch_gemv_wt<W_INT4, SCALE_F32>(a, kw, stream);
  }
  if (a.sdt == SCALE_BF16) return launch_gemv_wt<W_FP8, SCALE_BF16>(a, kw, stream);
  if (a.sdt == SCALE_F16) return launch_gemv_wt<W_FP8, SCALE_F16>(a, kw, stream);
  return launch_gemv_wt<W_FP8, SCALE_F32>(a, kw, stream);
}

}  // namespace hsq
