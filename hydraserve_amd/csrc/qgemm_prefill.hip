// Prefill-regime (M > 64) quantized weight GEMM for gfx950.
//
// Replaces the Triton launches of hydraserve/kernels/awq.py:52-74 and
// hydraserve/kernels/fp8.py:68-96 for large M.
//
// Tiling.  A workgroup (4 wavefronts) computes a BM x 256 output tile; wave w
// owns all BM rows and output columns [64w, 64w+64), i.e. a BM x 64 wave tile
// built from 32x32 v_mfma_f32_32x32x16_bf16 blocks (fp32 accumulators live in
// AGPRs).  K advances 64 at a time (one "unit"; half an INT4 group, half an FP8
// block).  The X tile [BM x 64] is staged through double-buffered LDS and
// shared by the four waves; every wave decodes only its own 64 weight rows
// straight from global memory into registers, so each weight element is
// decoded once per workgroup and no dequantized weight ever touches memory.
//
// Decode matches the reference's weight bits exactly:
//   INT4: bf16_rne((q - z) * s) computed as fma(q, s, -z*s) in fp32 (exact,
//         since (q-z)*s has at most 12 significant bits), then
//         v_cvt_pk_bf16_f32 -- identical to awq.py:18-22 and awq.py:136-137.
//   FP8:  bf16_rne(fp32(decode(b)) * fp32(s)) -- identical to the Triton kernel
//         at fp8.py:144-161 (v_cvt_pk_f32_fp8 decodes E4M3FN exactly).
// Output tiles are scheduled with the same stream-K split as the decode kernel.
#include "qgemm_common.h"

namespace hsq {

constexpr int PF_THREADS = 256;

template <int WT, int SDT, int BM>
struct Prefill {
  static constexpr int BN = 256;
  static constexpr int BK = 64;
  static constexpr int MI = BM / 32;
  static constexpr int AS = BK + 8;  // LDS row stride in bf16: 144 B spreads 16 rows over 64 banks
  static constexpr int XR = BM / 32;  // 16-byte X segments per thread per unit

  struct Smem {
    __attribute__((aligned(16))) uint16_t xs[2][BM][AS];
    int flag;
  };

  struct WRegs {
    u32x4_t q[2][WT == W_INT4 ? 1 : 2];
    float s[2];
    float nzs[2];  // INT4: -z*s
  };

  static __device__ __forceinline__ void tile_coords(const GemmArgs& a, int t, int& tm, int& tn) {
    tn = t / a.TM;
    tm = t - tn * a.TM;
  }

  static __device__ __forceinline__ void load_w(const GemmArgs& a, WRegs& r, int tn, int c, int wave, int l32,
                                                int h) {
    const int kw = (a.K + 7) >> 3;
    // Uniform: the whole 64-wide chunk is inside K and rows allow 16-byte loads.
    const bool full = a.wvec && (WT == W_INT4 ? (c + 1) * 8 <= kw : (c + 1) * BK <= a.K);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int row = tn * BN + wave * 64 + 32 * j + l32;
      row = row < a.N ? row : a.N - 1;
      if constexpr (WT == W_INT4) {
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(a.w) + row * a.ldw;
        const int w0 = c * 8 + 4 * h;
        if (full) {
          r.q[j][0] = *reinterpret_cast<const u32x4_t*>(wp + w0);
        } else {
          u32x4_t v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (w0 + e < kw) ? wp[w0 + e] : 0u;
          r.q[j][0] = v;
        }
        const int g = c >> 1;  // 128-wide group
        const float s = load_scale<SDT>(a.scale, row * a.lds + g);
        const uint32_t zw = static_cast<uint32_t>(a.zero[(row >> 3) * a.ldz + g]);
        const float z = static_cast<float>((zw >> ((row & 7) * 4)) & 0xFu);
        r.s[j] = s;
        r.nzs[j] = -(z * s);
      } else {
        const uint8_t* wp = reinterpret_cast<const uint8_t*>(a.w) + row * a.ldw;
        const int b0 = c * 64 + 32 * h;
        if (full) {
          r.q[j][0] = *reinterpret_cast<const u32x4_t*>(wp + b0);
          r.q[j][1] = *reinterpret_cast<const u32x4_t*>(wp + b0 + 16);
        } else {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            u32x4_t v;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              uint32_t word = 0;
#pragma unroll
              for (int by = 0; by < 4; ++by) {
                const int kk = b0 + hh * 16 + e * 4 + by;
                word |= static_cast<uint32_t>((kk < a.K) ? wp[kk] : 0) << (8 * by);
              }
              v[e] = word;
            }
            r.q[j][hh] = v;
          }
        }
        r.s[j] = load_scale<SDT>(a.scale, (row >> 7) * a.lds + (c >> 1));
        r.nzs[j] = 0.f;
      }
    }
  }

  // X tile rows [tm*BM, tm*BM+BM), K [c*64, c*64+64).  Thread tid takes
  // segment (tid & 7) of rows (tid >> 3) + 32q.  Rows past M repeat row M-1
  // (finite values, never stored); K past the end reads as zero.
  static __device__ __forceinline__ void load_x(const GemmArgs& a, u32x4_t (&xr)[XR], int tm, int c, int tid) {
    const int seg = tid & 7;
    const int k0 = c * BK + seg * 8;
    const bool full = a.xvec && (c + 1) * BK <= a.K;  // uniform
#pragma unroll
    for (int q = 0; q < XR; ++q) {
      int row = tm * BM + (tid >> 3) + 32 * q;
      row = row < a.M ? row : a.M - 1;
      const uint16_t* xp = a.x + row * a.ldx;
      if (full) {
        xr[q] = *reinterpret_cast<const u32x4_t*>(xp + k0);
      } else {
        u32x4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = (k0 + 2 * e < a.K) ? xp[k0 + 2 * e] : 0u;
          const uint32_t hi = (k0 + 2 * e + 1 < a.K) ? xp[k0 + 2 * e + 1] : 0u;
          v[e] = lo | (hi << 16);
        }
        xr[q] = v;
      }
    }
  }

  static __device__ __forceinline__ void store_x(Smem& sm, const u32x4_t (&xr)[XR], int b, int tid) {
    const int seg = tid & 7;
#pragma unroll
    for (int q = 0; q < XR; ++q)
      *reinterpret_cast<u32x4_t*>(&sm.xs[b][(tid >> 3) + 32 * q][seg * 8]) = xr[q];
  }

  static __device__ __forceinline__ void decode_b(const WRegs& r, bf16x8_t (&B)[2][4]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        u32x4_t p;
        if constexpr (WT == W_INT4) {
          const uint32_t w = r.q[j][0][t];
          const uint32_t t0 = opaque_and(w, 0x0F0F0F0Fu), t1 = opaque_and(w >> 4, 0x0F0F0F0Fu);
          const float s = r.s[j], c = r.nzs[j];
          p[0] = pack_bf16x2(fmaf(static_cast<float>(t0 & 0xFFu), s, c), fmaf(static_cast<float>(t1 & 0xFFu), s, c));
          p[1] = pack_bf16x2(fmaf(static_cast<float>((t0 >> 8) & 0xFFu), s, c),
                             fmaf(static_cast<float>((t1 >> 8) & 0xFFu), s, c));
          p[2] = pack_bf16x2(fmaf(static_cast<float>((t0 >> 16) & 0xFFu), s, c),
                             fmaf(static_cast<float>((t1 >> 16) & 0xFFu), s, c));
          p[3] = pack_bf16x2(fmaf(static_cast<float>(t0 >> 24), s, c), fmaf(static_cast<float>(t1 >> 24), s, c));
        } else {
          const float s = r.s[j];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const uint32_t d = r.q[j][t >> 1][(t & 1) * 2 + e];
            const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(d, false);
            const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(d, true);
            p[2 * e] = pack_bf16x2(lo[0] * s, lo[1] * s);
            p[2 * e + 1] = pack_bf16x2(hi[0] * s, hi[1] * s);
          }
        }
        B[j][t] = __builtin_bit_cast(bf16x8_t, p);
      }
  }

  static __device__ __forceinline__ void load_a(const Smem& sm, int b, int t, bf16x8_t (&A)[MI], int l32, int h) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
      A[i] = __builtin_bit_cast(bf16x8_t,
                                *reinterpret_cast<const u32x4_t*>(&sm.xs[b][32 * i + l32][32 * h + 8 * t]));
  }

  // Four k16 steps; the A fragments of step t+1 are read from LDS while the
  // MFMAs of step t run.
  static __device__ __forceinline__ void compute(const Smem& sm, int b, const bf16x8_t (&B)[2][4],
                                                 f32x16_t (&acc)[MI][2], int l32, int h) {
    bf16x8_t A[2][MI];
    load_a(sm, b, 0, A[0], l32, h);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < 3) load_a(sm, b, t + 1, A[(t + 1) & 1], l32, h);
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[t & 1][i], B[0][t], acc[i][0], 0, 0, 0);
        acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[t & 1][i], B[1][t], acc[i][1], 0, 0, 0);
      }
    }
  }

  // Lane (l32, h), register e of block (i, j): row 32i + 8(e/4) + 4h + e%4,
  // column 64*wave + 32j + l32.
  static __device__ __forceinline__ void store_tile(const GemmArgs& a, const f32x16_t (&acc)[MI][2], int t,
                                                    int wave, int l32, int h) {
    int tm, tn;
    tile_coords(a, t, tm, tn);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = tn * BN + wave * 64 + 32 * j + l32;
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = tm * BM + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
          if (m < a.M) a.y[m * a.ldy + n] = to_bf16_bits(acc[i][j][e]);
        }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  static constexpr int SLOT = 4 * MI * 2 * 16 * 64;
  // Partial layout (bytes in a slot): 16-byte chunk v (elements 4v..4v+3)
  // of accumulator block b = (wave*MI + i)*2 + j of a lane at
  // ((b*4 + v)*64 + lane)*16, so every 16-byte store or load covers 1 KB.
  static __device__ __forceinline__ uint32_t part_off(int b, int v, int lane) {
    return static_cast<uint32_t>(((b * 4 + v) * 64 + lane) * 16);
  }

  static __device__ __forceinline__ uint32_t slot_off(int p, int slot) {
    return static_cast<uint32_t>((p * 2 + slot) * SLOT * 4);
  }

  static __device__ __forceinline__ void finish_tile(const GemmArgs& a, Smem& sm, f32x16_t (&acc)[MI][2], int t,
                                                     int p, int64_t u0, int64_t u1, int tid) {
    const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int64_t ts = static_cast<int64_t>(t) * a.G, te = ts + a.G;
    if (u0 <= ts && u1 >= te) {
      store_tile(a, acc, t, wave, l32, h);
      return;
    }
    const int pf = unit_owner(ts, a.U, a.P), pl = unit_owner(te - 1, a.U, a.P);
    const auto pr = partial_rsrc(a.partials);
    const uint32_t mine = slot_off(p, partial_slot(p, t, a.G, a.U, a.P));
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          store_partial4(pr, mine + part_off((wave * MI + i) * 2 + j, v, lane),
                         f32x4_t{acc[i][j][4 * v], acc[i][j][4 * v + 1], acc[i][j][4 * v + 2], acc[i][j][4 * v + 3]});
        __builtin_amdgcn_sched_barrier(0);
      }
    if (!arrive_last(a.counters, t, pl - pf + 1, &sm.flag)) return;
    // Sum every contributor's slot (our own included) in workgroup order.
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[i][0] = acc[i][1] = f32x16_t{};
    for (int q = pf; q <= pl; ++q) {
      const uint32_t base = slot_off(q, partial_slot(q, t, a.G, a.U, a.P));
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const f32x4_t x = load_partial4(pr, base + part_off((wave * MI + i) * 2 + j, v, lane));
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[i][j][4 * v + c] += x[c];
          }
    }
    store_tile(a, acc, t, wave, l32, h);
    reset_counter(a.counters, t);
  }
};

template <int WT, int SDT, int BM>
__global__ __launch_bounds__(PF_THREADS) void qgemm_prefill_kernel(GemmArgs a) {
  using PF = Prefill<WT, SDT, BM>;
  __shared__ typename PF::Smem sm;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int p = blockIdx.x;
  const int64_t u0 = unit_begin(p, a.U, a.P), u1 = unit_begin(p + 1, a.U, a.P);
  if (u0 >= u1) return;

  u32x4_t xr[PF::XR];
  // Weight registers: `wc` feeds the unit being computed, `wn` is the next
  // unit's load already in flight (two units of weights ahead of the MFMAs).
  typename PF::WRegs wc, wn;
  const int n_units = static_cast<int>(u1 - u0);
  Cursor cur{static_cast<int>(u0 / a.G), static_cast<int>(u0 % a.G)};
  Cursor ld = cur;
  int tm, tn;
  PF::tile_coords(a, cur.t, tm, tn);
  PF::load_x(a, xr, tm, cur.c, tid);
  PF::load_w(a, wc, tn, cur.c, wave, l32, h);
  ld.advance(a.G);
  if (n_units > 1) {
    PF::tile_coords(a, ld.t, tm, tn);
    PF::load_w(a, wn, tn, ld.c, wave, l32, h);
  }
  ld.advance(a.G);
  PF::store_x(sm, xr, 0, tid);
  __syncthreads();

  // Tile-outer / unit-inner loops keep the accumulators' only loop-carried
  // definition the MFMA itself, so they stay in AGPRs.
  int j = 0;
  while (j < n_units) {
    const int t = cur.t;
    int tile_left = a.G - cur.c;
    if (tile_left > n_units - j) tile_left = n_units - j;
    PF::tile_coords(a, t, tm, tn);
    f32x16_t acc[PF::MI][2];
#pragma unroll
    for (int i = 0; i < PF::MI; ++i) acc[i][0] = acc[i][1] = f32x16_t{};
    for (int q = 0; q < tile_left; ++q, ++j) {
      const int b = j & 1;
      const bool last = (q + 1 == tile_left);
      if (!last) PF::load_x(a, xr, tm, cur.c + 1, tid);
      bf16x8_t B[2][4];
      PF::decode_b(wc, B);
      wc = wn;
      if (j + 2 < n_units) {
        int ltm, ltn;
        PF::tile_coords(a, ld.t, ltm, ltn);
        PF::load_w(a, wn, ltn, ld.c, wave, l32, h);
        ld.advance(a.G);
      }
      PF::compute(sm, b, B, acc, l32, h);
      if (!last) {
        PF::store_x(sm, xr, b ^ 1, tid);
        __syncthreads();
      }
      cur.advance(a.G);
    }
    PF::finish_tile(a, sm, acc, t, p, u0, u1, tid);
    if (j < n_units) {
      // First unit of the next tile goes to the other buffer.
      PF::tile_coords(a, cur.t, tm, tn);
      PF::load_x(a, xr, tm, cur.c, tid);
      PF::store_x(sm, xr, j & 1, tid);
    }
    __syncthreads();
  }
}

template <int WT, int SDT, int BM>
static hipError_t launch_prefill_t(const GemmArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((qgemm_prefill_kernel<WT, SDT, BM>), dim3(a.P), dim3(PF_THREADS), 0, stream, a);
  return hipGetLastError();
}

int prefill_slot_floats(int BM) { return 4 * (BM / 32) * 2 * 16 * 64; }

template <int WT, int SDT>
static hipError_t launch_prefill_wt(const GemmArgs& a, int BM, hipStream_t stream) {
  if (BM == 64) return launch_prefill_t<WT, SDT, 64>(a, stream);
  if (BM == 128) return launch_prefill_t<WT, SDT, 128>(a, stream);
  if (BM == 256) return launch_prefill_t<WT, SDT, 256>(a, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_prefill(int wt, const GemmArgs& a, int BM, hipStream_t stream) {
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_prefill_wt<W_INT4, SCALE_BF16>(a, BM, stream);
    if (a.sdt == SCALE_F16) return launch_prefill_wt<W_INT4, SCALE_F16>(a, BM, stream);
    return launch_prefill_wt<W_INT4, SCALE_F32>(a, BM, stream);
  }
  if (a.sdt == SCALE_BF16) return launch_prefill_wt<W_FP8, SCALE_BF16>(a, BM, stream);
  if (a.sdt == SCALE_F16) return launch_prefill_wt<W_FP8, SCALE_F16>(a, BM, stream);
  return launch_prefill_wt<W_FP8, SCALE_F32>(a, BM, stream);
}

}  // namespace hsq
