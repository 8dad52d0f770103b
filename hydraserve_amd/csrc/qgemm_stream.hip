// Decode-regime (M <= 64) quantized weight GEMM for gfx950: the fast path.
//
// Replaces the Triton launches of hydraserve/kernels/awq.py:52-74
// (_awq_gemm_kernel, awq.py:82-142) and hydraserve/kernels/fp8.py:68-96
// (_fp8_gemm_kernel, fp8.py:104-168) when the activation has at most 64 rows,
// K is a multiple of 128*NB and rows are 16-byte aligned (the host checks;
// other shapes take the masked kernel in qgemm_decode.hip).
//
// The kernel is a weight streamer: HBM bandwidth is the roofline, so the
// design minimises everything that is not a weight byte moving through the
// memory pipeline.
//   * A workgroup (4 wavefronts) owns a tile of 64*S weight rows; wave w owns
//     S strips of 16 rows.  K is walked in batches of NB chunks of 128 (one
//     INT4 group / one FP8 block per chunk); a batch is one stream-K step.
//   * Weights: every lane streams one 16-byte (INT4) or 32-byte (FP8) piece of
//     its row per chunk per strip straight into registers, NB chunks ahead.
//   * Scales / zero points: one vector load per strip per batch (NB groups).
//   * X: staged into LDS once per batch for all four waves, exactly M rows
//     (rows past M are never read: operand rows clamp to M-1 and the
//     corresponding outputs are not stored).  MFMA A operands are LDS reads.
//   * Steady state: every load unconditional, cursors in SGPRs, one barrier
//     per batch, so the compiler keeps the weight ring in flight.
//
// Arithmetic (exact unpack, weights never rounded to bf16):
//   INT4: nibble q -> bf16 128+q (v_perm_b32 + v_bfi_b32 under the exponent
//   of 128.0); T = MFMA(X, 128+q); Xg = MFMA(X, ones) (the group sum of X for
//   the same rows); acc += s * (T - (128+z) * Xg).
//   FP8: E4M3FN -> bf16 exactly (v_cvt_scalef32_pk_bf16_fp8, unit scale);
//   acc += s_block * MFMA(X, W).
#include <type_traits>

#include "qgemm_common.h"

namespace hsq {

constexpr int ST_THREADS = 256;

// No inline asm anywhere near the MFMAs: the compiler's MFMA hazard handling
// does not see through it (an empty asm on accumulators produced stale
// results on gfx950).  (x & mask) | magic with mask/magic in VGPRs compiles
// to a single v_and_or_b32.
__device__ __forceinline__ uint32_t insert_nibbles(uint32_t mask, uint32_t src, uint32_t magic) {
  return (src & mask) | magic;
}

template <int WT, int S>
struct StW;  // weights of one chunk for S strips

template <int S>
struct StW<W_INT4, S> {
  u32x4_t q[S];
};

template <int S>
struct StW<W_FP8, S> {
  u32x4_t q[S][2];
};

template <int WT, int S, int NB>
struct StScale;  // scales (and zero points) of one batch for S strips

template <int S, int NB>
struct StScale<W_INT4, S, NB> {
  uint32_t s[S][NB / 2];  // NB scales as bf16/f16 pairs, or NB/2 ... see loader
  uint32_t s2[S][NB / 2];  // second half when scales are f32
  uint32_t z[S][NB];      // zero-point words
};

template <int S, int NB>
struct StScale<W_FP8, S, NB> {
  uint32_t s[S][NB / 2];
  uint32_t s2[S][NB / 2];
};

template <int WT, int SDT, int MT, int S, int NB, int XR>
struct Stream {
  static constexpr int NT = 64 * S;
  static constexpr int SES = SDT == SCALE_F32 ? 4 : 2;
  static constexpr int XK = NB * 128;       // bf16 per X row per batch
  static constexpr int XSTRIDE = XK + 8;    // LDS row stride (bank spread)
  static constexpr int XSEG = NB * 16;      // 16-byte segments per X row per batch

  // Row addresses of one tile (lane's row l16 of each strip).
  struct Rows {
    const uint8_t* w[S];
    const uint8_t* s[S];
    const uint8_t* z[S];
    uint32_t zsh[S];
  };

  static __device__ __forceinline__ void set_rows(const GemmArgs& a, Rows& r, int t, int wave, int l16) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      int row = t * NT + (wave * S + s) * 16 + l16;
      row = row < a.N ? row : a.N - 1;
      if constexpr (WT == W_INT4) {
        r.w[s] = reinterpret_cast<const uint8_t*>(a.w) + row * a.ldw * 4;
        r.s[s] = reinterpret_cast<const uint8_t*>(a.scale) + row * a.lds * SES;
        r.z[s] = reinterpret_cast<const uint8_t*>(a.zero) + (row >> 3) * a.ldz * 4;
        r.zsh[s] = (row & 7) * 4;
      } else {
        r.w[s] = reinterpret_cast<const uint8_t*>(a.w) + row * a.ldw;
        r.s[s] = reinterpret_cast<const uint8_t*>(a.scale) + (row >> 7) * a.lds * SES;
        r.z[s] = nullptr;
        r.zsh[s] = 0;
      }
    }
  }

  static __device__ __forceinline__ void load_w(StW<WT, S>& r, const Rows& rw, int c, int h) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if constexpr (WT == W_INT4) {
        r.q[s] = *reinterpret_cast<const u32x4_t*>(rw.w[s] + c * 64 + 16 * h);
      } else {
        const uint8_t* p = rw.w[s] + c * 128 + 32 * h;
        r.q[s][0] = *reinterpret_cast<const u32x4_t*>(p);
        r.q[s][1] = *reinterpret_cast<const u32x4_t*>(p + 16);
      }
    }
  }

  // Scales of chunks [c0, c0+NB) (c0 % NB == 0); raw bits, decoded at use.
  static __device__ __forceinline__ void load_scales(StScale<WT, S, NB>& r, const Rows& rw, int c0) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const uint8_t* sp = rw.s[s] + c0 * SES;
      constexpr int WORDS = NB * SES / 4;  // 32-bit words of scales per batch
      uint32_t v[WORDS];
      if constexpr (WORDS == 16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4_t x = *reinterpret_cast<const u32x4_t*>(sp + 16 * q);
          v[4 * q] = x[0]; v[4 * q + 1] = x[1]; v[4 * q + 2] = x[2]; v[4 * q + 3] = x[3];
        }
      } else if constexpr (WORDS == 8) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const u32x4_t x = *reinterpret_cast<const u32x4_t*>(sp + 16 * q);
          v[4 * q] = x[0]; v[4 * q + 1] = x[1]; v[4 * q + 2] = x[2]; v[4 * q + 3] = x[3];
        }
      } else if constexpr (WORDS == 4) {
        const u32x4_t x = *reinterpret_cast<const u32x4_t*>(sp);
        v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
      } else if constexpr (WORDS == 2) {
        const uint2 x = *reinterpret_cast<const uint2*>(sp);
        v[0] = x.x; v[1] = x.y;
      } else {
        v[0] = *reinterpret_cast<const uint32_t*>(sp);
      }
      if constexpr (SES == 2) {
#pragma unroll
        for (int i = 0; i < NB / 2; ++i) r.s[s][i] = v[i];
      } else {
#pragma unroll
        for (int i = 0; i < NB / 2; ++i) {
          r.s[s][i] = v[2 * i];
          r.s2[s][i] = v[2 * i + 1];
        }
      }
      if constexpr (WT == W_INT4) {
        const uint8_t* zp = rw.z[s] + c0 * 4;
        if constexpr (NB == 8) {
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const u32x4_t x = *reinterpret_cast<const u32x4_t*>(zp + 16 * q);
            r.z[s][4 * q] = x[0]; r.z[s][4 * q + 1] = x[1]; r.z[s][4 * q + 2] = x[2]; r.z[s][4 * q + 3] = x[3];
          }
        } else if constexpr (NB == 4) {
          const u32x4_t x = *reinterpret_cast<const u32x4_t*>(zp);
          r.z[s][0] = x[0]; r.z[s][1] = x[1]; r.z[s][2] = x[2]; r.z[s][3] = x[3];
        } else {
          const uint2 x = *reinterpret_cast<const uint2*>(zp);
          r.z[s][0] = x.x; r.z[s][1] = x.y;
        }
      }
    }
  }

  static __device__ __forceinline__ float scale_of(const StScale<WT, S, NB>& r, int s, int u) {
    if constexpr (SES == 4) {
      return __uint_as_float((u & 1) ? r.s2[s][u >> 1] : r.s[s][u >> 1]);
    } else {
      const uint32_t pair = r.s[s][u >> 1];
      const uint32_t h16 = (u & 1) ? (pair >> 16) : (pair & 0xFFFFu);
      if constexpr (SDT == SCALE_BF16) return __uint_as_float(h16 << 16);
      return __half2float(__ushort_as_half(static_cast<unsigned short>(h16)));
    }
  }

  // X batch: rows [0, M), K [c0*128, c0*128 + XK), M <= XR.  256 threads
  // cover RPQ = 256 / XSEG rows per pass; thread tid takes segment
  // tid % XSEG of row tid / XSEG + RPQ*q.  Rows past M reload row M-1 (so
  // every load is unconditional) and are not stored.
  static_assert(ST_THREADS % XSEG == 0, "a pass must cover whole rows");
  static constexpr int RPQ = ST_THREADS / XSEG;
  static constexpr int XQ = (XR + RPQ - 1) / RPQ;

  static __device__ __forceinline__ void load_x(const GemmArgs& a, u32x4_t (&xr)[XQ], int c0, int tid) {
    const int seg = tid % XSEG;
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      int row = tid / XSEG + RPQ * q;
      row = row < a.M ? row : a.M - 1;
      xr[q] = *reinterpret_cast<const u32x4_t*>(a.x + row * a.ldx + c0 * 128 + seg * 8);
    }
  }

  static __device__ __forceinline__ void store_x(const GemmArgs& a, uint16_t* xs, const u32x4_t (&xr)[XQ], int tid) {
    const int seg = tid % XSEG;
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int row = tid / XSEG + RPQ * q;
      if (row < a.M) *reinterpret_cast<u32x4_t*>(xs + row * XSTRIDE + seg * 8) = xr[q];
    }
  }

  static __device__ __forceinline__ bf16x8_t int4_operand(uint32_t w, uint32_t nib_mask, uint32_t magic) {
    const uint32_t t = w >> 4;
    u32x4_t p;
    p[0] = insert_nibbles(nib_mask, __builtin_amdgcn_perm(t, w, 0x0C040C00u), magic);
    p[1] = insert_nibbles(nib_mask, __builtin_amdgcn_perm(t, w, 0x0C050C01u), magic);
    p[2] = insert_nibbles(nib_mask, __builtin_amdgcn_perm(t, w, 0x0C060C02u), magic);
    p[3] = insert_nibbles(nib_mask, __builtin_amdgcn_perm(t, w, 0x0C070C03u), magic);
    return __builtin_bit_cast(bf16x8_t, p);
  }

  static __device__ __forceinline__ bf16x8_t fp8_operand(uint32_t d0, uint32_t d1) {
    u32x4_t p;
    p[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
    p[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
    p[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
    p[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
    return __builtin_bit_cast(bf16x8_t, p);
  }

  // Unit u of the batch (chunk c0 + u).  Lane (l16, h): A rows 16i + l16
  // (clamped to M-1), K [u*128 + 32h + 8j, +8) of the staged batch.
  static __device__ __forceinline__ void compute(const uint16_t* xs, int u, const StW<WT, S>& w,
                                                 const StScale<WT, S, NB>& sc, const Rows& rw,
                                                 f32x4_t (&acc)[S][MT], int arow[MT], int h,
                                                 uint32_t nib_mask, uint32_t magic, bf16x8_t ones) {
    bf16x8_t A[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        A[i][j] = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const u32x4_t*>(xs + arow[i] * XSTRIDE + u * 128 + 32 * h + 8 * j));
    f32x4_t xg[MT];
    if constexpr (WT == W_INT4) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        xg[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) xg[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i][j], ones, xg[i], 0, 0, 0);
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      bf16x8_t B[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (WT == W_INT4) {
          B[j] = int4_operand(w.q[s][j], nib_mask, magic);
        } else {
          B[j] = fp8_operand(w.q[s][j >> 1][(j & 1) * 2], w.q[s][j >> 1][(j & 1) * 2 + 1]);
        }
      }
      const float sc_s = scale_of(sc, s, u);
      float negc = 0.f;
      if constexpr (WT == W_INT4) negc = -(128.0f + static_cast<float>((sc.z[s][u] >> rw.zsh[s]) & 0xFu));
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        f32x4_t tmp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i][j], B[j], tmp, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (WT == W_INT4) {
            acc[s][i][e] = fmaf(sc_s, fmaf(negc, xg[i][e], tmp[e]), acc[s][i][e]);
          } else {
            acc[s][i][e] = fmaf(sc_s, tmp[e], acc[s][i][e]);
          }
        }
      }
    }
  }

  // Lane (l16, h) of wave `wave`: rows 16i + 4h + e, column t*NT + (wave*S+s)*16 + l16.
  static __device__ __forceinline__ void store_tile(const GemmArgs& a, const f32x4_t (&acc)[S][MT], int t, int wave,
                                                    int l16, int h) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int n = t * NT + (wave * S + s) * 16 + l16;
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 16 * i + 4 * h + e;
          if (m < a.M) a.y[m * a.ldy + n] = to_bf16_bits(acc[s][i][e]);
        }
    }
  }

  static constexpr int SLOT = 4 * S * MT * 4 * 64;
  static __device__ __forceinline__ float* slot_ptr(const GemmArgs& a, int p, int slot) {
    return a.partials + (static_cast<int64_t>(p) * 2 + slot) * SLOT;
  }
  static __device__ __forceinline__ int part_off(int wave, int s, int i, int lane) {
    return (((wave * S + s) * MT + i) * 64 + lane) * 4;
  }

  static __device__ __forceinline__ void finish_tile(const GemmArgs& a, int* flag, f32x4_t (&acc)[S][MT], int t, int p,
                                                     int64_t b0, int64_t b1, int tid) {
    const int wave = tid >> 6, lane = tid & 63, l16 = lane & 15, h = lane >> 4;
    const int64_t ts = static_cast<int64_t>(t) * a.G, te = ts + a.G;
    if (b0 <= ts && b1 >= te) {
      store_tile(a, acc, t, wave, l16, h);
      return;
    }
    const int pf = unit_owner(ts, a.U, a.P), pl = unit_owner(te - 1, a.U, a.P);
    float* mine = slot_ptr(a, p, partial_slot(p, t, a.G, a.U, a.P));
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) store_partial(mine + part_off(wave, s, i, lane) + e, acc[s][i][e]);
    if (!arrive_last(a.counters, t, pl - pf + 1, flag)) return;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[s][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int q = pf; q <= pl; ++q) {
      const float* src = slot_ptr(a, q, partial_slot(q, t, a.G, a.U, a.P));
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[s][i][e] += load_partial(src + part_off(wave, s, i, lane) + e);
    }
    store_tile(a, acc, t, wave, l16, h);
    reset_counter(a.counters, t);
  }
};

// a.G = batches per tile, a.NB = NB, a.U = T * a.G, a.P = workgroups.
// Dynamic LDS: 2 X buffers of M rows (+ a flag word).
template <int WT, int SDT, int MT, int S, int NB, int XR>
__global__ __launch_bounds__(ST_THREADS) void qgemm_stream_kernel(GemmArgs a) {
  using D = Stream<WT, SDT, MT, S, NB, XR>;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* xs0 = smem;
  uint16_t* xs1 = smem + a.M * D::XSTRIDE;
  int* flag = reinterpret_cast<int*>(smem + 2 * a.M * D::XSTRIDE);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(tid >> 6));
  const int lane = tid & 63, l16 = lane & 15, h = lane >> 4;
  const int p = blockIdx.x;
  const int64_t b0 = unit_begin(p, a.U, a.P), b1 = unit_begin(p + 1, a.U, a.P);
  if (b0 >= b1) return;
  const int GC = a.G * NB;  // chunks per tile
  const uint32_t nib_mask = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t magic = opaque_and(0x43004300u, 0xFFFFFFFFu);
  const uint32_t one2 = opaque_and(0x3F803F80u, 0xFFFFFFFFu);
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{one2, one2, one2, one2});
  int arow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) arow[i] = (16 * i + l16) < a.M ? 16 * i + l16 : a.M - 1;

  // Cursors over chunks.  `ld` (weights) runs NB chunks ahead of `cur`; the
  // batch cursor `lb` (X, scales) one batch ahead.  Loaders stop at the
  // range's last chunk / batch: refills past it reload that (L2 hits).
  const int first = static_cast<int>(b0) * NB, last = static_cast<int>(b1) * NB - 1;
  Cursor cur{first / GC, first % GC};
  Cursor ld = cur;
  int ld_lin = first;
  typename D::Rows lrw, crw;
  D::set_rows(a, lrw, ld.t, wave, l16);
  crw = lrw;
  Cursor lb = cur;  // chunk cursor of the next batch to stage
  int lb_lin = first;
  typename D::Rows brw = lrw;  // rows of the tile `lb` is in
  auto advance_ld = [&]() {
    if (ld_lin < last) {
      ++ld_lin;
      ld.advance(GC);
      if (ld.c == 0) D::set_rows(a, lrw, ld.t, wave, l16);
    }
  };
  auto advance_lb = [&]() {
    if (lb_lin + NB <= last) {
      lb_lin += NB;
      lb.c += NB;
      if (lb.c == GC) {
        lb.c = 0;
        ++lb.t;
        D::set_rows(a, brw, lb.t, wave, l16);
      }
    }
  };

  StW<WT, S> ring[NB];
  StScale<WT, S, NB> sc_cur, sc_next;
  u32x4_t xr[D::XQ];
  // Prologue: batch 0's X and scales, NB chunks of weights, batch 1's X/scales.
  D::load_x(a, xr, lb.c, tid);
  D::load_scales(sc_cur, brw, lb.c);
  advance_lb();
#pragma unroll
  for (int r = 0; r < NB; ++r) {
    D::load_w(ring[r], lrw, ld.c, h);
    advance_ld();
  }
  D::store_x(a, xs0, xr, tid);
  D::load_x(a, xr, lb.c, tid);
  D::load_scales(sc_next, brw, lb.c);
  advance_lb();
  __syncthreads();

  int64_t batch = b0;
  int buf = 0;
  while (batch < b1) {
    const int t = cur.t;
    int64_t seg_end = (static_cast<int64_t>(t) + 1) * a.G;
    if (seg_end > b1) seg_end = b1;
    f32x4_t acc[S][MT];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[s][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (; batch < seg_end; ++batch) {
      const uint16_t* xs = buf ? xs1 : xs0;
#pragma unroll
      for (int r = 0; r < NB; ++r) {
        D::compute(xs, r, ring[r], sc_cur, crw, acc, arow, h, nib_mask, magic, ones);
        D::load_w(ring[r], lrw, ld.c, h);  // weights NB chunks ahead
        advance_ld();
        __builtin_amdgcn_sched_barrier(0);
      }
      // Publish the next batch's X into the other buffer, then prefetch the
      // one after (its registers were consumed by the store).
      D::store_x(a, buf ? xs0 : xs1, xr, tid);
      sc_cur = sc_next;
      D::load_x(a, xr, lb.c, tid);
      D::load_scales(sc_next, brw, lb.c);
      advance_lb();
      __syncthreads();
      buf ^= 1;
      cur.c += NB;
      if (cur.c == GC) {
        cur.c = 0;
        ++cur.t;
      }
    }
    D::finish_tile(a, flag, acc, t, p, b0, b1, tid);
    if (cur.c == 0) D::set_rows(a, crw, cur.t, wave, l16);
  }
}

template <int WT, int SDT, int MT, int S, int NB, int XR>
static hipError_t launch_stream_t(const GemmArgs& a, hipStream_t stream) {
  using D = Stream<WT, SDT, MT, S, NB, XR>;
  const size_t lds = static_cast<size_t>(2) * a.M * D::XSTRIDE * 2 + 16;
  hipLaunchKernelGGL((qgemm_stream_kernel<WT, SDT, MT, S, NB, XR>), dim3(a.P), dim3(ST_THREADS), lds, stream, a);
  return hipGetLastError();
}

template <int WT, int SDT>
static hipError_t launch_stream_wt(const GemmArgs& a, int MT, int S, hipStream_t stream) {
  const int xr = a.M <= 4 ? 4 : 16 * MT;
#define HSQ_ST(mt, s, nb, r) \
  if (MT == mt && S == s && a.NB == nb && xr == r) return launch_stream_t<WT, SDT, mt, s, nb, r>(a, stream);
  HSQ_ST(1, 1, 8, 4) HSQ_ST(1, 2, 8, 4) HSQ_ST(1, 1, 8, 16) HSQ_ST(1, 2, 8, 16)
  HSQ_ST(1, 1, 4, 4) HSQ_ST(1, 2, 4, 4) HSQ_ST(1, 1, 4, 16) HSQ_ST(1, 2, 4, 16)
  HSQ_ST(2, 1, 4, 32) HSQ_ST(2, 2, 4, 32)
  HSQ_ST(4, 1, 2, 64) HSQ_ST(4, 2, 2, 64)
#undef HSQ_ST
  return hipErrorInvalidValue;
}

int stream_slot_floats(int MT, int S) { return 4 * S * MT * 4 * 64; }

// Can the fast path run this problem with NB chunks per batch?  Scale and
// zero-point rows are read with one vector per batch, so their base and row
// stride must be aligned to that vector.
bool stream_ok(const GemmArgs& a, int wt, int NB) {
  if (a.M < 1 || a.M > 64 || !a.xvec || !a.wvec || a.K % (128 * NB) != 0) return false;
  const int ses = a.sdt == SCALE_F32 ? 4 : 2;
  const int sbytes = NB * ses;  // scale bytes per batch per row
  const int salign = sbytes >= 16 ? 16 : sbytes;
  if ((a.lds * ses) % salign != 0 || reinterpret_cast<uintptr_t>(a.scale) % salign != 0) return false;
  if (wt == W_INT4) {
    const int zbytes = NB * 4;
    const int zalign = zbytes >= 16 ? 16 : zbytes;
    if ((a.ldz * 4) % zalign != 0 || reinterpret_cast<uintptr_t>(a.zero) % zalign != 0) return false;
  }
  return true;
}

hipError_t launch_stream(int wt, const GemmArgs& a, int MT, int S, hipStream_t stream) {
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_stream_wt<W_INT4, SCALE_BF16>(a, MT, S, stream);
    if (a.sdt == SCALE_F16) return launch_stream_wt<W_INT4, SCALE_F16>(a, MT, S, stream);
    return launch_stream_wt<W_INT4, SCALE_F32>(a, MT, S, stream);
  }
  if (a.sdt == SCALE_BF16) return launch_stream_wt<W_FP8, SCALE_BF16>(a, MT, S, stream);
  if (a.sdt == SCALE_F16) return launch_stream_wt<W_FP8, SCALE_F16>(a, MT, S, stream);
  return launch_stream_wt<W_FP8, SCALE_F32>(a, MT, S, stream);
}

}  // namespace hsq
