// Decode-regime (M <= 64) quantized weight GEMM for gfx950.
//
// Replaces the launch of hydraserve/kernels/awq.py:52-74 (_awq_gemm_kernel,
// awq.py:82-142) and hydraserve/kernels/fp8.py:68-96 (_fp8_gemm_kernel,
// fp8.py:104-168) when the flattened activation has at most 64 rows.
//
// Shape of the work.  A workgroup is 4 wavefronts; each wavefront owns S
// "strips" of 16 weight rows (output features), so a tile is 64*S rows.  A unit
// is one tile x one 128-wide K chunk (one INT4 group, one FP8 scale block).
// For every unit the workgroup stages the X chunk [M x 128] in LDS once and
// each wavefront streams its weight strips straight from HBM into registers
// with 16-byte loads (one INT4 strip-chunk = 16 rows x 64 B, one FP8
// strip-chunk = 16 rows x 128 B), NBUF units ahead of use.
//
// Arithmetic.  Weights are decoded in registers and fed to
// v_mfma_f32_16x16x32_bf16 with X padded to 16*MT rows.  The K order inside a
// chunk is permuted identically for X and W (any common permutation leaves the
// dot product unchanged), which lets every lane take one 16-byte run of a
// weight row.
//
//   INT4: a nibble q is turned into the bf16 value 128+q by inserting it into
//   the mantissa of 128.0 (0x4300), two nibbles per v_bfi_b32.  For each group
//   the MFMA yields T = sum_k x_k (128 + q_k); the true group sum is
//   sum_k x_k (q_k - z) = T - (128 + z) * Xg with Xg = sum_k x_k (computed once
//   per chunk in LDS), then scaled by s and accumulated:
//       acc += s * (T - (128 + z) * Xg).
//   Integer unpack is exact; the weight is never rounded to bf16, so the result
//   differs from the reference's bf16-rounded dequantized weight only by that
//   rounding (well inside the stated tolerance).
//
//   FP8: E4M3FN bytes convert exactly to bf16 (v_cvt_scalef32_pk_bf16_fp8 with
//   unit scale; every finite E4M3FN value, subnormals included, is a bf16).
//   The 128x128 block scale is constant across a strip and a chunk, so it is
//   applied once per chunk to the MFMA result: acc += s_block * T.
//
// KFULL variant: when K is a multiple of 128 and X / W rows are 16-byte
// aligned, every load in the loop is an unconditional vector load (no branch,
// so the compiler can keep NBUF units of loads in flight).  Other shapes use
// the masked variant.
#include <type_traits>

#include "qgemm_common.h"

namespace hsq {

constexpr int DEC_THREADS = 256;
constexpr int XS_STRIDE = 136;  // bf16 per LDS row: 128 + 8 pad (bank spread)

// v_bfi_b32: (mask & src) | (~mask & base), one instruction.
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t src, uint32_t base) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(src), "v"(base));
  return r;
}

template <int WT, int S>
struct WRegs;

template <int S>
struct WRegs<W_INT4, S> {
  u32x4_t q[S];
  float s[S];
  uint32_t z[S];  // zero-point word (nibble selected at use)
};

template <int S>
struct WRegs<W_FP8, S> {
  u32x4_t q[S][2];
  float s[S];
};

// Per-strip row addresses for one tile (recomputed when the tile changes).
template <int S>
struct RowPtrs {
  const uint8_t* w[S];   // weight row
  const uint8_t* s[S];   // scale row (INT4: row n; FP8: row n/128)
  const int32_t* z[S];   // INT4 zero-point row n/8
  uint32_t zsh[S];       // INT4: 4 * (n % 8)
};

template <int WT, int SDT, int MT, int S, bool KFULL>
struct Decode {
  static constexpr int NT = 64 * S;
  static constexpr int ROWS = 16 * MT;
  static constexpr int SES = SDT == SCALE_F32 ? 4 : 2;  // scale element size

  struct Smem {
    __attribute__((aligned(16))) uint16_t xs[2][ROWS][XS_STRIDE];
    __attribute__((aligned(16))) float xsum[2][ROWS];
    int flag;
  };

  static __device__ __forceinline__ void set_rows(const GemmArgs& a, RowPtrs<S>& rp, int t, int wave, int l16) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      int row = t * NT + (wave * S + s) * 16 + l16;
      row = row < a.N ? row : a.N - 1;
      if constexpr (WT == W_INT4) {
        rp.w[s] = reinterpret_cast<const uint8_t*>(a.w) + row * a.ldw * 4;
        rp.s[s] = reinterpret_cast<const uint8_t*>(a.scale) + row * a.lds * SES;
        rp.z[s] = a.zero + (row >> 3) * a.ldz;
        rp.zsh[s] = (row & 7) * 4;
      } else {
        rp.w[s] = reinterpret_cast<const uint8_t*>(a.w) + row * a.ldw;
        rp.s[s] = reinterpret_cast<const uint8_t*>(a.scale) + (row >> 7) * a.lds * SES;
        rp.z[s] = nullptr;
        rp.zsh[s] = 0;
      }
    }
  }

  // ---- weight loads ------------------------------------------------------
  static __device__ __forceinline__ void load_w(const GemmArgs& a, WRegs<WT, S>& r, const RowPtrs<S>& rp, int c,
                                                int h) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if constexpr (WT == W_INT4) {
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(rp.w[s]);
        const int w0 = c * 16 + 4 * h;
        if constexpr (KFULL) {
          r.q[s] = *reinterpret_cast<const u32x4_t*>(wp + w0);
        } else {
          const int kw = (a.K + 7) >> 3;
          u32x4_t v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (w0 + e < kw) ? wp[w0 + e] : 0u;
          r.q[s] = v;
        }
        r.s[s] = load_scale<SDT>(rp.s[s], c);
        r.z[s] = static_cast<uint32_t>(rp.z[s][c]);
      } else {
        const uint8_t* wp = rp.w[s];
        const int b0 = c * 128 + 32 * h;
        if constexpr (KFULL) {
          r.q[s][0] = *reinterpret_cast<const u32x4_t*>(wp + b0);
          r.q[s][1] = *reinterpret_cast<const u32x4_t*>(wp + b0 + 16);
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
                const uint32_t byte = (kk < a.K) ? wp[kk] : 0u;
                word |= byte << (8 * by);
              }
              v[e] = word;
            }
            r.q[s][hh] = v;
          }
        }
        r.s[s] = load_scale<SDT>(rp.s[s], c);
      }
    }
  }

  // ---- X staging -----------------------------------------------------------
  // Thread tid handles 16-byte segments idx = tid + 256*q: row idx/16, seg idx%16.
  // KFULL: rows >= M load row M-1 (no branch); store_x never writes them.
  static __device__ __forceinline__ void load_x(const GemmArgs& a, u32x4_t (&xr)[MT], int c, int tid) {
#pragma unroll
    for (int q = 0; q < MT; ++q) {
      const int row = (tid >> 4) + 16 * q;
      const int k0 = c * 128 + (tid & 15) * 8;
      if constexpr (KFULL) {
        const int rc = row < a.M ? row : a.M - 1;
        xr[q] = *reinterpret_cast<const u32x4_t*>(a.x + rc * a.ldx + k0);
      } else {
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (row < a.M) {
          const uint16_t* xp = a.x + row * a.ldx;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t lo = (k0 + 2 * e < a.K) ? xp[k0 + 2 * e] : 0u;
            const uint32_t hi = (k0 + 2 * e + 1 < a.K) ? xp[k0 + 2 * e + 1] : 0u;
            v[e] = lo | (hi << 16);
          }
        }
        xr[q] = v;
      }
    }
  }

  static __device__ __forceinline__ void store_x(const GemmArgs& a, Smem& sm, const u32x4_t (&xr)[MT],
                                                 int b, int tid) {
#pragma unroll
    for (int q = 0; q < MT; ++q) {
      const int row = (tid >> 4) + 16 * q;
      if (16 * q >= a.M) continue;  // uniform: a 16-row block wholly past M stays zero
      const int seg = tid & 15;
      u32x4_t v = xr[q];
      const bool live = row < a.M;  // rows past M (clamped loads) must stay zero
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = live ? v[e] : 0u;
      if constexpr (WT == W_INT4) {
        // Per-row sum of the chunk (exact bf16 values, fp32 adds).
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          part += __uint_as_float(v[e] << 16) + __uint_as_float(v[e] & 0xFFFF0000u);
        part += __shfl_xor(part, 1, 16);
        part += __shfl_xor(part, 2, 16);
        part += __shfl_xor(part, 4, 16);
        part += __shfl_xor(part, 8, 16);
        if (seg == 0) sm.xsum[b][row] = part;
        // K order inside 8: (0,4),(1,5),(2,6),(3,7) to match the nibble pairs.
        u32x4_t p;
        p[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
        p[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
        p[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
        p[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
        v = p;
      }
      *reinterpret_cast<u32x4_t*>(&sm.xs[b][row][seg * 8]) = v;
    }
  }

  // ---- one unit of MFMA work -----------------------------------------------
  static __device__ __forceinline__ void compute(const Smem& sm, int b, const WRegs<WT, S>& r,
                                                 const RowPtrs<S>& rp, f32x4_t (&acc)[S][MT], int l16, int h,
                                                 uint32_t nib_mask, uint32_t magic) {
    bf16x8_t A[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        A[i][j] = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const u32x4_t*>(&sm.xs[b][16 * i + l16][32 * h + 8 * j]));
    f32x4_t X[MT];
    if constexpr (WT == W_INT4) {
#pragma unroll
      for (int i = 0; i < MT; ++i) X[i] = *reinterpret_cast<const f32x4_t*>(&sm.xsum[b][16 * i + 4 * h]);
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      bf16x8_t B[4];
      if constexpr (WT == W_INT4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = r.q[s][j];
          u32x4_t p;
          p[0] = bfi(nib_mask, w, magic);
          p[1] = bfi(nib_mask, w >> 4, magic);
          p[2] = bfi(nib_mask, w >> 8, magic);
          p[3] = bfi(nib_mask, w >> 12, magic);
          B[j] = __builtin_bit_cast(bf16x8_t, p);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t d0 = r.q[s][j >> 1][(j & 1) * 2];
          const uint32_t d1 = r.q[s][j >> 1][(j & 1) * 2 + 1];
          u32x4_t p;
          p[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
          p[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
          p[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
          p[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
          B[j] = __builtin_bit_cast(bf16x8_t, p);
        }
      }
      float negc = 0.f;
      if constexpr (WT == W_INT4) negc = -(128.0f + static_cast<float>((r.z[s] >> rp.zsh[s]) & 0xFu));
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        f32x4_t tmp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i][j], B[j], tmp, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (WT == W_INT4) {
            acc[s][i][e] = fmaf(r.s[s], fmaf(negc, X[i][e], tmp[e]), acc[s][i][e]);
          } else {
            acc[s][i][e] = fmaf(r.s[s], tmp[e], acc[s][i][e]);
          }
        }
      }
    }
  }

  // ---- tile completion ---------------------------------------------------
  // Lane (l16, h) of wave `wave` holds rows m = 16i + 4h + e, column
  // n = t*NT + (wave*S + s)*16 + l16.
  static __device__ __forceinline__ void store_tile(const GemmArgs& a, const f32x4_t (&acc)[S][MT], int t,
                                                    int wave, int l16, int h) {
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

  static constexpr int SLOT = 4 * S * MT * 4 * 64;  // floats per partial slot
  // Partial layout (bytes in a slot): the f32x4 accumulator of block
  // b = (wave*S + s)*MT + i of a lane at (b*64 + lane)*16, so every 16-byte
  // store or load covers 1 KB.
  static __device__ __forceinline__ uint32_t part_off(int wave, int s, int i, int lane) {
    return static_cast<uint32_t>((((wave * S + s) * MT + i) * 64 + lane) * 16);
  }

  static __device__ __forceinline__ uint32_t slot_off(int p, int slot) {
    return static_cast<uint32_t>((p * 2 + slot) * SLOT * 4);
  }

  static __device__ __forceinline__ void finish_tile(const GemmArgs& a, Smem& sm, f32x4_t (&acc)[S][MT], int t,
                                                     int p, int64_t u0, int64_t u1, int tid) {
    const int wave = tid >> 6, lane = tid & 63, l16 = lane & 15, h = lane >> 4;
    const int64_t ts = static_cast<int64_t>(t) * a.G, te = ts + a.G;
    if (u0 <= ts && u1 >= te) {
      store_tile(a, acc, t, wave, l16, h);
      return;
    }
    const int pf = unit_owner(ts, a.U, a.P), pl = unit_owner(te - 1, a.U, a.P);
    const auto pr = partial_rsrc(a.partials);
    const uint32_t mine = slot_off(p, partial_slot(p, t, a.G, a.U, a.P));
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) store_partial4(pr, mine + part_off(wave, s, i, lane), acc[s][i]);
    if (!arrive_last(a.counters, t, pl - pf + 1, &sm.flag)) return;
    // Sum every contributor's slot (our own included) in workgroup order.
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[s][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int q = pf; q <= pl; ++q) {
      const uint32_t base = slot_off(q, partial_slot(q, t, a.G, a.U, a.P));
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[s][i] += load_partial4(pr, base + part_off(wave, s, i, lane));
    }
    store_tile(a, acc, t, wave, l16, h);
    reset_counter(a.counters, t);
  }
};

// Stream-K steps are batches of NB consecutive K chunks of one tile (the host
// guarantees NB divides the chunk count), so every batch runs the same
// unrolled, branch-free body: each of its NB units consumes one slot of the
// register rings and refills that slot with the unit NB ahead.  Refills past
// the workgroup's range reload its last unit (an L2 hit) instead of being
// predicated, which keeps every load in the loop unconditional and counted.
template <int WT, int SDT, int MT, int S, int NB, bool KFULL>
__global__ __launch_bounds__(DEC_THREADS) void qgemm_decode_kernel(GemmArgs a) {
  using D = Decode<WT, SDT, MT, S, KFULL>;
  __shared__ typename D::Smem sm;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, l16 = lane & 15, h = lane >> 4;
  const int p = blockIdx.x;
  const int64_t b0 = unit_begin(p, a.U, a.P), b1 = unit_begin(p + 1, a.U, a.P);
  if (b0 >= b1) return;
  const int GC = a.G * NB;  // chunks per tile
  // Constants for the nibble -> bf16 insert, kept in VGPRs for v_bfi_b32.
  const uint32_t nib_mask = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t magic = opaque_and(0x43004300u, 0xFFFFFFFFu);

  // Rows M..16*MT-1 of both X buffers are zero for the whole kernel.
  for (int idx = tid; idx < 2 * D::ROWS * (XS_STRIDE / 2); idx += DEC_THREADS) {
    const int b = idx / (D::ROWS * (XS_STRIDE / 2));
    const int rem = idx % (D::ROWS * (XS_STRIDE / 2));
    const int row = rem / (XS_STRIDE / 2), col = rem % (XS_STRIDE / 2);
    if (row >= a.M) reinterpret_cast<uint32_t*>(&sm.xs[b][row][0])[col] = 0u;
  }
  for (int idx = tid; idx < 2 * D::ROWS; idx += DEC_THREADS)
    if ((idx % D::ROWS) >= a.M) sm.xsum[idx / D::ROWS][idx % D::ROWS] = 0.f;

  // Unit cursors (tile, chunk): `cur` is the unit being computed, `ld` the
  // next unit to load.  `ld` stops at the last unit of the range.
  const int first = static_cast<int>(b0) * NB, last = static_cast<int>(b1) * NB - 1;
  Cursor cur{first / GC, first % GC};
  Cursor ld = cur;
  int ld_lin = first;
  RowPtrs<S> lrp, rp;
  D::set_rows(a, lrp, ld.t, wave, l16);
  rp = lrp;
  auto advance_ld = [&]() {
    if (ld_lin < last) {
      ++ld_lin;
      ld.advance(GC);
      if (ld.c == 0) D::set_rows(a, lrp, ld.t, wave, l16);
    }
  };

  u32x4_t xr[NB][MT];
  WRegs<WT, S> wr[NB];
#pragma unroll
  for (int r = 0; r < NB; ++r) {
    D::load_x(a, xr[r], ld.c, tid);
    D::load_w(a, wr[r], lrp, ld.c, h);
    advance_ld();
  }
  D::store_x(a, sm, xr[0], 0, tid);
  __syncthreads();

  int j = 0;  // units done
  int64_t batch = b0;
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
#pragma unroll
      for (int r = 0; r < NB; ++r, ++j) {
        const int b = j & 1;
        D::load_x(a, xr[r], ld.c, tid);  // refill slot r with unit j + NB
        D::compute(sm, b, wr[r], rp, acc, l16, h, nib_mask, magic);
        D::load_w(a, wr[r], lrp, ld.c, h);
        advance_ld();
        // X of unit j+1 (slot r+1) into the other buffer; after the range's
        // last unit this writes a buffer nobody reads.
        D::store_x(a, sm, xr[(r + 1) % NB], b ^ 1, tid);
        __syncthreads();
        cur.advance(GC);
      }
    }
    D::finish_tile(a, sm, acc, t, p, b0, b1, tid);
    if (cur.c == 0) D::set_rows(a, rp, cur.t, wave, l16);
  }
}

// Host-side launcher; returns hipError_t.
template <int WT, int SDT, int MT, int S>
static hipError_t launch_decode_t(const GemmArgs& a, bool kfull, hipStream_t stream) {
  if (a.NB == 4 && kfull)
    hipLaunchKernelGGL((qgemm_decode_kernel<WT, SDT, MT, S, 4, true>), dim3(a.P), dim3(DEC_THREADS), 0, stream, a);
  else if (a.NB == 1)
    hipLaunchKernelGGL((qgemm_decode_kernel<WT, SDT, MT, S, 1, false>), dim3(a.P), dim3(DEC_THREADS), 0, stream, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

int decode_slot_floats(int MT, int S) { return 4 * S * MT * 4 * 64; }

template <int WT, int SDT>
static hipError_t launch_decode_wt(const GemmArgs& a, int MT, int S, bool kfull, hipStream_t stream) {
#define HSQ_DEC(mt, s) \
  if (MT == mt && S == s) return launch_decode_t<WT, SDT, mt, s>(a, kfull, stream);
  HSQ_DEC(1, 1) HSQ_DEC(1, 2) HSQ_DEC(1, 4)
  HSQ_DEC(2, 1) HSQ_DEC(2, 2)
  HSQ_DEC(4, 1) HSQ_DEC(4, 2)
#undef HSQ_DEC
  return hipErrorInvalidValue;
}

// The KFULL path needs K % 128 == 0 and 16-byte aligned X and W rows, and the
// host plans it with NB = 4 chunks per stream-K step.
bool decode_kfull(int K, int xvec, int wvec) { return (K % 128 == 0) && xvec && wvec && ((K / 128) % 4 == 0); }

hipError_t launch_decode(int wt, const GemmArgs& a, int MT, int S, hipStream_t stream) {
  const bool kfull = decode_kfull(a.K, a.xvec, a.wvec);
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_decode_wt<W_INT4, SCALE_BF16>(a, MT, S, kfull, stream);
    if (a.sdt == SCALE_F16) return launch_decode_wt<W_INT4, SCALE_F16>(a, MT, S, kfull, stream);
    return launch_decode_wt<W_INT4, SCALE_F32>(a, MT, S, kfull, stream);
  }
  if (a.sdt == SCALE_BF16) return launch_decode_wt<W_FP8, SCALE_BF16>(a, MT, S, kfull, stream);
  if (a.sdt == SCALE_F16) return launch_decode_wt<W_FP8, SCALE_F16>(a, MT, S, kfull, stream);
  return launch_decode_wt<W_FP8, SCALE_F32>(a, MT, S, kfull, stream);
}

}  // namespace hsq
