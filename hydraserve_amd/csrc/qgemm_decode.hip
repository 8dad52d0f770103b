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
// strip-chunk = 16 rows x 128 B), a few units ahead of use.
//
// Arithmetic.  Weights are decoded in registers and fed to
// v_mfma_f32_16x16x32_bf16 with X padded to 16*MT rows.  The K order inside a
// chunk is permuted identically for X and W (any common permutation leaves the
// dot product unchanged), which lets every lane take one 16-byte run of a
// weight row.
//
//   INT4: a nibble q is turned into the bf16 value 128+q by OR-ing it into the
//   mantissa of 128.0 (0x4300), two nibbles per instruction.  For each group the
//   MFMA yields T = sum_k x_k (128 + q_k); the true group sum is
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
#include "qgemm_common.h"

namespace hsq {

constexpr int DEC_THREADS = 256;
constexpr int XS_STRIDE = 136;  // bf16 per LDS row: 128 + 8 pad (bank spread)

template <int WT, int S>
struct WRegs;

template <int S>
struct WRegs<W_INT4, S> {
  u32x4_t q[S];
  float s[S];
  float negc[S];  // -(128 + z)
};

template <int S>
struct WRegs<W_FP8, S> {
  u32x4_t q[S][2];
  float s[S];
};

template <int WT, int SDT, int MT, int S>
struct Decode {
  static constexpr int NT = 64 * S;
  static constexpr int ROWS = 16 * MT;

  struct Smem {
    __attribute__((aligned(16))) uint16_t xs[2][ROWS][XS_STRIDE];
    __attribute__((aligned(16))) float xsum[2][ROWS];
    int flag;
  };

  // ---- weight loads ------------------------------------------------------
  static __device__ __forceinline__ void load_w(const GemmArgs& a, WRegs<WT, S>& r, int t, int c,
                                                int wave, int l16, int h) {
    // `full` is uniform: the whole chunk is inside K and rows allow 16-byte loads.
    const int kw = (a.K + 7) >> 3;  // INT4 words per row
    const bool full = a.wvec && (WT == W_INT4 ? (c + 1) * 16 <= kw : (c + 1) * 128 <= a.K);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      int row = t * NT + (wave * S + s) * 16 + l16;
      row = row < a.N ? row : a.N - 1;
      if constexpr (WT == W_INT4) {
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(a.w) + row * a.ldw;
        const int w0 = c * 16 + 4 * h;
        if (full) {
          r.q[s] = *reinterpret_cast<const u32x4_t*>(wp + w0);
        } else {
          u32x4_t v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (w0 + e < kw) ? wp[w0 + e] : 0u;
          r.q[s] = v;
        }
        r.s[s] = load_scale<SDT>(a.scale, row * a.lds + c);
        const uint32_t zw = static_cast<uint32_t>(a.zero[(row >> 3) * a.ldz + c]);
        r.negc[s] = -(128.0f + static_cast<float>((zw >> ((row & 7) * 4)) & 0xFu));
      } else {
        const uint8_t* wp = reinterpret_cast<const uint8_t*>(a.w) + row * a.ldw;
        const int b0 = c * 128 + 32 * h;
        if (full) {
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
        r.s[s] = load_scale<SDT>(a.scale, (row >> 7) * a.lds + c);
      }
    }
  }

  // ---- X staging -----------------------------------------------------------
  // Thread tid handles 16-byte segments idx = tid + 256*q: row idx/16, seg idx%16.
  static __device__ __forceinline__ void load_x(const GemmArgs& a, u32x4_t (&xr)[MT], int c, int tid) {
    const bool full = a.xvec && (c + 1) * 128 <= a.K;  // uniform
#pragma unroll
    for (int q = 0; q < MT; ++q) {
      const int row = (tid >> 4) + 16 * q;
      const int k0 = c * 128 + (tid & 15) * 8;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (row < a.M) {
        const uint16_t* xp = a.x + row * a.ldx;
        if (full) {
          v = *reinterpret_cast<const u32x4_t*>(xp + k0);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t lo = (k0 + 2 * e < a.K) ? xp[k0 + 2 * e] : 0u;
            const uint32_t hi = (k0 + 2 * e + 1 < a.K) ? xp[k0 + 2 * e + 1] : 0u;
            v[e] = lo | (hi << 16);
          }
        }
      }
      xr[q] = v;
    }
  }

  static __device__ __forceinline__ void store_x(const GemmArgs& a, Smem& sm, const u32x4_t (&xr)[MT],
                                                 int b, int tid) {
#pragma unroll
    for (int q = 0; q < MT; ++q) {
      const int row = (tid >> 4) + 16 * q;
      if (row >= a.M) continue;  // rows >= M stay zero (set once)
      const int seg = tid & 15;
      u32x4_t v = xr[q];
      if constexpr (WT == W_INT4) {
        // Per-row sum of the chunk (exact bf16 values, fp32 adds).
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          part += bf16_to_f32(v[e] & 0xFFFFu) + bf16_to_f32(v[e] >> 16);
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
                                                 f32x4_t (&acc)[S][MT], int l16, int h) {
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
          p[0] = (w & 0x000F000Fu) | 0x43004300u;
          p[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
          p[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
          p[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
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
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        f32x4_t tmp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i][j], B[j], tmp, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (WT == W_INT4) {
            acc[s][i][e] = fmaf(r.s[s], fmaf(r.negc[s], X[i][e], tmp[e]), acc[s][i][e]);
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
  // Partial layout: f32x4 at ((wave*S + s)*MT + i)*64 + lane (16 B per lane).
  static __device__ __forceinline__ int64_t part_off(int wave, int s, int i, int lane) {
    return ((static_cast<int64_t>(wave * S + s) * MT + i) * 64 + lane) * 4;
  }

  static __device__ __forceinline__ float* slot_ptr(const GemmArgs& a, int p, int slot) {
    return a.partials + (static_cast<int64_t>(p) * 2 + slot) * SLOT;
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
    float* mine = slot_ptr(a, p, partial_slot(p, t, a.G, a.U, a.P));
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) store_partial(mine + part_off(wave, s, i, lane) + e, acc[s][i][e]);
    if (!arrive_last(a.counters, t, pl - pf + 1, &sm.flag)) return;
    // Sum every contributor's slot (our own included) in workgroup order.
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

template <int WT, int SDT, int MT, int S, int NBUF>
__global__ __launch_bounds__(DEC_THREADS) void qgemm_decode_kernel(GemmArgs a) {
  using D = Decode<WT, SDT, MT, S>;
  __shared__ typename D::Smem sm;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, l16 = lane & 15, h = lane >> 4;
  const int p = blockIdx.x;
  const int64_t u0 = unit_begin(p, a.U, a.P), u1 = unit_begin(p + 1, a.U, a.P);
  if (u0 >= u1) return;

  // Rows M..16*MT-1 of both X buffers are zero for the whole kernel.
  for (int idx = tid; idx < 2 * D::ROWS * (XS_STRIDE / 2); idx += DEC_THREADS) {
    const int b = idx / (D::ROWS * (XS_STRIDE / 2));
    const int rem = idx % (D::ROWS * (XS_STRIDE / 2));
    const int row = rem / (XS_STRIDE / 2), col = rem % (XS_STRIDE / 2);
    if (row >= a.M) reinterpret_cast<uint32_t*>(&sm.xs[b][row][0])[col] = 0u;
  }
  for (int idx = tid; idx < 2 * D::ROWS; idx += DEC_THREADS)
    if ((idx % D::ROWS) >= a.M) sm.xsum[idx / D::ROWS][idx % D::ROWS] = 0.f;

  const int n_units = static_cast<int>(u1 - u0);
  Cursor cur{static_cast<int>(u0 / a.G), static_cast<int>(u0 % a.G)};
  Cursor ld = cur;  // next unit whose weights are to be loaded
  u32x4_t xr[MT];
  D::load_x(a, xr, cur.c, tid);
  WRegs<WT, S> wr[NBUF];
#pragma unroll
  for (int r = 0; r < NBUF; ++r)
    if (r < n_units) {
      D::load_w(a, wr[r], ld.t, ld.c, wave, l16, h);
      ld.advance(a.G);
    }
  D::store_x(a, sm, xr, 0, tid);
  __syncthreads();

  f32x4_t acc[S][MT];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[s][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int jb = 0; jb < n_units; jb += NBUF) {
#pragma unroll
    for (int r = 0; r < NBUF; ++r) {
      const int j = jb + r;
      if (j < n_units) {
        const int b = j & 1;
        const bool more = j + 1 < n_units;
        Cursor nxt = cur;
        nxt.advance(a.G);
        if (more) D::load_x(a, xr, nxt.c, tid);
        D::compute(sm, b, wr[r], acc, l16, h);
        if (j + NBUF < n_units) {
          D::load_w(a, wr[r], ld.t, ld.c, wave, l16, h);
          ld.advance(a.G);
        }
        if (cur.c == a.G - 1 || !more) {
          D::finish_tile(a, sm, acc, cur.t, p, u0, u1, tid);
#pragma unroll
          for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < MT; ++i) acc[s][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        if (more) D::store_x(a, sm, xr, b ^ 1, tid);
        __syncthreads();
        cur = nxt;
      }
    }
  }
}

// Host-side launcher; returns hipError_t.
template <int WT, int SDT, int MT, int S>
static hipError_t launch_decode_t(const GemmArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((qgemm_decode_kernel<WT, SDT, MT, S, 3>), dim3(a.P), dim3(DEC_THREADS), 0, stream, a);
  return hipGetLastError();
}

int decode_slot_floats(int MT, int S) { return 4 * S * MT * 4 * 64; }

template <int WT, int SDT>
static hipError_t launch_decode_wt(const GemmArgs& a, int MT, int S, hipStream_t stream) {
#define HSQ_DEC(mt, s) \
  if (MT == mt && S == s) return launch_decode_t<WT, SDT, mt, s>(a, stream);
  HSQ_DEC(1, 1) HSQ_DEC(1, 2) HSQ_DEC(1, 4)
  HSQ_DEC(2, 1) HSQ_DEC(2, 2)
  HSQ_DEC(4, 1) HSQ_DEC(4, 2)
#undef HSQ_DEC
  return hipErrorInvalidValue;
}

hipError_t launch_decode(int wt, const GemmArgs& a, int MT, int S, hipStream_t stream) {
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_decode_wt<W_INT4, SCALE_BF16>(a, MT, S, stream);
    if (a.sdt == SCALE_F16) return launch_decode_wt<W_INT4, SCALE_F16>(a, MT, S, stream);
    return launch_decode_wt<W_INT4, SCALE_F32>(a, MT, S, stream);
  }
  if (a.sdt == SCALE_BF16) return launch_decode_wt<W_FP8, SCALE_BF16>(a, MT, S, stream);
  if (a.sdt == SCALE_F16) return launch_decode_wt<W_FP8, SCALE_F16>(a, MT, S, stream);
  return launch_decode_wt<W_FP8, SCALE_F32>(a, MT, S, stream);
}

}  // namespace hsq
