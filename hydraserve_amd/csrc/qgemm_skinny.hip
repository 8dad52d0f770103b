// Decode-regime (1..64 activation rows) quantized weight GEMM for gfx950:
// register-streamed weights, X shared through LDS, 16x16x32 bf16 MFMA.
//
// Replaces the Triton launches of hydraserve/kernels/awq.py:52-74
// (_awq_gemm_kernel, awq.py:82-142) and hydraserve/kernels/fp8.py:68-96
// (_fp8_gemm_kernel, fp8.py:104-168) for activations of at most 64 rows.
//
// Work split.  A unit is (tile of BT = 16*S*NB weight rows, KC consecutive
// 128-wide K chunks).  Units are numbered tile-major and a persistent grid
// of P workgroups takes equal contiguous ranges (stream-K, qgemm_common.h).
// The NW = NB*KC wavefronts of a workgroup work on the same unit at once:
// wave w takes K phase ph = w / NB (chunk KC*c + ph of the unit) of the S
// 16-row blocks of block group bg = w % NB.  At any moment a workgroup's
// loads thus cover a few rows over KC*64 (INT4) contiguous bytes each rather
// than many rows over 64 bytes each -- HBM serves the former markedly
// faster -- and the unit's X chunks [16*MT rows x 128*KC] are staged once in
// LDS for all waves.  At the end of a tile the KC phases of each block meet
// in LDS.
//
// Weights never pass through LDS.  Lane (l16, h) of a wave loads, for each
// of its row blocks, the 16 bytes (INT4; FP8: 32) at byte 16h (32h) of row
// l16's 64-byte (128-byte) chunk: one load instruction covers 16 rows x 64
// contiguous bytes.  Those registers are the MFMA A operand: step j takes the
// lane's K offsets 32h + 8j .. +8, and the B operand (X) is read from LDS at
// the same offsets.  A ring of R units of such loads stays in flight per
// wave, with the unit's staging loads (X, scales, zero points) beside them.
//
// INT4 arithmetic (group rewrite).  A nibble q becomes the bf16 128+q with
// one v_and_or_b32 per two nibbles; the MFMA computes, per row n and X row
// m, T = sum_k x[m,k] * (128 + q[n,k]) over one chunk (= one quantization
// group) in fp32, and the unit adds s[n] * (T - (128 + z[n]) * Xg[m]) to the
// accumulator, Xg[m] being the fp32 sum of the chunk's X values.  This is
// the reference's sum_k x * ((q - z) * s) without rounding each dequantized
// weight to bf16 first (hydraserve/kernels/awq.py:136-137 rounds it).
// FP8: E4M3FN -> bf16 is exact; the unit adds s * T with s the 128x128
// block's scale.
//
// Per unit, in this order: (1) the staging of unit u+1 (loaded R-1 units
// earlier into registers) goes into LDS buffer (u+1)&1, (2) unit u is
// computed from buffer u&1, (3) the weight slot and staging set of unit u are
// refilled with unit u+R's loads, (4) one workgroup barrier.
#include <type_traits>

#include "qgemm_ops.h"

namespace hsq {

template <int I, int N, typename F>
__device__ __forceinline__ void static_for_impl(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_impl<I + 1, N>(f);
  }
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<0, N>(f);
}

// Scale entries (unit, phase, row) one workgroup may stage: its range holds
// at most kSkinnyMaxEntries / (BT * KC) units (the host raises the grid to
// stay below).
constexpr int kSkinnyMaxEntries = 6144;

template <int WT, int SDT, int MT, int S, int NB, int KC, int R, bool XD>
struct Skinny {
  static constexpr int NW = NB * KC;
  static constexpr int THREADS = 64 * NW;
  static constexpr int BT = 16 * S * NB;   // weight rows per tile
  static constexpr int MR = 16 * MT;       // X rows staged per unit
  static constexpr int LPB = WT == W_INT4 ? 1 : 2;    // 16-byte weight loads per row block per chunk
  static constexpr int CB = WT == W_INT4 ? 64 : 128;  // weight bytes per row per chunk
  static constexpr int XROW = 272;                    // LDS bytes per staged X row (256 + 16 of padding)
  static constexpr int XPIECES = MR * 16 * KC;        // 16-byte X pieces per unit
  static constexpr int XP = (XPIECES + THREADS - 1) / THREADS;
  static constexpr int SLOT = BT * MR;                // floats of one partial tile
  // Scales of every unit of the workgroup's range are staged once, at the
  // start: INT4 one per (unit, phase, row), FP8 one per (unit, phase).
  static constexpr int SROW = WT == W_INT4 ? BT : 1;
  static constexpr int UMAX = kSkinnyMaxEntries / (BT * KC);
  // Row-major [row][unit*KC + phase] with an odd row stride: the staging
  // writes (consecutive lanes: consecutive groups of one row) and the
  // per-unit reads (four rows, one group) both spread over the banks.
  static constexpr int SPW = UMAX * KC + 1;

  struct Smem {
    __attribute__((aligned(16))) uint8_t x[XD ? 1 : 2][KC][XD ? 16 : MR * XROW];
    __attribute__((aligned(16))) f32x4_t red[KC > 1 ? KC - 1 : 1][NB][S][MT][64];
    __attribute__((aligned(16))) float sc[SROW][SPW];                        // scales
    __attribute__((aligned(16))) float nz[WT == W_INT4 ? SROW : 1][SPW];  // -(128 + zero point)
    int flag;
  };

  struct Stage {
    u32x4_t xv[XD ? 1 : XP];
  };
};

template <int WT, int SDT, int MT, int S, int NB, int KC, int R, bool XD>
__global__ __launch_bounds__(64 * NB * KC) void qgemm_skinny_kernel(GemmArgs a) {
  using D = Skinny<WT, SDT, MT, S, NB, KC, R, XD>;
  __shared__ typename D::Smem sm;
  const int tid = threadIdx.x;
  const int lane = tid & 63, l16 = lane & 15, h = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bg = wave % NB, ph = wave / NB;
  const int p = blockIdx.x;
  const int64_t u0 = unit_begin(p, a.U, a.P), u1 = unit_begin(p + 1, a.U, a.P);
  if (u0 >= u1) return;
  const int G = a.G;  // units per tile
  const int M = a.M, N = a.N;
  const int rb = static_cast<int>(WT == W_INT4 ? a.ldw * 4 : a.ldw);  // bytes per weight row
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(a.w, static_cast<int64_t>(N - 1) * rb + (WT == W_INT4 ? a.K / 2 : a.K));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (static_cast<int64_t>(M - 1) * a.ldx + a.K) * 2);
  constexpr int SES = SDT == SCALE_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t rsc =
      make_rsrc(a.scale, (static_cast<int64_t>(WT == W_INT4 ? N - 1 : (N - 1) >> 7) * a.lds + a.K / 128) * SES);
  const __amdgpu_buffer_rsrc_t rzp =
      make_rsrc(WT == W_INT4 ? static_cast<const void*>(a.zero) : a.scale,
                WT == W_INT4 ? (static_cast<int64_t>((N - 1) >> 3) * a.ldz + a.K / 128) * 4 : 4);

  // ---- X staging (the unit's X chunks, rows < M only) -------------------------
  // X piece i < M*16*KC: phase i / (16M), row (i / 16) % M, 16-byte segment
  // i % 16.  Lanes without a piece load from past the buffer's end (a buffer
  // load returns zero there without a memory access), so every wave issues
  // the same loads.  Staged rows >= M are never written: they only feed
  // output columns that are never stored.
  const int xpieces = M * 16 * KC;
  uint32_t xoff[D::XP];
  int xdst[D::XP];  // LDS byte offset of the piece inside a buffer, or -1
#pragma unroll
  for (int k = 0; k < D::XP; ++k) {
    const int i = tid + k * D::THREADS;
    if (i < xpieces) {
      const int q = i / (16 * M), m = (i >> 4) % M, seg = i & 15;
      xoff[k] = static_cast<uint32_t>((m * static_cast<int>(a.ldx) + 128 * q + 8 * seg) * 2);
      xdst[k] = q * D::MR * D::XROW + m * D::XROW + seg * 16;
    } else {
      xoff[k] = 0x80000000u;
      xdst[k] = -1;
    }
  }
  typename D::Stage stg[R];
  auto issue_stage = [&](typename D::Stage& st, int t, int c) __attribute__((always_inline)) {
    (void)t;
#pragma unroll
    for (int k = 0; k < D::XP; ++k)
      st.xv[k] = bload<u32x4_t>(rx, xoff[k], static_cast<uint32_t>(c) * (256u * KC));
  };
  auto commit_stage = [&](const typename D::Stage& st, int buf, int t) __attribute__((always_inline)) {
    (void)t;
#pragma unroll
    for (int k = 0; k < D::XP; ++k) {
      if (k * D::THREADS < xpieces && xdst[k] >= 0) {
        u32x4_t v = st.xv[k];
        if constexpr (WT == W_INT4) v = permute_x(v);
        *reinterpret_cast<u32x4_t*>(&sm.x[buf][0][0] + xdst[k]) = v;
      }
    }
  };

  // ---- scales and zero points of the whole range, staged once -----------------
  // Per tile segment of the range, entries (row, group) with the group
  // running fastest, so consecutive lanes read consecutive scales.
  auto stage_scales = [&]() __attribute__((always_inline)) {
    for (int64_t us = u0; us < u1;) {
      const int t = static_cast<int>(us / G), c0 = static_cast<int>(us % G);
      const int c1 = static_cast<int>(G < c0 + (u1 - us) ? G : c0 + (u1 - us));
      const int ng = (c1 - c0) * KC, g0 = c0 * KC;
      const int du0 = static_cast<int>(us - u0);
      const int total = D::SROW * ng;
      constexpr int QB = 4;
      for (int base = tid; base < total; base += QB * D::THREADS) {
        uint32_t sv[QB], zv[QB];
#pragma unroll
        for (int k = 0; k < QB; ++k) {
          int i = base + k * D::THREADS;
          i = i < total ? i : total - 1;
          const int rl = i / ng, gi = i - rl * ng;
          int row = WT == W_INT4 ? t * D::BT + rl : (t * D::BT) >> 7;
          row = row < N ? row : N - 1;
          const int64_t e = static_cast<int64_t>(WT == W_INT4 ? row : row) * a.lds + g0 + gi;
          if constexpr (SDT == SCALE_F32) sv[k] = bload<uint32_t>(rsc, static_cast<uint32_t>(e * 4), 0u);
          else sv[k] = bload<uint16_t>(rsc, static_cast<uint32_t>(e * 2), 0u);
          if constexpr (WT == W_INT4)
            zv[k] = bload<uint32_t>(rzp, static_cast<uint32_t>((static_cast<int64_t>(row >> 3) * a.ldz + g0 + gi) * 4), 0u);
        }
#pragma unroll
        for (int k = 0; k < QB; ++k) {
          const int i = base + k * D::THREADS;
          if (i < total) {
            const int rl = i / ng, gi = i - rl * ng;
            const int du = du0 + gi / KC, q = gi % KC;
            float sf;
            if constexpr (SDT == SCALE_F32) sf = __uint_as_float(sv[k]);
            else if constexpr (SDT == SCALE_BF16) sf = __uint_as_float(sv[k] << 16);
            else sf = __half2float(__ushort_as_half(static_cast<unsigned short>(sv[k])));
            sm.sc[rl][du * KC + q] = sf;
            if constexpr (WT == W_INT4) {
              const int row = t * D::BT + rl;
              sm.nz[rl][du * KC + q] = -(128.0f + static_cast<float>((zv[k] >> (4 * (row & 7))) & 0xFu));
            }
          }
        }
      }
      us += c1 - c0;
    }
  };

  // ---- weight ring ------------------------------------------------------------
  u32x4_t ring[R][S][D::LPB];
  uint32_t woff[S];
  auto set_wtile = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      int row = t * D::BT + (bg * S + s) * 16 + l16;
      row = row < N ? row : N - 1;
      woff[s] = static_cast<uint32_t>(row * rb) + static_cast<uint32_t>(16 * D::LPB * h);
    }
  };
  // X direct (XD): each wave loads its own B fragments beside its weights:
  // lane (l16, h) reads X[16mt + l16][32h .. 32h+32) of its chunk (rows past
  // M from past the buffer's end).
  constexpr int XR = XD ? R : 1;
  u32x4_t xr[XR][MT][4];
  uint32_t xdoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + l16;
    xdoff[mt] = m < M ? static_cast<uint32_t>((m * static_cast<int>(a.ldx) + 32 * h) * 2) : 0x80000000u;
  }
  auto load_unit = [&](u32x4_t (&slot)[S][D::LPB], u32x4_t (&xs)[MT][4], int c) __attribute__((always_inline)) {
    const uint32_t so = static_cast<uint32_t>((c * KC + ph) * D::CB);
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int e = 0; e < D::LPB; ++e) slot[s][e] = bload<u32x4_t>(rw, woff[s] + 16u * e, so);
    if constexpr (XD) {
      const uint32_t xs_off = static_cast<uint32_t>((c * KC + ph) * 256);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) xs[mt][j] = bload<u32x4_t>(rx, xdoff[mt] + 16u * j, xs_off);
    }
  };

  Cursor cc{static_cast<int>(u0 / G), static_cast<int>(u0 % G)};  // compute (u)
  Cursor cm = cc;                                                   // staging commit (u+1)
  Cursor cl = cc;                                                   // loads (u+R)
  const int64_t ulast = u1 - 1;

  // Prologue: staging and weight loads of units u0 .. u0+R-1 (ring slot /
  // staging set r holds unit u0+r), then unit u0's staging into LDS.
  set_wtile(cl.t);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if constexpr (!XD) issue_stage(stg[r], cl.t, cl.c);
    load_unit(ring[r], xr[XD ? r : 0], cl.c);
    if (u0 + r < ulast) {
      cl.advance(G);
      if (cl.c == 0) set_wtile(cl.t);
    }
  }
  stage_scales();
  if constexpr (!XD) commit_stage(stg[0], static_cast<int>(u0 & 1), cm.t);
  __syncthreads();

  const uint32_t nib_mask = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t magic = opaque_and(0x43004300u, 0xFFFFFFFFu);
  const uint32_t one2 = opaque_and(0x3F803F80u, 0xFFFFFFFFu);  // bf16 1.0 in both halves
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{one2, one2, one2, one2});
  f32x4_t acc[S][MT];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[s][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Tile t is done (or the range ends inside it): combine the K phases in
  // LDS, then store it or hand it over through the partial slots.
  auto finish = [&](int t) __attribute__((always_inline)) {
    if constexpr (KC > 1) {
      if (ph > 0) {
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) sm.red[ph - 1][bg][s][mt][lane] = acc[s][mt];
      }
      __syncthreads();
      if (ph == 0) {
#pragma unroll
        for (int q = 0; q < KC - 1; ++q)
#pragma unroll
          for (int s = 0; s < S; ++s)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const f32x4_t v = sm.red[q][bg][s][mt][lane];
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[s][mt][e] += v[e];
            }
      }
    }
    auto store = [&](const f32x4_t (&v)[S][MT]) __attribute__((always_inline)) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int n0 = t * D::BT + (bg * S + s) * 16 + 4 * h;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = 16 * mt + l16;
          if (m < M) {
            uint16_t* yp = a.y + static_cast<int64_t>(m) * a.ldy + n0;
            if (n0 + 3 < N && (reinterpret_cast<uintptr_t>(yp) & 7) == 0) {
              uint2 o;
              o.x = pack_bf16x2(v[s][mt][0], v[s][mt][1]);
              o.y = pack_bf16x2(v[s][mt][2], v[s][mt][3]);
              *reinterpret_cast<uint2*>(yp) = o;
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (n0 + e < N) yp[e] = to_bf16_bits(v[s][mt][e]);
            }
          }
        }
      }
    };
    const int64_t ts = static_cast<int64_t>(t) * G, te = ts + G;
    if (u0 <= ts && u1 >= te) {
      if (ph == 0) store(acc);
      return;
    }
    const int pf = unit_owner(ts, a.U, a.P), pl = unit_owner(te - 1, a.U, a.P);
    const auto pr = partial_rsrc(a.partials);
    auto poff = [&](int q, int s, int mt) __attribute__((always_inline)) {
      const int slot = partial_slot(q, t, G, a.U, a.P);
      return static_cast<uint32_t>((q * 2 + slot) * D::SLOT * 4) +
             static_cast<uint32_t>((((bg * S + s) * MT + mt) * 64 + lane) * 16);
    };
    if (ph == 0) {
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) store_partial4(pr, poff(p, s, mt), acc[s][mt]);
    }
    if (arrive_last(a.counters, t, pl - pf + 1, &sm.flag)) {
      if (ph == 0) {
        // Sum every contributor's slot (ours included) in workgroup order,
        // four contributors' loads in flight at a time.
        constexpr int QB = 4;
        f32x4_t sum[S][MT];
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) sum[s][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        for (int q0 = pf; q0 <= pl; q0 += QB) {
          f32x4_t v[QB][S][MT];
#pragma unroll
          for (int i = 0; i < QB; ++i) {
            const int q = q0 + i <= pl ? q0 + i : pl;
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) v[i][s][mt] = load_partial4(pr, poff(q, s, mt));
          }
#pragma unroll
          for (int i = 0; i < QB; ++i)
            if (q0 + i <= pl) {
#pragma unroll
              for (int s = 0; s < S; ++s)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                  for (int e = 0; e < 4; ++e) sum[s][mt][e] += v[i][s][mt][e];
            }
        }
        store(sum);
      }
      reset_counter(a.counters, t);
    }
  };

  // One unit of work; r (= (u - u0) mod R) is the ring slot / staging set.
  auto unit = [&](auto rc, int64_t u) __attribute__((always_inline)) {
    constexpr int r = decltype(rc)::value;
    const int buf = static_cast<int>(u & 1);
    // (1) unit u+1's staging (set r+1) into the other buffer.
    if constexpr (!XD) {
      if (u + 1 <= ulast) {
        cm.advance(G);
        commit_stage(stg[(r + 1) % R], buf ^ 1, cm.t);
      }
    }
    // (2) compute unit u: this wave's chunk KC*c + ph of its S row blocks.
    const uint8_t* xb = &sm.x[XD ? 0 : buf][ph][0];
    f32x4_t T[S][MT];
    f32x4_t Tg[MT];  // INT4: the chunk's X sums, via MFMA with an all-ones A
    bf16x8_t wq[S][2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x8_t xf[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (XD) {
          u32x4_t v = xr[r][mt][j];
          if constexpr (WT == W_INT4) v = permute_x(v);
          xf[mt] = __builtin_bit_cast(bf16x8_t, v);
        } else {
          xf[mt] = __builtin_bit_cast(
              bf16x8_t, *reinterpret_cast<const u32x4_t*>(xb + (16 * mt + l16) * D::XROW + (4 * h + j) * 16));
        }
        if constexpr (WT == W_INT4)
          Tg[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, xf[mt], j == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f}
                                                                                 : Tg[mt], 0, 0, 0);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        bf16x8_t wf;
        if constexpr (WT == W_INT4) {
          if ((j & 1) == 0) int4_operand2(ring[r][s][0][j], ring[r][s][0][j + 1], nib_mask, magic, wq[s][0], wq[s][1]);
          wf = wq[s][j & 1];
        } else {
          wf = fp8_operand(ring[r][s][j >> 1][(j & 1) * 2], ring[r][s][j >> 1][(j & 1) * 2 + 1]);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          T[s][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xf[mt], j == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f}
                                                                                : T[s][mt], 0, 0, 0);
      }
    }
    // (3) every word of slot r has been unpacked and staging set r was
    // committed one unit ago: refill both with unit u+R (past the range end:
    // the last unit again, so that every unit issues the same loads).
    if constexpr (!XD) issue_stage(stg[r], cl.t, cl.c);
    load_unit(ring[r], xr[XD ? r : 0], cl.c);
    if (u + R < ulast) {
      cl.advance(G);
      if (cl.c == 0) set_wtile(cl.t);
    }
    const int du = static_cast<int>(u - u0);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int rl = (bg * S + s) * 16 + 4 * h;
      f32x4_t sc;
      if constexpr (WT == W_FP8) {
        const float s0 = sm.sc[0][du * KC + ph];
        sc = f32x4_t{s0, s0, s0, s0};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[e] = sm.sc[rl + e][du * KC + ph];
      }
      if constexpr (WT == W_INT4) {
        f32x4_t nz;
#pragma unroll
        for (int e = 0; e < 4; ++e) nz[e] = sm.nz[rl + e][du * KC + ph];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[s][mt][e] = fmaf(sc[e], fmaf(nz[e], Tg[mt][e], T[s][mt][e]), acc[s][mt][e]);
        }
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[s][mt][e] = fmaf(sc[e], T[s][mt][e], acc[s][mt][e]);
      }
    }
    if (cc.c == G - 1 || u == ulast) {
      finish(cc.t);
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[s][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    cc.advance(G);
    // (4) buffer u&1 is free once every wave is past here.
    if constexpr (!XD) __syncthreads();
  };

  // Whole groups of R units in a loop whose every iteration issues the same
  // loads (so the compiler's wait counts stay exact across the back edge),
  // then the remaining units.
  int64_t ub = u0;
  for (; ub + (R - 1) <= ulast; ub += R)
    static_for<R>([&](auto rc) __attribute__((always_inline)) { unit(rc, ub + decltype(rc)::value); });
  static_for<R - 1>([&](auto rc) __attribute__((always_inline)) {
    if (ub + decltype(rc)::value <= ulast) unit(rc, ub + decltype(rc)::value);
  });
}

constexpr size_t kSkinnyLdsLimit = 160 * 1024;

template <int WT, int SDT, int MT, int S, int NB, int KC, int R, bool XD>
static hipError_t launch_skinny_t(const GemmArgs& a, hipStream_t stream) {
  if constexpr (sizeof(typename Skinny<WT, SDT, MT, S, NB, KC, R, XD>::Smem) > kSkinnyLdsLimit) {
    return hipErrorInvalidValue;  // skinny_fits() keeps the host from choosing this
  } else {
    hipLaunchKernelGGL((qgemm_skinny_kernel<WT, SDT, MT, S, NB, KC, R, XD>), dim3(a.P), dim3(64 * NB * KC), 0,
                       stream, a);
    return hipGetLastError();
  }
}

// Host mirror of the LDS footprint (Skinny::Smem, 16-byte aligned parts).
bool skinny_fits(int wt, int m, int s, int nb, int kc, bool xd) {
  const size_t mt = (m + 15) / 16, bt = 16 * s * nb;
  const size_t x = xd ? 16 * kc : 2 * kc * 16 * mt * 272;
  const size_t red = (kc > 1 ? kc - 1 : 1) * nb * s * mt * 1024;
  const size_t umax = kSkinnyMaxEntries / (bt * kc);
  const size_t srow = wt == W_INT4 ? bt : 1;
  const size_t sc = ((umax * kc + 1) * srow * 4 + 15) / 16 * 16;
  const size_t total = x + red + sc * (wt == W_INT4 ? 2 : 1) + 16;
  return total <= kSkinnyLdsLimit;
}

int skinny_slot_floats(int mt, int s, int nb) { return 16 * s * nb * 16 * mt; }
int skinny_bt(int s, int nb) { return 16 * s * nb; }
int skinny_max_units(int s, int nb, int kc) { return kSkinnyMaxEntries / (16 * s * nb * kc); }

bool skinny_ok(const GemmArgs& a, int wt, int kc) {
  if (a.M < 1 || a.M > 64 || a.N <= 0 || a.K <= 0 || a.K % (128 * kc) != 0 || !a.xvec || !a.wvec) return false;
  const int64_t lim = int64_t(1) << 31;
  const int64_t rb = wt == W_INT4 ? a.ldw * 4 : a.ldw;
  if (static_cast<int64_t>(a.N) * rb >= lim) return false;
  if ((static_cast<int64_t>(a.M) * a.ldx + a.K) * 2 >= lim) return false;
  const int64_t ses = a.sdt == SCALE_F32 ? 4 : 2;
  if ((static_cast<int64_t>(a.N) * a.lds + a.K / 128) * ses >= lim) return false;
  if (wt == W_INT4 && (static_cast<int64_t>(a.N / 8 + 1) * a.ldz + a.K / 128) * 4 >= lim) return false;
  return true;
}

template <int WT, int SDT, int S, int NB, int KC>
static hipError_t launch_skinny_m(const GemmArgs& a, bool xd, hipStream_t stream) {
  const int mt = (a.M + 15) / 16;
  if (mt == 1 && xd) return launch_skinny_t<WT, SDT, 1, S, NB, KC, 4, true>(a, stream);
  if (mt == 1) return launch_skinny_t<WT, SDT, 1, S, NB, KC, 4, false>(a, stream);
  if (mt == 2) return launch_skinny_t<WT, SDT, 2, S, NB, KC, 4, false>(a, stream);
  if constexpr (S == 1) {
    if (mt == 3) return launch_skinny_t<WT, SDT, 3, S, NB, KC, 4, false>(a, stream);
    if constexpr (KC < 4) return launch_skinny_t<WT, SDT, 4, S, NB, KC, 4, false>(a, stream);
  }
  return hipErrorInvalidValue;  // four K phases of 64 X rows do not fit LDS
}

template <int WT, int SDT>
static hipError_t launch_skinny_s(const GemmArgs& a, int s, int nb, int kc, bool xd, hipStream_t stream) {
  if (s == 1 && nb == 2 && kc == 4) return launch_skinny_m<WT, SDT, 1, 2, 4>(a, xd, stream);
  if (s == 1 && nb == 4 && kc == 2) return launch_skinny_m<WT, SDT, 1, 4, 2>(a, xd, stream);
  if (s == 1 && nb == 8 && kc == 1) return launch_skinny_m<WT, SDT, 1, 8, 1>(a, xd, stream);
  if (a.M <= 32) {
    if (s == 2 && nb == 2 && kc == 4) return launch_skinny_m<WT, SDT, 2, 2, 4>(a, xd, stream);
    if (s == 2 && nb == 4 && kc == 2) return launch_skinny_m<WT, SDT, 2, 4, 2>(a, xd, stream);
    if (s == 2 && nb == 1 && kc == 8) return launch_skinny_m<WT, SDT, 2, 1, 8>(a, xd, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_skinny(int wt, const GemmArgs& a, int s, int nb, int kc, bool xd, hipStream_t stream) {
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_skinny_s<W_INT4, SCALE_BF16>(a, s, nb, kc, xd, stream);
    if (a.sdt == SCALE_F16) return launch_skinny_s<W_INT4, SCALE_F16>(a, s, nb, kc, xd, stream);
    return launch_skinny_s<W_INT4, SCALE_F32>(a, s, nb, kc, xd, stream);
  }
  if (a.sdt == SCALE_BF16) return launch_skinny_s<W_FP8, SCALE_BF16>(a, s, nb, kc, xd, stream);
  if (a.sdt == SCALE_F16) return launch_skinny_s<W_FP8, SCALE_F16>(a, s, nb, kc, xd, stream);
  return launch_skinny_s<W_FP8, SCALE_F32>(a, s, nb, kc, xd, stream);
}

}  // namespace hsq
