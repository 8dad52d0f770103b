// Decode-regime (17..128 activation rows) quantized weight GEMM for gfx950:
// an LDS-DMA streamer feeding 32x32 MFMA tiles.
//
// Replaces the Triton launches of hydraserve/kernels/awq.py:52-74
// (_awq_gemm_kernel, awq.py:82-142) and hydraserve/kernels/fp8.py:68-96
// (_fp8_gemm_kernel, fp8.py:104-168) for activations of 17..128 rows, where
// the weight stream is still the roofline but every weight feeds 32-64
// output rows.
//
//   * A workgroup (NW = 4 wavefronts) owns a BM x BN output tile,
//     BM = 32*BMI rows (all of M), BN = 32*NJ*NW weight rows; wave w owns
//     weight rows [32*NJ*w, +32*NJ): BMI x NJ blocks of 32x32 fp32
//     accumulators.  (8 waves of one column block each -- two per SIMD --
//     measured no faster: per unit, each SIMD's VALU and MFMA work is the
//     same either way.)
//   * K advances 64 per unit; units are scheduled stream-K over a persistent
//     grid.  Everything a unit needs -- the X tile [BM x 64] (shared by the
//     four waves), each wave's packed weights, scales and (INT4) zero-point
//     words -- goes from global memory straight into a ring of D unit slots
//     in LDS (buffer_load ... lds), D-1 units ahead of the MFMAs, with no
//     staging registers.  The stream runs on across tile boundaries inside
//     the workgroup's range.  The only memory instructions in the loop are
//     these loads, so "unit k+1 has landed" is an exact vmcnt count, and
//     ~(D-2) units (~64 KB per CU) stay in flight.
//   * Weights, scales and zero points in a slot are private to the wave that
//     loaded them; only X needs the one workgroup barrier per unit, placed
//     before the last K16 step so that the next unit's first A fragments are
//     read during it.
//   * Dequantisation and K permutation are those of the 256x256-tile prefill
//     kernel: bf16_rne((q - z) * s) exactly (INT4, via v_fma_mix_f32 on
//     0x6400|q), bf16_rne(fp32(e4m3) * s) (FP8), and lane half h of step t
//     takes K offsets 32h + 8t .. +8 of the unit.
//
// LDS slot layout (bytes): X [BM rows x 128] with 16-byte K segment g of row
// r at slot g ^ ((r >> 1) & 7); then per wave its weights [32*NJ rows x RB]
// (INT4 RB = 32: 16-byte half h of row r at h ^ ((r >> 3) & 1); FP8 RB = 64:
// 16-byte chunk s at s ^ ((r >> 2) & 3)), so that the 16-byte reads of 16
// consecutive rows are conflict-free; then per wave 64 scale dwords and (INT4)
// 64 zero-point dwords.

#include "qgemm_common.h"
#include "qgemm_ops.h"

namespace hsq {

constexpr int MID_D = 6;  // ring depth (units)

template <int WT, int SDT, int BMI, int NJ, int NW>
struct Mid {
  static_assert((4 * BMI) % NW == 0, "every wave issues the same number of X loads");
  static constexpr int D = MID_D;
  static constexpr int THREADS = 64 * NW;
  static constexpr int BM = 32 * BMI;
  static constexpr int BN = 32 * NJ * NW;
  static constexpr int RB = WT == W_INT4 ? 32 : 64;  // weight bytes per row per unit
  static constexpr int RW = WT == W_INT4 ? 1 : 2;    // 16-byte reads per row per unit
  static constexpr int XB = BM * 128;
  static constexpr int WBW = 32 * NJ * RB;  // weight bytes per wave per unit
  static constexpr int SBW = 256;           // scale bytes per wave
  static constexpr int ZBW = WT == W_INT4 ? 256 : 0;
  static constexpr int SLOTB = XB + NW * (WBW + SBW + ZBW);
  // LDS-DMA loads per wave per unit: X, weights, scales, zero points.
  static constexpr int LX = 4 * BMI / NW;
  static constexpr int LW = WBW / 1024;
  static constexpr int L = LX + LW + 1 + (WT == W_INT4 ? 1 : 0);
  static constexpr int SES = SDT == SCALE_F32 ? 4 : 2;
  static constexpr int SLOT = NW * BMI * NJ * 1024;  // floats of one partial tile

  struct Smem {
    __attribute__((aligned(1024))) uint8_t ring[D][SLOTB];
    int flag;
  };

  static __device__ __forceinline__ int woff(int wave) { return XB + wave * (WBW + SBW + ZBW); }

  struct Rsrc {
    __amdgpu_buffer_rsrc_t x, w, s, z;
  };

  // Lane-constant parts of the DMA sources.
  struct Src {
    uint32_t x[LX];   // X byte offset of the lane's 16 bytes in X load q (K offset added per unit)
    int wr[LW];       // weight row (within the wave's rows) of the lane in weight load d
    uint32_t wb[LW];  // byte offset inside that row's unit run
    int sr;           // scale row (within the wave's rows) of the lane
  };

  // Raw register copy of one unit's wave-private slot data.
  struct Raw {
    u32x4_t q[NJ][RW];
    uint32_t sd[NJ];  // scale dword (2-byte scales: the aligned dword holding it)
    uint32_t zd[NJ];  // INT4 zero-point word of row block j
    uint32_t sh[NJ];  // bit offset of the scale inside sd
  };

  static __device__ __forceinline__ void sources(const GemmArgs& a, Src& s, int wave, int lane) {
    // X load q of wave w fills tile rows 8(NW*q + w) .. +8: row r = 8(NW*q + w) + lane/8,
    // slot lane%8 = K segment (lane%8) ^ ((r >> 1) & 7).  Rows past M repeat M-1.
#pragma unroll
    for (int q = 0; q < LX; ++q) {
      const int r = 8 * (NW * q + wave) + (lane >> 3);
      const int row = r < a.M ? r : a.M - 1;
      const int seg = (lane & 7) ^ ((r >> 1) & 7);
      s.x[q] = static_cast<uint32_t>((row * a.ldx + seg * 8) * 2);
    }
#pragma unroll
    for (int d = 0; d < LW; ++d) {
      if constexpr (WT == W_INT4) {
        // 32 rows of 32 bytes: lane -> row 32d + lane/2, half (lane&1) ^ ((row>>3)&1)
        const int lr = 32 * d + (lane >> 1);
        s.wr[d] = lr;
        s.wb[d] = 16u * static_cast<uint32_t>((lane & 1) ^ ((lr >> 3) & 1));
      } else {
        // 16 rows of 64 bytes: lane -> row 16d + lane/4, chunk (lane&3) ^ ((row>>2)&3)
        const int lr = 16 * d + (lane >> 2);
        s.wr[d] = lr;
        s.wb[d] = 16u * static_cast<uint32_t>((lane & 3) ^ ((lr >> 2) & 3));
      }
    }
    s.sr = lane & (32 * NJ - 1);
  }

  // Issue the LDS-DMA loads of unit (t, c) into the slot at byte `slot`.
  static __device__ __forceinline__ void issue(const GemmArgs& a, const Rsrc& rs, const Src& s, Smem& sm, int slot,
                                               int t, int c, int wave, int lane) {
    uint8_t* base = &sm.ring[0][0] + slot;
    const uint32_t kx = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(c) * 128u);
#pragma unroll
    for (int q = 0; q < LX; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.x, base + 1024 * (NW * q + wave), 16, s.x[q], kx, 0, 0);
    const int row0 = t * BN + wave * 32 * NJ;  // first weight row of the wave
    uint8_t* wbase = base + woff(wave);
#pragma unroll
    for (int d = 0; d < LW; ++d) {
      const uint32_t off = static_cast<uint32_t>((row0 + s.wr[d]) * a.ldw) * (WT == W_INT4 ? 4u : 1u) +
                           static_cast<uint32_t>(c) * RB + s.wb[d];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.w, wbase + 1024 * d, 16, off, 0, 0, 0);
    }
    const int g = c >> 1;
    if constexpr (WT == W_INT4) {
      const int64_t e = static_cast<int64_t>(row0 + s.sr) * a.lds + g;
      const uint32_t sb = static_cast<uint32_t>(e * SES) & ~3u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.s, wbase + WBW, 4, sb, 0, 0, 0);
      const uint32_t zb = static_cast<uint32_t>(((row0 >> 3) + (lane & (4 * NJ - 1))) * a.ldz + g) * 4u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.z, wbase + WBW + SBW, 4, zb, 0, 0, 0);
    } else {
      const int64_t e = static_cast<int64_t>(row0 >> 7) * a.lds + g;
      const uint32_t sb = static_cast<uint32_t>(e * SES) & ~3u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.s, wbase + WBW, 4, sb, 0, 0, 0);
    }
  }

  // The wave's weights, scales and zero points of unit (t, c) from the slot
  // at byte `slot` into registers.
  static __device__ __forceinline__ void read_raw(const GemmArgs& a, const Smem& sm, Raw& r, int slot, int t, int c,
                                                  int wave, int l32, int h) {
    const uint8_t* wbase = &sm.ring[0][0] + slot + woff(wave);
    const int g = c >> 1;
    const int row0 = t * BN + wave * 32 * NJ;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int lr = 32 * j + l32;
      if constexpr (WT == W_INT4) {
        r.q[j][0] = *reinterpret_cast<const u32x4_t*>(wbase + lr * 32 + 16 * (h ^ ((lr >> 3) & 1)));
        r.zd[j] = *reinterpret_cast<const uint32_t*>(wbase + WBW + SBW + (lr >> 3) * 4);
        r.sd[j] = *reinterpret_cast<const uint32_t*>(wbase + WBW + lr * 4);
        r.sh[j] = SES == 2 ? static_cast<uint32_t>(((static_cast<int64_t>(row0 + lr) * a.lds + g) & 1) * 16) : 0u;
      } else {
#pragma unroll
        for (int e = 0; e < 2; ++e)
          r.q[j][e] = *reinterpret_cast<const u32x4_t*>(wbase + lr * 64 + 16 * ((2 * h + e) ^ ((lr >> 2) & 3)));
        r.sd[j] = *reinterpret_cast<const uint32_t*>(wbase + WBW);
        r.sh[j] = SES == 2 ? static_cast<uint32_t>(((static_cast<int64_t>(row0 >> 7) * a.lds + g) & 1) * 16) : 0u;
        r.zd[j] = 0;
      }
    }
  }

  // Fragment (column block j, step t): 8 weights of the lane's row.
  // nib_mask = 0x000F000F and magic = 0x64006400 arrive as registers the
  // compiler cannot fold, so each output dword is one shift and one
  // v_and_or_b32 rather than a shift, an AND and an OR with literals.
  static __device__ __forceinline__ bf16x8_t decode(const Raw& r, int j, int t, int l32, uint32_t nib_mask,
                                                    uint32_t magic) {
    u32x4_t p;
    float s;
    if constexpr (SDT == SCALE_F32) {
      s = __uint_as_float(r.sd[j]);
    } else if constexpr (SDT == SCALE_BF16) {
      s = __uint_as_float((r.sd[j] >> r.sh[j]) << 16);
    } else {
      s = __half2float(__ushort_as_half(static_cast<unsigned short>(r.sd[j] >> r.sh[j])));
    }
    if constexpr (WT == W_INT4) {
      typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
      const float zp = static_cast<float>(1024u + ((r.zd[j] >> ((l32 & 7) * 4)) & 0xFu));
      const float c = SDT == SCALE_F32 ? zp : -(zp * s);
      const uint32_t w = r.q[j][0][t];
      float f[8];
#pragma unroll
      for (int sh = 0; sh < 4; ++sh) {
        const f16x2_t v = __builtin_bit_cast(f16x2_t, insert_nibbles(nib_mask, w >> (4 * sh), magic));
        if constexpr (SDT == SCALE_F32) {
          f[sh] = (static_cast<float>(v[0]) - c) * s;
          f[sh + 4] = (static_cast<float>(v[1]) - c) * s;
        } else {
          f[sh] = __builtin_fmaf(static_cast<float>(v[0]), s, c);
          f[sh + 4] = __builtin_fmaf(static_cast<float>(v[1]), s, c);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = pack_bf16x2(f[2 * e], f[2 * e + 1]);
    } else {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t d = r.q[j][t >> 1][(t & 1) * 2 + e];
        const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(d, false);
        const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(d, true);
        p[2 * e] = pack_bf16x2(lo[0] * s, lo[1] * s);
        p[2 * e + 1] = pack_bf16x2(hi[0] * s, hi[1] * s);
      }
    }
    return __builtin_bit_cast(bf16x8_t, p);
  }

  // A fragment of row block i, step t from the X tile of the slot at `slot`.
  static __device__ __forceinline__ bf16x8_t read_a(const Smem& sm, int slot, uint32_t aoff, int i) {
    return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(&sm.ring[0][0] + slot + aoff + 4096 * i));
  }

  // Fused SiLU-and-mul epilogue (a.silu_mul): weight rows interleave gate and
  // up in 16-row blocks, so lanes l32 < 16 of a 32-column block hold gate
  // row g = 16*(n/32) + l32 and lanes l32 + 16 the matching up row.  As in
  // the reference's unfused sequence (hydraserve/model/runtime.py:1202-1210,
  // silu_and_mul at hydraserve/kernels/activation.py:66-76), gate and up are
  // rounded to bf16 first, then out = gate * sigmoid(gate) * up in fp32,
  // rounded to bf16, into y [M, N/2].  N is a multiple of 32, so a lane and
  // its partner are in range together.
  static __device__ __forceinline__ void store_silu_mul(const GemmArgs& a, const f32x16_t& v, int n, int i,
                                                        int l32, int h) {
    const int col = (n >> 5) * 16 + (n & 15);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float own = bf16_to_f32(to_bf16_bits(v[e]));
      const float up = __shfl_xor(own, 16);
      const int m = 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
      if (l32 < 16 && m < a.M && n < a.N) {
        const float sig = 1.0f / (1.0f + expf(-own));
        a.y[m * a.ldy + col] = to_bf16_bits(own * sig * up);
      }
    }
  }

  // Lane (l32, h), register e of block (i, j): row 32i + 8(e/4) + 4h + e%4,
  // column t*BN + 32*NJ*wave + 32j + l32.
  static __device__ __forceinline__ void store_tile(const GemmArgs& a, const f32x16_t (&acc)[BMI][NJ], int t,
                                                    int wave, int l32, int h) {
    if (a.silu_mul) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < BMI; ++i) store_silu_mul(a, acc[i][j], t * BN + wave * 32 * NJ + 32 * j + l32, i, l32, h);
      return;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = t * BN + wave * 32 * NJ + 32 * j + l32;
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < BMI; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
          if (m < a.M) a.y[m * a.ldy + n] = to_bf16_bits(acc[i][j][e]);
        }
    }
  }

  // Partial layout (bytes in a slot): 16-byte chunk v (elements 4v..4v+3)
  // of accumulator block b = (wave*BMI + i)*NJ + j of a lane at
  // ((b*4 + v)*64 + lane)*16, so every 16-byte store or load covers 1 KB.
  static __device__ __forceinline__ uint32_t part_off(int b, int v, int lane) {
    return static_cast<uint32_t>(((b * 4 + v) * 64 + lane) * 16);
  }

  static __device__ __forceinline__ uint32_t slot_off(int p, int slot) {
    return static_cast<uint32_t>((p * 2 + slot) * SLOT * 4);
  }

  static __device__ __forceinline__ void finish_tile(const GemmArgs& a, Smem& sm, const f32x16_t (&acc)[BMI][NJ],
                                                     int t, int p, int64_t u0, int64_t u1, int tid) {
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
    for (int i = 0; i < BMI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          store_partial4(pr, mine + part_off((wave * BMI + i) * NJ + j, v, lane),
                         f32x4_t{acc[i][j][4 * v], acc[i][j][4 * v + 1], acc[i][j][4 * v + 2], acc[i][j][4 * v + 3]});
    if (!arrive_last(a.counters, t, pl - pf + 1, &sm.flag)) return;
    // Sum every contributor's slot (ours included) in workgroup order; all
    // of one contributor's loads are in flight before any is summed.
    f32x16_t sum[BMI][NJ];
#pragma unroll
    for (int i = 0; i < BMI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) sum[i][j] = f32x16_t{};
    for (int q = pf; q <= pl; ++q) {
      const uint32_t base = slot_off(q, partial_slot(q, t, a.G, a.U, a.P));
      f32x4_t x[BMI][NJ][4];
#pragma unroll
      for (int i = 0; i < BMI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) x[i][j][v] = load_partial4(pr, base + part_off((wave * BMI + i) * NJ + j, v, lane));
#pragma unroll
      for (int i = 0; i < BMI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int c = 0; c < 4; ++c) sum[i][j][4 * v + c] += x[i][j][v][c];
    }
    if (a.silu_mul) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < BMI; ++i) store_silu_mul(a, sum[i][j], t * BN + wave * 32 * NJ + 32 * j + l32, i, l32, h);
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int n = t * BN + wave * 32 * NJ + 32 * j + l32;
#pragma unroll
        for (int i = 0; i < BMI; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int m = 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
            if (m < a.M && n < a.N) a.y[m * a.ldy + n] = to_bf16_bits(sum[i][j][e]);
          }
      }
    }
    reset_counter(a.counters, t);
  }
};

// a.G = 64-wide K units per tile, a.T = tiles (BN weight rows each; BM >= M),
// a.U = T * G, a.P = workgroups.
template <int WT, int SDT, int BMI, int NJ, int NW>
__global__ __launch_bounds__(64 * NW, 1) void qgemm_mid_kernel(GemmArgs a) {
  using K = Mid<WT, SDT, BMI, NJ, NW>;
  constexpr int D = K::D;
  __shared__ typename K::Smem sm;
  const int tid = threadIdx.x;
  // The wave index is uniform; stating it keeps LDS-DMA bases (M0) scalar.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int p = blockIdx.x;
  const int64_t u0 = unit_begin(p, a.U, a.P), u1 = unit_begin(p + 1, a.U, a.P);
  if (u0 >= u1) return;
  const int total = static_cast<int>(u1 - u0);

  typename K::Rsrc rs;
  rs.x = make_rsrc(a.x, (static_cast<int64_t>(a.M - 1) * a.ldx + a.K) * 2);
  if constexpr (WT == W_INT4) {
    rs.w = make_rsrc(a.w, static_cast<int64_t>(a.N) * a.ldw * 4);
    rs.z = make_rsrc(a.zero, static_cast<int64_t>((a.N + 7) / 8) * a.ldz * 4);
    rs.s = make_rsrc(a.scale, ((static_cast<int64_t>(a.N - 1) * a.lds + a.K / 128) * K::SES + 3) & ~int64_t(3));
  } else {
    rs.w = make_rsrc(a.w, static_cast<int64_t>(a.N) * a.ldw);
    rs.z = rs.w;
    rs.s = make_rsrc(a.scale,
                     ((static_cast<int64_t>((a.N - 1) / 128) * a.lds + (a.K + 127) / 128) * K::SES + 3) & ~int64_t(3));
  }
  typename K::Src src;
  K::sources(a, src, wave, lane);
  uint32_t aoff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) aoff[t] = l32 * 128 + (((4 * h + t) ^ ((l32 >> 1) & 7)) * 16);
  const uint32_t nib_mask = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t magic = opaque_and(0x64006400u, 0xFFFFFFFFu);

  // DMA cursor: the next unit to load (tile dt, chunk dc), advanced without
  // divisions and held at the range's last unit once the range is exhausted
  // (those loads are harmless and never used).
  const int t_first = static_cast<int>(u0 / a.G), c_first = static_cast<int>(u0 - static_cast<int64_t>(t_first) * a.G);
  int dt = t_first, dc = c_first, di = 0;
  auto issue_next = [&](int slot_idx) __attribute__((always_inline)) {
    K::issue(a, rs, src, sm, __builtin_amdgcn_readfirstlane(slot_idx * K::SLOTB), dt, dc, wave, lane);
    if (++di < total) {
      if (++dc == a.G) {
        dc = 0;
        ++dt;
      }
    }
  };
  // Compute-side cursor of the unit after the current one (its raw data is
  // read one unit ahead), same clamping.
  int nt = t_first, nc = c_first, ni = 0;
  auto advance_next = [&]() __attribute__((always_inline)) {
    if (++ni < total) {
      if (++nc == a.G) {
        nc = 0;
        ++nt;
      }
    }
  };

  // Prologue: unit 0 alone first (every workgroup's first loads then form a
  // burst of one unit, not D-1: measured 6.5 us to the first unit otherwise),
  // then units 1 .. D-2 in flight while unit 0 is computed.
  issue_next(0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
#pragma unroll
  for (int s = 1; s < D - 1; ++s) issue_next(s);
  __syncthreads();
  typename K::Raw r0, r1;
  bf16x8_t A[BMI], B[NJ];
  K::read_raw(a, sm, r0, 0, nt, nc, wave, l32, h);
#pragma unroll
  for (int i = 0; i < BMI; ++i) A[i] = K::read_a(sm, 0, aoff[0], i);
#pragma unroll
  for (int j = 0; j < NJ; ++j) B[j] = K::decode(r0, j, 0, l32, nib_mask, magic);

  // One unit k (slot k % D): at entry A, B hold its step 0 and Rc its raw
  // data; at exit A, B hold step 0 of unit k+1 and Rn its raw data.
  int k = 0;
  auto unit = [&](typename K::Raw& Rc, typename K::Raw& Rn, f32x16_t(&acc)[BMI][NJ]) __attribute__((always_inline)) {
    const int sc = (k % D) * K::SLOTB, sn = ((k + 1) % D) * K::SLOTB;
    // Unit k+1 has landed (own loads): everything issued after it may stay in flight.
    {
      constexpr int later = (D - 3) * K::L;
      __builtin_amdgcn_s_waitcnt((later & 15) | ((later >> 4) << 14) | 0x0F70);
    }
    issue_next((k + D - 1) % D);
    advance_next();
    K::read_raw(a, sm, Rn, sn, nt, nc, wave, l32, h);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t == 3) {
        // Every wave has waited for its own loads of unit k+1 (step 0), so
        // after this barrier unit k+1's X is complete.  A bare barrier: the
        // workgroup fence of __syncthreads would also wait for every load
        // in flight.  This wave's pending LDS reads (of slot k-1's
        // successor) finish first, so no slot is overwritten under a read.
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
      }
      bf16x8_t An[BMI], Bn[NJ];
#pragma unroll
      for (int i = 0; i < BMI; ++i) An[i] = t < 3 ? K::read_a(sm, sc, aoff[t + 1], i) : K::read_a(sm, sn, aoff[0], i);
#pragma unroll
      for (int j = 0; j < NJ; ++j) Bn[j] = t < 3 ? K::decode(Rc, j, t + 1, l32, nib_mask, magic) : K::decode(Rn, j, 0, l32, nib_mask, magic);
#pragma unroll
      for (int i = 0; i < BMI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[i], B[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < BMI; ++i) A[i] = An[i];
#pragma unroll
      for (int j = 0; j < NJ; ++j) B[j] = Bn[j];
      __builtin_amdgcn_sched_barrier(0);
    }
    ++k;
  };

  int t = t_first, c = c_first;  // tile and chunk of unit k
  while (k < total) {
    const int n = (a.G - c) < (total - k) ? (a.G - c) : (total - k);
    f32x16_t acc[BMI][NJ];
#pragma unroll
    for (int i = 0; i < BMI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16_t{};
    // Units in pairs so the raw register sets alternate without copies; an
    // odd count peels one unit and swaps the sets once.
    int q = 0;
    if (n & 1) {
      unit(r0, r1, acc);
      const typename K::Raw tr = r0;
      r0 = r1;
      r1 = tr;
      q = 1;
    }
    for (; q < n; q += 2) {
      unit(r0, r1, acc);
      unit(r1, r0, acc);
    }
    K::finish_tile(a, sm, acc, t, p, u0, u1, tid);
    ++t;
    c = 0;
  }
  // Drain the clamped prefetches before the workgroup exits.
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

template <int WT, int SDT, int BMI, int NJ, int NW>
static hipError_t launch_mid_t(const GemmArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((qgemm_mid_kernel<WT, SDT, BMI, NJ, NW>), dim3(a.P), dim3(64 * NW), 0, stream, a);
  return hipGetLastError();
}

int mid_slot_floats(int bmi, int nj, int nw) { return nw * bmi * nj * 1024; }

// K a multiple of 128, 16-byte aligned rows, M <= 128, every buffer byte
// offset below 2^31.
bool mid_ok(const GemmArgs& a, int wt) {
  if (a.M <= 0 || a.M > 128 || a.N <= 0 || a.K <= 0 || a.K % 128 != 0 || !a.xvec || !a.wvec) return false;
  const int64_t lim = int64_t(1) << 31;
  const int64_t xb = (static_cast<int64_t>(a.M) * a.ldx + a.K) * 2;
  const int64_t wb = (static_cast<int64_t>(a.N) + 256) * a.ldw * (wt == W_INT4 ? 4 : 1);
  const int64_t sb = (static_cast<int64_t>(a.N) + 256) * a.lds * 4;
  const int64_t zb = (static_cast<int64_t>(a.N / 8) + 64) * a.ldz * 4;
  return xb < lim && wb < lim && sb < lim && zb < lim;
}

template <int WT, int SDT>
static hipError_t launch_mid_s(const GemmArgs& a, int bmi, int nj, int nw, hipStream_t stream) {
  if (nw != 4) return hipErrorInvalidValue;
  if (bmi == 1 && nj == 1) return launch_mid_t<WT, SDT, 1, 1, 4>(a, stream);
  if (bmi == 1 && nj == 2) return launch_mid_t<WT, SDT, 1, 2, 4>(a, stream);
  if (bmi == 2 && nj == 1) return launch_mid_t<WT, SDT, 2, 1, 4>(a, stream);
  if (bmi == 2 && nj == 2) return launch_mid_t<WT, SDT, 2, 2, 4>(a, stream);
  if (bmi == 3 && nj == 1) return launch_mid_t<WT, SDT, 3, 1, 4>(a, stream);
  if (bmi == 4 && nj == 1) return launch_mid_t<WT, SDT, 4, 1, 4>(a, stream);
  if constexpr (WT == W_INT4) {
    // FP8 weights double the slot's weight bytes: 3-4 row blocks with two
    // column blocks per wave would not fit the LDS ring.
    // (4 row blocks x 2 column blocks would spill.)
    if (bmi == 3 && nj == 2) return launch_mid_t<WT, SDT, 3, 2, 4>(a, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_mid(int wt, const GemmArgs& a, int bmi, int nj, int nw, hipStream_t stream) {
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_mid_s<W_INT4, SCALE_BF16>(a, bmi, nj, nw, stream);
    if (a.sdt == SCALE_F16) return launch_mid_s<W_INT4, SCALE_F16>(a, bmi, nj, nw, stream);
    return launch_mid_s<W_INT4, SCALE_F32>(a, bmi, nj, nw, stream);
  }
  if (a.sdt == SCALE_BF16) return launch_mid_s<W_FP8, SCALE_BF16>(a, bmi, nj, nw, stream);
  if (a.sdt == SCALE_F16) return launch_mid_s<W_FP8, SCALE_F16>(a, bmi, nj, nw, stream);
  return launch_mid_s<W_FP8, SCALE_F32>(a, bmi, nj, nw, stream);
}

}  // namespace hsq
