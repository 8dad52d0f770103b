// Prefill-regime quantized weight GEMM for gfx950: 256x256 output tiles.
//
// Replaces the Triton launches of hydraserve/kernels/awq.py:52-74
// (_awq_gemm_kernel, awq.py:82-142) and hydraserve/kernels/fp8.py:68-96
// (_fp8_gemm_kernel, fp8.py:104-168) for large M.
//
// Budget that shapes the kernel (measured on MI355X): a 32x32x16 bf16 MFMA
// issues every 32 cycles per SIMD, up to ~4 independent VALU ops co-issue with
// each one for free, and LDS serves ~100-140 B/clk per CU.  So:
//   * a workgroup (4 wavefronts) owns a 256x256 output tile; wave w owns all
//     256 rows and output columns [64w, 64w+64): 8x2 blocks of 32x32 fp32
//     accumulators (256 AGPRs).  Every weight element a wave decodes feeds 8
//     MFMA row blocks, which brings the exact dequantisation to ~2.4 VALU ops
//     per MFMA;
//   * K advances 64 per unit.  X tiles [256 x 64] go from global memory
//     straight into a ring of three LDS buffers (buffer_load ... lds, two
//     units ahead; no staging registers) and are read as A fragments by all
//     four waves: 32 KB per wave per unit, ~80 B/clk per CU at full MFMA
//     rate.  One barrier per unit, before its last K16 step, after which the
//     next unit's first A fragments are read during that step;
//   * weights stream from global memory into registers two units ahead and
//     are dequantised one K16 step ahead of their MFMAs;
//   * XCD-aware stream-K: workgroups are numbered so that the ones sharing an
//     XCD (dispatch round-robins workgroups over the 8 XCDs) take one
//     contiguous run of tiles, and tiles are numbered M-major, so an XCD's
//     workgroups share the same 256-row X slice in their L2 while all XCDs
//     sweep the weight columns in step (shared through the MALL).
//
// Dequantisation matches the reference's weight bits:
//   INT4: bf16_rne((q - z) * s) (awq.py:18-22, awq.py:136-137).  The nibble
//         is OR-ed under the exponent of 1024.0 in fp16 (0x6400 | q = 1024+q)
//         and v_fma_mix_f32 computes (1024+q)*s - (1024+z)*s, exact in fp32
//         for bf16/fp16 scales (both products have at most 22 significant
//         bits), then v_cvt_pk_bf16_f32 rounds once.  fp32 scales take
//         ((q - z) * s) rounded in fp32 first, as the reference does.
//   FP8:  bf16_rne(fp32(decode(b)) * fp32(s)) (fp8.py:144-161); E4M3FN ->
//         fp32 is exact (v_cvt_pk_f32_fp8).
// Within a unit the K order is permuted identically for X and W: lane half h
// of every MFMA step t takes K offsets 32h + 8t .. +8, so each lane reads one
// contiguous 16-byte (INT4) / 32-byte (FP8) run of its weight row per unit.
//
// Tiled weights (TL, the load-time tiled copy: rows 16t..16t+15 of 128-wide
// K chunk g at byte (g * N/16 + t) * TB, TB = 1 KiB INT4 / 2 KiB FP8): the
// same registers come from fewer cache lines per load instruction (FP8: four
// contiguous 256-byte runs instead of 32 rows x 32 bytes; INT4: 16 rows x
// 64 bytes per two tiles instead of 32 lines), and INT4 words arrive with
// their nibbles paired (position i < 4 holds K offset 2i, i + 4 holds 2i + 1).
//
// Shapes (checked on the host, wide_ok): K a multiple of 128, X and W rows
// 16-byte aligned; M and N are free (rows past the end are clamped on load
// and masked on store).

#include "qgemm_common.h"
#include "qgemm_ops.h"

namespace hsq {

constexpr int WD_THREADS = 256;

template <int WT, int SDT, bool SILU = false, bool TL = false>
struct Wide {
  static constexpr int BM = 256;
  static constexpr int BN = 256;
  static constexpr int BK = 64;
  static constexpr int MI = BM / 32;
  static constexpr int XB = BM * BK * 2;  // bytes of one X tile in LDS
  static constexpr int XR = BM * BK * 2 / (1024 * 4);  // 1 KB LDS-DMA loads per wave per unit
  static constexpr int RW = WT == W_INT4 ? 1 : 2;  // 16-byte weight loads per row per unit
  static constexpr int SLOT = 4 * MI * 2 * 16 * 64;  // floats of one partial tile

  // X ring: tile row r (128 bytes) holds its 16-byte K segment g at slot
  // g ^ ((r >> 1) & 7).  A 16-byte LDS read serves 16 lanes per pass; with
  // rows 128 bytes apart, rows r and r+1 fall in opposite halves of the 64
  // banks and the XOR gives the 8 rows of each parity 8 distinct 16-byte bank
  // groups, so the A-fragment reads of 16 consecutive rows are conflict-free.
  struct Smem {
    __attribute__((aligned(1024))) uint8_t xs[3][XB];
    int flag;
  };

  // Raw loads of one unit for the lane's two rows: weights, scale bits and
  // (INT4) zero-point words.  Nothing is derived from them until they are
  // decoded, so issuing the loads never makes the wave wait for them.
  struct Raw {
    u32x4_t q0[RW], q1[RW];
    uint32_t s0, s1, z0, z1;
  };

  static __device__ __forceinline__ void coords(const GemmArgs& a, int t, int& tm, int& tn) {
    const int tnn = a.T / a.TM;
    tm = t / tnn;
    tn = t - tm * tnn;
  }

  // Per-tile byte offsets of the lane's loads (buffer loads: SGPR resource,
  // 32-bit lane offset, uniform per-unit offset).
  struct Offs {
    uint32_t x[XR];     // X source of the lane's 16 bytes in LDS-DMA load q
    uint32_t w[2];      // weight row j at the lane's 16/32-byte run of a unit
    uint32_t s[2];      // scale row j (INT4) / scale block row (FP8)
    uint32_t z[2];      // INT4 zero-point word row of row j
    uint32_t zsh[2];    // nibble shift of row j
  };

  static __device__ __forceinline__ void offsets(const GemmArgs& a, Offs& o, int tm, int tn, int wave, int l32,
                                                 int h, int tid) {
    // Load q of wave w fills LDS rows 8(4q + w) .. +8 (1 KB, lane l at byte
    // 16 l): tile row r = 8(4q + w) + l/8, slot l%8, i.e. K segment
    // (l%8) ^ ((r >> 1) & 7).
    const int lane = tid & 63;
#pragma unroll
    for (int q = 0; q < XR; ++q) {
      const int r = 8 * (4 * q + wave) + (lane >> 3);
      int row = tm * BM + r;
      row = row < a.M ? row : a.M - 1;
      const int seg = (lane & 7) ^ ((r >> 1) & 7);
      o.x[q] = static_cast<uint32_t>((row * a.ldx + seg * 8) * 2);
    }
    constexpr int SES = SDT == SCALE_F32 ? 4 : 2;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int row = tn * BN + wave * 64 + 32 * j + l32;
      row = row < a.N ? row : a.N - 1;
      if constexpr (WT == W_INT4) {
        o.w[j] = static_cast<uint32_t>(row * a.ldw * 4 + 16 * h);
        o.s[j] = static_cast<uint32_t>(row * a.lds * SES);
        o.z[j] = static_cast<uint32_t>((row >> 3) * a.ldz * 4);
        o.zsh[j] = (row & 7) * 4;
      } else {
        o.w[j] = static_cast<uint32_t>(row * a.ldw + 32 * h);
        o.s[j] = static_cast<uint32_t>((row >> 7) * a.lds * SES);
        o.z[j] = o.zsh[j] = 0;
      }
      if constexpr (TL) {
        if constexpr (WT == W_INT4) o.w[j] = static_cast<uint32_t>((row >> 4) * 1024 + (row & 15) * 64 + 16 * h);
        else o.w[j] = static_cast<uint32_t>((row >> 4) * 2048 + 16 * (32 * h + (row & 15)));
      }
    }
  }

  struct Rsrc {
    __amdgpu_buffer_rsrc_t x, w, s, z;
  };

  static __device__ __forceinline__ void load_raw(const Rsrc& rs, const Offs& o, Raw& r, int c, uint32_t ts) {
    load_w(rs, o, r, c, ts);
    load_sz(rs, o, r, c);
  }

  // Weights of unit c into r.  Tiled: chunk c/2 starts at byte
  // (c/2) * tstride, and unit c is its half c % 2 (INT4: bytes 32.. of each
  // 64-byte tile row; FP8: the second KiB of each tile).
  static __device__ __forceinline__ void load_w(const Rsrc& rs, const Offs& o, Raw& r, int c, uint32_t tstride) {
    uint32_t sw;
    if constexpr (TL) {
      sw = static_cast<uint32_t>(c >> 1) * tstride + static_cast<uint32_t>(c & 1) * (WT == W_INT4 ? 32u : 1024u);
    } else {
      (void)tstride;
      sw = static_cast<uint32_t>(c) * (WT == W_INT4 ? 32u : 64u);
    }
    const uint32_t soff_w = __builtin_amdgcn_readfirstlane(sw);
    constexpr uint32_t kSecond = TL ? 256u : 16u;  // FP8: the lane's second 16 K
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4_t* dst = j == 0 ? r.q0 : r.q1;
      dst[0] = bload<u32x4_t>(rs.w, o.w[j], soff_w);
      if constexpr (WT == W_FP8) dst[1] = bload<u32x4_t>(rs.w, o.w[j] + kSecond, soff_w);
    }
  }

  // Scale bits and (INT4) zero-point words of unit c's group into r.
  static __device__ __forceinline__ void load_sz(const Rsrc& rs, const Offs& o, Raw& r, int c) {
    const uint32_t g = static_cast<uint32_t>(c >> 1);
    constexpr uint32_t SES = SDT == SCALE_F32 ? 4 : 2;
    const uint32_t soff_s = __builtin_amdgcn_readfirstlane(g * SES);
    const uint32_t soff_z = __builtin_amdgcn_readfirstlane(g * 4u);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t sb;
      if constexpr (SDT == SCALE_F32) {
        sb = bload<uint32_t>(rs.s, o.s[j], soff_s);
      } else {
        sb = bload<uint16_t>(rs.s, o.s[j], soff_s);
      }
      uint32_t zw = 0;
      if constexpr (WT == W_INT4) zw = bload<uint32_t>(rs.z, o.z[j], soff_z);
      if (j == 0) {
        r.s0 = sb;
        r.z0 = zw;
      } else {
        r.s1 = sb;
        r.z1 = zw;
      }
    }
  }

  // X rows [tm*BM, +BM), K [c*64, +64) into the LDS buffer at byte `buf`.
  // Rows past M repeat row M-1 (finite, never stored).
  static __device__ __forceinline__ void dma_x(const Rsrc& rs, const Offs& o, Smem& sm, int buf, int c, int wave) {
    const uint32_t soff = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(c) * 128u);
#pragma unroll
    for (int q = 0; q < XR; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.x, &sm.xs[0][0] + buf + 1024 * (4 * q + wave), 16, o.x[q], soff,
                                               0, 0);
  }

  // Fragment (row half j, step t) of the next unit: 8 weights of the lane's
  // row in K order.
  // nib_mask = 0x000F000F and magic = 0x64006400 arrive as registers the
  // compiler cannot fold: one shift and one v_and_or_b32 per output dword.
  static __device__ __forceinline__ bf16x8_t decode(const Raw& r, const uint32_t (&zsh)[2], int j, int t,
                                                    uint32_t nib_mask, uint32_t magic) {
    u32x4_t p;
    const u32x4_t* q = j == 0 ? r.q0 : r.q1;
    const uint32_t sb = j == 0 ? r.s0 : r.s1;
    float s;
    if constexpr (SDT == SCALE_F32) {
      s = __uint_as_float(sb);
    } else if constexpr (SDT == SCALE_BF16) {
      s = __uint_as_float(sb << 16);
    } else {
      s = __half2float(__ushort_as_half(static_cast<unsigned short>(sb)));
    }
    if constexpr (WT == W_INT4) {
      // 1024 + z, and the constant of fma(1024 + q, s, c): -(1024 + z) * s
      // (fp32 scales: 1024 + z itself, subtracted before the multiply).
      const float zp = static_cast<float>(1024u + (((j == 0 ? r.z0 : r.z1) >> zsh[j]) & 0xFu));
      const float c = SDT == SCALE_F32 ? zp : -(zp * s);
      typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
      const uint32_t w = q[0][t];
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
      if constexpr (TL) {
        // Paired nibbles: f[sh] is K offset 2sh, f[sh + 4] is 2sh + 1.
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = pack_bf16x2(f[e], f[e + 4]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = pack_bf16x2(f[2 * e], f[2 * e + 1]);
      }
    } else {
      (void)zsh;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t d = q[t >> 1][(t & 1) * 2 + e];
        const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(d, false);
        const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(d, true);
        p[2 * e] = pack_bf16x2(lo[0] * s, lo[1] * s);
        p[2 * e + 1] = pack_bf16x2(hi[0] * s, hi[1] * s);
      }
    }
    return __builtin_bit_cast(bf16x8_t, p);
  }

  // A fragment of row block i, step t: row 32i + l32, K segment 4h + t.
  // aoff[t] = l32*128 + ((4h + t) ^ ((l32 >> 1) & 7))*16.
  static __device__ __forceinline__ bf16x8_t read_a(const Smem& sm, int buf, uint32_t aoff, int i) {
    return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(&sm.xs[0][0] + buf + aoff + 4096 * i));
  }

  // One unit: four K16 steps of 16 MFMAs (8 row blocks x 2 column blocks)
  // on A/B fragments prepared one step ahead.  At entry A and B hold step 0
  // of this unit (X in LDS buffer bc, raw weights Rc); at exit, step 0 of the
  // next unit (bn, Rn).  Step 3 starts by waiting for every load in flight
  // (the next unit's X and weights, issued one unit ago) and the workgroup
  // barrier; then the loads of the unit after next are issued: X by LDS-DMA
  // into bd (last read before this barrier) and its weights into Rc (last
  // decoded during step 2).  SHARE: unit cnext2 is the odd half of the
  // 128-K group whose even half Rn holds (landed at that wait), so its scale
  // and zero point are copied from Rn instead of loaded again.
  template <bool SHARE>
  static __device__ __forceinline__ void unit(Smem& sm, int bc, int bn, int bd, int cnext2, bf16x8_t (&A)[MI],
                                              bf16x8_t (&B)[2], Raw& Rc, const Raw& Rn, const Rsrc& rs,
                                              const Offs& o, const uint32_t (&aoff)[4], f32x16_t (&acc)[MI][2],
                                              int wave, uint32_t nm, uint32_t mg, uint32_t ts) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t == 3) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        dma_x(rs, o, sm, bd, cnext2, wave);
        load_w(rs, o, Rc, cnext2, ts);
        if constexpr (SHARE) {
          Rc.s0 = Rn.s0;
          Rc.s1 = Rn.s1;
          Rc.z0 = Rn.z0;
          Rc.z1 = Rn.z1;
        } else {
          load_sz(rs, o, Rc, cnext2);
        }
      }
      bf16x8_t An[MI], Bn[2];
#pragma unroll
      for (int i = 0; i < MI; ++i) An[i] = t < 3 ? read_a(sm, bc, aoff[t + 1], i) : read_a(sm, bn, aoff[0], i);
#pragma unroll
      for (int j = 0; j < 2; ++j) Bn[j] = t < 3 ? decode(Rc, o.zsh, j, t + 1, nm, mg) : decode(Rn, o.zsh, j, 0, nm, mg);
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[i], B[0], acc[i][0], 0, 0, 0);
        acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[i], B[1], acc[i][1], 0, 0, 0);
      }
      // Per row block: one LDS read, two MFMAs, ~5 VALU ops.
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
      }
#pragma unroll
      for (int i = 0; i < MI; ++i) A[i] = An[i];
      B[0] = Bn[0];
      B[1] = Bn[1];
      // Keep the next step's MFMAs (which consume the reads just issued)
      // out of this step, so LDS latency hides behind this step's MFMAs.
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // One output element (row m, column n < N) of lane l32 in the fused
  // SiLU-and-mul instance (SILU, a.silu_mul): the weight rows interleave gate and up
  // in 16-row blocks, so lane l32 < 16 of a 32-column block holds gate column
  // g = 16*(n/32) + l32 and lane l32 + 16 the matching up column.  As in the
  // reference's unfused sequence (hydraserve/model/runtime.py:1202-1210,
  // silu_and_mul at hydraserve/kernels/activation.py:66-76), gate and up are
  // rounded to bf16 first, then out = gate * sigmoid(gate) * up in fp32,
  // rounded to bf16, into y [M, N/2].  Every lane of the wave calls this for
  // the same (m, register) together, so the cross-lane exchange sees its
  // partner; N is a multiple of 32, so a lane and its partner agree on n < N.
  static __device__ __forceinline__ void put_silu(const GemmArgs& a, int m, int n, float v, int l32) {
    const float own = bf16_to_f32(to_bf16_bits(v));
    const float up = __shfl_xor(own, 16);
    if (l32 < 16 && m < a.M) {
      const float sig = 1.0f / (1.0f + expf(-own));
      a.y[m * a.ldy + (n >> 5) * 16 + (n & 15)] = to_bf16_bits(own * sig * up);
    }
  }

  // Lane (l32, h), register e of block (i, j): row 32i + 8(e/4) + 4h + e%4,
  // column 64*wave + 32j + l32.
  static __device__ __forceinline__ void store_tile(const GemmArgs& a, const f32x16_t (&acc)[MI][2], int tm,
                                                    int tn, int wave, int l32, int h) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = tn * BN + wave * 64 + 32 * j + l32;
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = tm * BM + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
          if constexpr (SILU) {
            put_silu(a, m, n, acc[i][j][e], l32);
          } else {
            if (m < a.M) a.y[m * a.ldy + n] = to_bf16_bits(acc[i][j][e]);
          }
        }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Partial layout (bytes in a slot): 16-byte chunk v (elements 4v..4v+3)
  // of accumulator block b = (wave*MI + i)*2 + j of a lane at
  // ((b*4 + v)*64 + lane)*16, so every 16-byte store or load covers 1 KB.
  static __device__ __forceinline__ uint32_t part_off(int b, int v, int lane) {
    return static_cast<uint32_t>(((b * 4 + v) * 64 + lane) * 16);
  }

  static __device__ __forceinline__ uint32_t slot_off(int v, int slot) {
    return static_cast<uint32_t>((v * 2 + slot) * SLOT * 4);
  }

  static __device__ __forceinline__ void finish_tile(const GemmArgs& a, Smem& sm, f32x16_t (&acc)[MI][2], int t,
                                                     int tm, int tn, int v, int64_t u0, int64_t u1, int tid) {
    const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int64_t ts = static_cast<int64_t>(t) * a.G, te = ts + a.G;
    if (u0 <= ts && u1 >= te) {
      store_tile(a, acc, tm, tn, wave, l32, h);
      return;
    }
    const int pf = unit_owner(ts, a.U, a.P), pl = unit_owner(te - 1, a.U, a.P);
    const auto pr = partial_rsrc(a.partials);
    // A range that comes from earlier tiles and ends in this one reaches it
    // last (the other contributors work on it at the start of their ranges,
    // or have only this tile), so it first looks at the
    // arrival counter: when every other contributor has arrived, it settles
    // with its own sums from the accumulators and stores no partial.
    // Otherwise (or when it does not end here) it stores its partial and
    // arrives; whoever arrives last settles from the stored partials.  No
    // workgroup waits for another, and the sum runs in workgroup order
    // either way, so the result does not depend on who settles.
    bool own = false;
    if (u0 < ts && u1 <= te) {
      if (tid == 0)
        sm.flag = __hip_atomic_load(&a.counters[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == pl - pf;
      __syncthreads();
      own = sm.flag != 0;
    }
    if (!own) {
      const uint32_t mine = slot_off(v, partial_slot(v, t, a.G, a.U, a.P));
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4)
            store_partial4(pr, mine + part_off((wave * MI + i) * 2 + j, c4, lane),
                           f32x4_t{acc[i][j][4 * c4], acc[i][j][4 * c4 + 1], acc[i][j][4 * c4 + 2], acc[i][j][4 * c4 + 3]});
          __builtin_amdgcn_sched_barrier(0);
        }
      if (!arrive_last(a.counters, t, pl - pf + 1, &sm.flag)) return;
    }
    // Sum every contributor's partial in workgroup order, two row blocks at
    // a time: all 16 of a contributor's 16-byte loads for them are in flight
    // before any is summed.
#pragma unroll
    for (int i0 = 0; i0 < MI; i0 += 2) {
      f32x16_t sum[2][2] = {};
      for (int q = pf; q <= pl; ++q) {
        if (own && q == v) {
#pragma unroll
          for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int j = 0; j < 2; ++j) sum[ii][j] += acc[i0 + ii][j];
          continue;
        }
        const uint32_t base = slot_off(q, partial_slot(q, t, a.G, a.U, a.P));
        f32x4_t x[2][2][4];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4)
              x[ii][j][c4] = load_partial4(pr, base + part_off((wave * MI + i0 + ii) * 2 + j, c4, lane));
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
              for (int c = 0; c < 4; ++c) sum[ii][j][4 * c4 + c] += x[ii][j][c4][c];
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = tn * BN + wave * 64 + 32 * j + l32;
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int m = tm * BM + 32 * (i0 + ii) + 8 * (e >> 2) + 4 * h + (e & 3);
            if constexpr (SILU) {
              if (n < a.N) put_silu(a, m, n, sum[ii][j][e], l32);
            } else {
              if (m < a.M && n < a.N) a.y[m * a.ldy + n] = to_bf16_bits(sum[ii][j][e]);
            }
          }
      }
    }
    reset_counter(a.counters, t);
  }
};

// a.G = 128-wide K groups per tile (the stream-K unit; the pipeline runs on
// 64-wide halves of them), a.T = tiles, a.TM = tiles along M, a.U = T * G,
// a.P = workgroups.  Tile t covers rows (t / (T/TM)) * 256 and
// weight rows (t % (T/TM)) * 256.
template <int WT, int SDT, bool SILU, bool TL>
__global__ __launch_bounds__(WD_THREADS, 1) void qgemm_wide_kernel(GemmArgs a) {
  using W = Wide<WT, SDT, SILU, TL>;
  __shared__ typename W::Smem sm;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int p = blockIdx.x;
  // Workgroups of one XCD (p % 8) take one contiguous run of units.
  const int v = (a.P % 8 == 0 && !(a.tune & 1)) ? (p % 8) * (a.P / 8) + p / 8 : p;
  const int64_t u0 = unit_begin(v, a.U, a.P), u1 = unit_begin(v + 1, a.U, a.P);
  // Byte extents of the buffers (wide_ok keeps them below 2^32).
  typename W::Rsrc rs;
  rs.x = make_rsrc(a.x, (static_cast<int64_t>(a.M - 1) * a.ldx + a.K) * 2);
  if constexpr (WT == W_INT4) {
    rs.w = make_rsrc(a.w, (static_cast<int64_t>(a.N - 1) * a.ldw + a.K / 8) * 4);
    rs.z = make_rsrc(a.zero, (static_cast<int64_t>((a.N - 1) / 8) * a.ldz + a.K / 128) * 4);
    rs.s = make_rsrc(a.scale, (static_cast<int64_t>(a.N - 1) * a.lds + a.K / 128) * (SDT == SCALE_F32 ? 4 : 2));
  } else {
    rs.w = make_rsrc(a.w, static_cast<int64_t>(a.N - 1) * a.ldw + a.K);
    rs.z = rs.w;
    rs.s = make_rsrc(a.scale, (static_cast<int64_t>((a.N - 1) / 128) * a.lds + a.K / 128) *
                                  (SDT == SCALE_F32 ? 4 : 2));
  }
  // Tiled copy: N/16 tiles of TB bytes per 128-wide K chunk (wide_tiles_ok
  // keeps the whole copy below 2^31 bytes).
  const uint32_t ts = static_cast<uint32_t>(a.N / 16) * (WT == W_INT4 ? 1024u : 2048u);
  if constexpr (TL) rs.w = make_rsrc(a.wtiles, static_cast<int64_t>(ts) * (a.K / 128));

  uint32_t aoff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) aoff[t] = l32 * 128 + (((4 * h + t) ^ ((l32 >> 1) & 7)) * 16);
  const uint32_t nm = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t mg = opaque_and(0x64006400u, 0xFFFFFFFFu);

  int64_t u = u0;
  while (u < u1) {
    const int t = static_cast<int>(u / a.G);
    const int gb = static_cast<int>(u - static_cast<int64_t>(t) * a.G);
    const int ge = static_cast<int>((u1 - static_cast<int64_t>(t) * a.G) < a.G ? (u1 - static_cast<int64_t>(t) * a.G)
                                                                                : a.G);
    // 64-wide units [cb, ce): an even start and an even count.
    const int cb = 2 * gb, ce = 2 * ge, n = ce - cb;
    int tm, tn;
    W::coords(a, t, tm, tn);

    // Prologue: X(cb), X(cb+1) into LDS buffers 0, 1; weights of cb and
    // cb+1 into registers; step 0 of cb prepared.
    typename W::Offs o;
    W::offsets(a, o, tm, tn, wave, l32, h, tid);
    typename W::Raw r0, r1;
    const int c1 = cb + 1;
    W::dma_x(rs, o, sm, 0, cb, wave);
    W::dma_x(rs, o, sm, W::XB, c1, wave);
    W::load_raw(rs, o, r0, cb, ts);
    W::load_raw(rs, o, r1, c1, ts);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    bf16x8_t A[W::MI], B[2];
#pragma unroll
    for (int i = 0; i < W::MI; ++i) A[i] = W::read_a(sm, 0, aoff[0], i);
    B[0] = W::decode(r0, o.zsh, 0, 0, nm, mg);
    B[1] = W::decode(r0, o.zsh, 1, 0, nm, mg);

    f32x16_t acc[W::MI][2];
#pragma unroll
    for (int i = 0; i < W::MI; ++i) acc[i][0] = acc[i][1] = f32x16_t{};

    // LDS buffers rotate b0 (this unit) -> b1 (next) -> b2 (DMA target).
    // Unit indices past the tile's last are clamped (their loads are
    // harmless and never used).  Units run in pairs (one 128-K group) so
    // that the two raw-weight register sets alternate without copies and
    // the odd half reuses the even half's scale and zero point; the pair
    // loop has a single exit (a break between the two units makes the
    // register allocator shuffle the accumulators).
    int b0 = 0, b1 = W::XB, b2 = 2 * W::XB;
    for (int q = 0; q < n; q += 2) {
      const int cn0 = cb + q + 2 < ce ? cb + q + 2 : ce - 1;
      const int cn1 = cb + q + 3 < ce ? cb + q + 3 : ce - 1;
      W::template unit<false>(sm, b0, b1, b2, cn0, A, B, r0, r1, rs, o, aoff, acc, wave, nm, mg, ts);
      W::template unit<true>(sm, b1, b2, b0, cn1, A, B, r1, r0, rs, o, aoff, acc, wave, nm, mg, ts);
      const int tb = b0;
      b0 = b2;
      b2 = b1;
      b1 = tb;
    }
    // Drain the clamped prefetches before the buffers are reused.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    W::finish_tile(a, sm, acc, t, tm, tn, v, u0, u1, tid);
    __syncthreads();
    u += ge - gb;
  }
}

template <int WT, int SDT, bool SILU = false, bool TL = false>
static hipError_t launch_wide_t(const GemmArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((qgemm_wide_kernel<WT, SDT, SILU, TL>), dim3(a.P), dim3(WD_THREADS), 0, stream, a);
  return hipGetLastError();
}

int wide_slot_floats() { return Wide<W_INT4, SCALE_BF16>::SLOT; }

bool wide_ok(const GemmArgs& a, int wt) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.K % 128 != 0 || !a.xvec || !a.wvec) return false;
  // Every buffer-load byte offset must fit in 32 bits.
  const int64_t lim = int64_t(1) << 31;
  const int64_t xb = (static_cast<int64_t>(a.M) * a.ldx + a.K) * 2;
  const int64_t wb = wt == W_INT4 ? (static_cast<int64_t>(a.N) * a.ldw + a.K / 8) * 4
                                  : static_cast<int64_t>(a.N) * a.ldw + a.K;
  const int64_t sb = (static_cast<int64_t>(a.N) * a.lds + a.K / 128) * 4;
  const int64_t zb = (static_cast<int64_t>(a.N / 8 + 1) * a.ldz + a.K / 128) * 4;
  return xb < lim && wb < lim && sb < lim && zb < lim;
}

bool wide_tiles_ok(const GemmArgs& a, int wt) {
  const int64_t bytes = static_cast<int64_t>(a.N) * a.K / (wt == W_INT4 ? 2 : 1);
  return a.wtiles != nullptr && a.N % 16 == 0 && a.K % 128 == 0 && bytes < (int64_t(1) << 31);
}

hipError_t launch_wide(int wt, const GemmArgs& a, hipStream_t stream) {
  if (wt == W_INT4 && a.silu_mul && a.wtiles != nullptr) {
    if (a.sdt == SCALE_BF16) return launch_wide_t<W_INT4, SCALE_BF16, true, true>(a, stream);
    if (a.sdt == SCALE_F16) return launch_wide_t<W_INT4, SCALE_F16, true, true>(a, stream);
    return launch_wide_t<W_INT4, SCALE_F32, true, true>(a, stream);
  }
  if (wt == W_INT4 && a.silu_mul) {
    if (a.sdt == SCALE_BF16) return launch_wide_t<W_INT4, SCALE_BF16, true>(a, stream);
    if (a.sdt == SCALE_F16) return launch_wide_t<W_INT4, SCALE_F16, true>(a, stream);
    return launch_wide_t<W_INT4, SCALE_F32, true>(a, stream);
  }
  if (a.silu_mul) return hipErrorInvalidValue;
  if (a.wtiles != nullptr) {
    if (wt == W_INT4) {
      if (a.sdt == SCALE_BF16) return launch_wide_t<W_INT4, SCALE_BF16, false, true>(a, stream);
      if (a.sdt == SCALE_F16) return launch_wide_t<W_INT4, SCALE_F16, false, true>(a, stream);
      return launch_wide_t<W_INT4, SCALE_F32, false, true>(a, stream);
    }
    if (a.sdt == SCALE_BF16) return launch_wide_t<W_FP8, SCALE_BF16, false, true>(a, stream);
    if (a.sdt == SCALE_F16) return launch_wide_t<W_FP8, SCALE_F16, false, true>(a, stream);
    return launch_wide_t<W_FP8, SCALE_F32, false, true>(a, stream);
  }
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_wide_t<W_INT4, SCALE_BF16>(a, stream);
    if (a.sdt == SCALE_F16) return launch_wide_t<W_INT4, SCALE_F16>(a, stream);
    return launch_wide_t<W_INT4, SCALE_F32>(a, stream);
  }
  if (a.sdt == SCALE_BF16) return launch_wide_t<W_FP8, SCALE_BF16>(a, stream);
  if (a.sdt == SCALE_F16) return launch_wide_t<W_FP8, SCALE_F16>(a, stream);
  return launch_wide_t<W_FP8, SCALE_F32>(a, stream);
}

}  // namespace hsq
