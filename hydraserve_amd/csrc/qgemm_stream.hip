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
//     its row per chunk per strip into a register ring one batch deep: chunk
//     r of batch b+1 is requested as soon as chunk r of batch b is consumed.
//     The ring and the accumulators are the only registers carried from one
//     batch to the next, so the compiler never copies a register that still
//     has a load in flight (such a copy waits for every older load, i.e.
//     drains the ring).
//   * X, scales and zero points of batch b+1 are fetched into registers at
//     the start of batch b and published to LDS (double-buffered) at its end,
//     with one barrier per batch.  For INT4 the fp32 sum of every 128-value
//     group of X is computed while publishing.  Lanes read their scales and
//     zero points for a batch from LDS with one vector read each.
//   * Every global load is unconditional (cursors clamp at the range's end
//     and rows clamp at N-1 / M-1; clamped results are never stored).
//
// Arithmetic (exact unpack, weights never rounded to bf16):
//   INT4: nibble q -> bf16 128+q (v_perm_b32 + v_and_or_b32 under the
//   exponent of 128.0); T = MFMA(X, 128+q); Xg = the fp32 sum of the group's
//   128 X values; acc += s * (T - (128+z) * Xg).
//   FP8: E4M3FN -> bf16 exactly (v_cvt_scalef32_pk_bf16_fp8, unit scale);
//   acc += s_block * MFMA(X, W).
#include <type_traits>

#include "qgemm_ops.h"

namespace hsq {

constexpr int ST_THREADS = 256;

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

// Batch cursor: linear batch index, tile, batch within the tile.  advance()
// stops at the range's last batch, so loads issued for "the next batch" at
// the end of the range reload that batch (cache hits).
struct BCur {
  int lin, t, c;
  __device__ __forceinline__ bool advance(int last, int G) {
    if (lin < last) {
      ++lin;
      if (++c == G) {
        c = 0;
        ++t;
        return true;
      }
    }
    return false;
  }
};

template <int WT, int SDT, int MT, int S, int NB, int XR>
struct Stream {
  static constexpr int NT = 64 * S;          // weight rows per tile
  static constexpr int SES = SDT == SCALE_F32 ? 4 : 2;
  static constexpr int XK = NB * 128;        // bf16 per X row per batch
  static constexpr int XSTRIDE = XK + 8;     // LDS row stride (bank spread)
  static constexpr int XSEG = NB * 16;       // 16-byte segments per X row per batch
  static_assert(ST_THREADS % XSEG == 0, "a staging pass must cover whole rows");
  static constexpr int RPQ = ST_THREADS / XSEG;  // X rows per staging pass
  static constexpr int XQ = (XR + RPQ - 1) / RPQ;
  // INT4 group sums: [chunk][row], rows padded to RX so a lane reads its
  // four rows with one b128.
  static constexpr int RX = 16 * MT;
  static constexpr int XGF = WT == W_INT4 ? NB * RX : 0;
  // Scale staging.  INT4: one scale row per weight row; FP8: one per tile
  // (a tile never straddles a 128-row block).  SB bytes per row per batch,
  // moved in units of SU bytes.
  static constexpr int SROWS = WT == W_INT4 ? NT : 1;
  static constexpr int SB = NB * SES;
  static constexpr int SU = SB < 16 ? SB : 16;
  static constexpr int SUN = SROWS * (SB / SU);
  static_assert(SUN <= ST_THREADS, "one staging unit per thread");
  // Zero points (INT4): one int32 row per 8 weight rows, NB words per batch.
  static constexpr int ZB = NB * 4;
  static constexpr int ZU = ZB < 16 ? ZB : 16;
  static constexpr int ZUN = WT == W_INT4 ? (NT / 8) * (ZB / ZU) : 1;
  static constexpr int SBYTES = SROWS * SB;
  static constexpr int ZBYTES = WT == W_INT4 ? (NT / 8) * ZB : 0;
  static constexpr int STAGE_BYTES = (SBYTES + ZBYTES + 15) / 16 * 16;

  static __host__ __device__ size_t lds_bytes(int M) {
    return static_cast<size_t>(2) * M * XSTRIDE * 2 + 2 * XGF * 4 + 2 * STAGE_BYTES + 16;
  }

  // Loads are raw buffer loads: a resource descriptor in SGPRs, a per-lane
  // 32-bit offset fixed for the tile (VGPR) and a uniform offset (SGPR) that
  // the chunk / batch step advances, so no VALU address arithmetic sits
  // between loads.  The host guarantees every operand spans < 2^31 bytes.
  struct Rsrc {
    __amdgpu_buffer_rsrc_t w, s, z, x;
  };

  static __device__ __forceinline__ Rsrc make_rsrcs(const GemmArgs& a) {
    Rsrc r;
    const int64_t rb = WT == W_INT4 ? a.ldw * 4 : a.ldw;
    r.w = make_rsrc(a.w, static_cast<int64_t>(a.N - 1) * rb + (WT == W_INT4 ? a.K / 2 : a.K));
    if constexpr (WT == W_INT4) {
      const int g = a.K / 128;
      r.s = make_rsrc(a.scale, (static_cast<int64_t>(a.N - 1) * a.lds + g) * SES);
      r.z = make_rsrc(a.zero, (static_cast<int64_t>((a.N + 7) / 8 - 1) * a.ldz + g) * 4);
    } else {
      r.s = make_rsrc(a.scale, (static_cast<int64_t>((a.N + 127) / 128 - 1) * a.lds + a.K / 128) * SES);
      r.z = r.s;
    }
    r.x = make_rsrc(a.x, (static_cast<int64_t>(a.M - 1) * a.ldx + a.K) * 2);
    return r;
  }

  // Weights: lane row t*NT + (wave*S+s)*16 + l16, clamped to N-1.
  struct WRows {
    uint32_t sbase;     // byte offset of the tile's first row
    uint32_t off[S];    // lane's offset from it
  };
  // Scale / zero-point staging rows of a tile (one unit per thread).
  struct SRows {
    uint32_t sb, zb;    // tile bases
    uint32_t soff, zoff;
  };

  static __device__ __forceinline__ void set_wrows(const GemmArgs& a, WRows& r, int t, int wave, int lane) {
    const int l16 = lane & 15, h = lane >> 4;
    const int rb = static_cast<int>(WT == W_INT4 ? a.ldw * 4 : a.ldw);  // bytes per weight row
    const int r0 = t * NT;
    r.sbase = static_cast<uint32_t>(r0 * rb);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      int row = r0 + (wave * S + s) * 16 + l16;
      row = row < a.N ? row : a.N - 1;
      r.off[s] = static_cast<uint32_t>((row - r0) * rb) + (WT == W_INT4 ? 16u : 32u) * h;
    }
  }

  static __device__ __forceinline__ void set_srows(const GemmArgs& a, SRows& r, int t, int tid) {
    const int su = tid < SUN ? tid : SUN - 1;
    constexpr int SPR = SB / SU;  // units per scale row
    const int r0 = t * NT;
    if constexpr (WT == W_INT4) {
      const int sr = static_cast<int>(a.lds) * SES;
      int row = r0 + su / SPR;
      row = row < a.N ? row : a.N - 1;
      r.sb = static_cast<uint32_t>(r0 * sr);
      r.soff = static_cast<uint32_t>((row - r0) * sr + (su % SPR) * SU);
      constexpr int ZPR = ZB / ZU;
      const int zr = static_cast<int>(a.ldz) * 4;
      const int zu = tid < ZUN ? tid : ZUN - 1;
      const int z0 = r0 / 8;
      int zrow = z0 + zu / ZPR;
      const int zrows = (a.N + 7) / 8;
      zrow = zrow < zrows ? zrow : zrows - 1;
      r.zb = static_cast<uint32_t>(z0 * zr);
      r.zoff = static_cast<uint32_t>((zrow - z0) * zr + (zu % ZPR) * ZU);
    } else {
      r.sb = static_cast<uint32_t>((r0 >> 7) * static_cast<int>(a.lds) * SES);
      r.soff = static_cast<uint32_t>((su % SPR) * SU);
      r.zb = 0;
      r.zoff = 0;
    }
  }

  static __device__ __forceinline__ void load_w(const Rsrc& rs, StW<WT, S>& r, const WRows& rw, int c) {
    constexpr int CB = WT == W_INT4 ? 64 : 128;  // bytes of a row per chunk
    const uint32_t so = rw.sbase + static_cast<uint32_t>(c * CB);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if constexpr (WT == W_INT4) {
        r.q[s] = bload<u32x4_t>(rs.w, rw.off[s], so);
      } else {
        r.q[s][0] = bload<u32x4_t>(rs.w, rw.off[s], so);
        r.q[s][1] = bload<u32x4_t>(rs.w, rw.off[s] + 16, so);
      }
    }
  }

  // ---- staging of a batch (chunks c0 .. c0+NB-1) --------------------------
  struct XStage {
    u32x4_t x[XQ];
  };
  struct SStage {
    Blob<SU> s;
    Blob<ZU> z;
  };
  struct Stage {
    XStage x;
    SStage s;
  };

  // X rows [0, M): thread tid takes segment tid % XSEG of rows
  // tid / XSEG + RPQ*q; rows past M reload row M-1 and are not published.
  // Per-thread offset of its X staging segment (fixed for the kernel).
  static __device__ __forceinline__ uint32_t x_off(const GemmArgs& a, int q, int tid) {
    int row = tid / XSEG + RPQ * q;
    row = row < a.M ? row : a.M - 1;
    return static_cast<uint32_t>(row * static_cast<int>(a.ldx) * 2 + (tid % XSEG) * 16);
  }

  static __device__ __forceinline__ void load_x(const Rsrc& rs, XStage& st, const uint32_t (&xo)[XQ], int c0) {
#pragma unroll
    for (int q = 0; q < XQ; ++q) st.x[q] = bload<u32x4_t>(rs.x, xo[q], static_cast<uint32_t>(c0 * 256));
  }

  static __device__ __forceinline__ void load_sc(const Rsrc& rs, SStage& st, const SRows& sr, int c0) {
    st.s = bload<Blob<SU>>(rs.s, sr.soff, sr.sb + static_cast<uint32_t>(c0 * SES));
    if constexpr (WT == W_INT4) st.z = bload<Blob<ZU>>(rs.z, sr.zoff, sr.zb + static_cast<uint32_t>(c0 * 4));
  }

  // Publish staged X: rows into xs and, for INT4, the fp32 sum of every
  // 128-value group into xg (8 values per thread, then a butterfly over the
  // 16 consecutive lanes holding one group).
  static __device__ __forceinline__ void store_x(const GemmArgs& a, uint16_t* xs, float* xg, const XStage& st,
                                                 int tid) {
    const int seg = tid % XSEG;
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int row = tid / XSEG + RPQ * q;
      if constexpr (WT == W_INT4) {
        if (row < a.M) *reinterpret_cast<u32x4_t*>(xs + row * XSTRIDE + seg * 8) = permute_x(st.x[q]);
      } else {
        if (row < a.M) *reinterpret_cast<u32x4_t*>(xs + row * XSTRIDE + seg * 8) = st.x[q];
      }
      if constexpr (WT == W_INT4) {
        float v = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v += __uint_as_float(st.x[q][e] << 16);
          v += __uint_as_float(st.x[q][e] & 0xFFFF0000u);
        }
        v += __shfl_xor(v, 8, 16);
        v += __shfl_xor(v, 4, 16);
        v += __shfl_xor(v, 2, 16);
        v += __shfl_xor(v, 1, 16);
        if ((seg & 15) == 0 && row < a.M) xg[(seg >> 4) * RX + row] = v;
      }
    }
  }

  static __device__ __forceinline__ void store_sc(uint8_t* sb, const SStage& st, int tid) {
    if (tid < SUN) *reinterpret_cast<Blob<SU>*>(sb + tid * SU) = st.s;
    if constexpr (WT == W_INT4) {
      if (tid < ZUN) *reinterpret_cast<Blob<ZU>*>(sb + SBYTES + tid * ZU) = st.z;
    }
  }

  // ---- per-lane scales of the current batch -------------------------------
  struct LaneScales {
    Blob<SB> s[WT == W_INT4 ? S : 1];
    Blob<ZB> z[WT == W_INT4 ? S : 1];
  };

  static __device__ __forceinline__ void read_scales(LaneScales& ls, const uint8_t* sb, int wave, int l16) {
    if constexpr (WT == W_INT4) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int lr = (wave * S + s) * 16 + l16;
        ls.s[s] = *reinterpret_cast<const Blob<SB>*>(sb + lr * SB);
        ls.z[s] = *reinterpret_cast<const Blob<ZB>*>(sb + SBYTES + (lr >> 3) * ZB);
      }
    } else {
      ls.s[0] = *reinterpret_cast<const Blob<SB>*>(sb);
    }
  }

  static __device__ __forceinline__ float scale_of(const LaneScales& ls, int s, int u) {
    const int si = WT == W_INT4 ? s : 0;
    if constexpr (SES == 4) {
      return __uint_as_float(ls.s[si][u]);
    } else {
      const uint32_t pair = ls.s[si][u >> 1];
      const uint32_t h16 = (u & 1) ? (pair >> 16) : (pair & 0xFFFFu);
      if constexpr (SDT == SCALE_BF16) return __uint_as_float(h16 << 16);
      return __half2float(__ushort_as_half(static_cast<unsigned short>(h16)));
    }
  }

  // ---- per-chunk pipeline pieces --------------------------------------------
  // Chunk u of the batch.  Lane (l16, h): A rows 16i + l16 (clamped to M-1),
  // K [u*128 + 32h + 8j, +8) of the staged batch; B column l16 of each strip.
  struct AFrag {
    bf16x8_t a[MT][4];
    f32x4_t xg[MT];
  };
  struct BOp {
    bf16x8_t b[S][4];
  };
  struct TOut {
    f32x4_t t[S][MT];
  };

  static __device__ __forceinline__ void read_a(AFrag& f, const uint16_t* xs, const float* xgs, int u,
                                                const int (&arow)[MT], int h) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        f.a[i][j] = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const u32x4_t*>(xs + arow[i] * XSTRIDE + u * 128 + 32 * h + 8 * j));
    if constexpr (WT == W_INT4) {
#pragma unroll
      for (int i = 0; i < MT; ++i) f.xg[i] = *reinterpret_cast<const f32x4_t*>(xgs + u * RX + 16 * i + 4 * h);
    }
  }

  static __device__ __forceinline__ void unpack(BOp& b, const StW<WT, S>& w, uint32_t nib_mask, uint32_t magic) {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (WT == W_INT4) {
          b.b[s][j] = int4_operand(w.q[s][j], nib_mask, magic);
        } else {
          b.b[s][j] = fp8_operand(w.q[s][j >> 1][(j & 1) * 2], w.q[s][j >> 1][(j & 1) * 2 + 1]);
        }
      }
  }

  static __device__ __forceinline__ void mfma(TOut& o, const AFrag& f, const BOp& b) {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a[i][j], b.b[s][j], t, 0, 0, 0);
        o.t[s][i] = t;
      }
  }

  // acc += s * (T - (128+z) * Xg)  (INT4)   /   acc += s * T  (FP8)
  static __device__ __forceinline__ void fold(f32x4_t (&acc)[S][MT], const TOut& o, const f32x4_t (&xg)[MT],
                                              const LaneScales& ls, int u, uint32_t zsh) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float sc = scale_of(ls, s, u);
      float negc = 0.f;
      if constexpr (WT == W_INT4) negc = -(128.0f + static_cast<float>((ls.z[s][u] >> zsh) & 0xFu));
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (WT == W_INT4) {
            acc[s][i][e] = fmaf(sc, fmaf(negc, xg[i][e], o.t[s][i][e]), acc[s][i][e]);
          } else {
            acc[s][i][e] = fmaf(sc, o.t[s][i][e], acc[s][i][e]);
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
  static __device__ __forceinline__ uint32_t slot_off(int p, int slot) {
    return static_cast<uint32_t>((p * 2 + slot) * SLOT * 4);
  }
  // The f32x4 accumulator of block (wave, s, i) of a lane sits at byte
  // (((wave*S + s)*MT + i)*64 + lane)*16 of the slot: every 16-byte store or
  // load covers 1 KB.
  static __device__ __forceinline__ uint32_t part_off(int wave, int s, int i, int lane) {
    return static_cast<uint32_t>((((wave * S + s) * MT + i) * 64 + lane) * 16);
  }

  // End of tile t inside this workgroup's range.  A tile the range covers
  // whole is stored as bf16; otherwise the fp32 partial goes to this
  // workgroup's slot and true is returned: the tile still has to be settled.
  // Nothing here waits for memory, so the weight pipeline keeps streaming.
  static __device__ __forceinline__ bool end_tile(const GemmArgs& a, const f32x4_t (&acc)[S][MT], int t, int p,
                                                  int64_t b0, int64_t b1, int tid) {
    const int wave = tid >> 6, lane = tid & 63, l16 = lane & 15, h = lane >> 4;
    const int64_t ts = static_cast<int64_t>(t) * a.G, te = ts + a.G;
    if (b0 <= ts && b1 >= te) {
      store_tile(a, acc, t, wave, l16, h);
      return false;
    }
    const auto pr = partial_rsrc(a.partials);
    const uint32_t mine = slot_off(p, partial_slot(p, t, a.G, a.U, a.P));
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) store_partial4(pr, mine + part_off(wave, s, i, lane), acc[s][i]);
    return true;
  }

  // Settle this range's split tiles (t0, t1; -1 = none) once the range is
  // done: one drain for the partial stores, one arrival round for both
  // tiles; the last contributor of a tile sums every partial in workgroup
  // order (deterministic), stores bf16 and resets the counter.  Partial loads
  // are 16-byte coherent loads that stay in flight together.
  static __device__ __forceinline__ void settle(const GemmArgs& a, int* flag, int t0, int t1, int tid) {
    const int wave = tid >> 6, lane = tid & 63, l16 = lane & 15, h = lane >> 4;
    int pf[2], pl[2];
    const int tt[2] = {t0, t1};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      pf[k] = pl[k] = 0;
      if (tt[k] >= 0) {
        const int64_t ts = static_cast<int64_t>(tt[k]) * a.G;
        pf[k] = unit_owner(ts, a.U, a.P);
        pl[k] = unit_owner(ts + a.G - 1, a.U, a.P);
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial stores are acknowledged
    __syncthreads();
    if (tid < 2) {
      int last = 0;
      if (tt[tid] >= 0) {
        const int old = __hip_atomic_fetch_add(&a.counters[tt[tid]], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == pl[tid] - pf[tid];
      }
      flag[tid] = last;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (!flag[k]) continue;
      const int t = tt[k];
      f32x4_t acc[S][MT];
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[s][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const auto pr = partial_rsrc(a.partials);
      for (int q = pf[k]; q <= pl[k]; ++q) {
        const uint32_t base = slot_off(q, partial_slot(q, t, a.G, a.U, a.P));
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int i = 0; i < MT; ++i) acc[s][i] += load_partial4(pr, base + part_off(wave, s, i, lane));
      }
      store_tile(a, acc, t, wave, l16, h);
      if (tid == 0) __hip_atomic_store(&a.counters[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
};

// a.G = batches per tile, a.NB = NB, a.U = T * a.G, a.P = workgroups.
// Dynamic LDS (Stream::lds_bytes): 2 X buffers of M rows, 2 group-sum buffers
// (INT4), 2 scale/zero-point buffers, a flag word.
//
// Pipeline, batch b on the compute side.  Everything is fetched two batches
// ahead, because the memory counter completes loads in issue order: waiting
// for any load also waits for every older one, so data that is consumed one
// batch after it was requested would force the whole next batch of weights
// to land as well.
//   * weights: a register ring two batches deep (ring[b % 2][chunk]); the slot
//     of chunk r is refilled with chunk r of batch b+2 right after use;
//   * X, scales and zero points of batch b+2 are loaded into the register
//     set named for b's parity at the start of batch b and published to LDS
//     at the end of batch b+1.
// The batch loop is unrolled twice so every ring slot and register set has
// a fixed name: nothing loaded is ever copied (a copy would also wait).
template <int WT, int SDT, int MT, int S, int NB, int XR>
__global__ __launch_bounds__(ST_THREADS) void qgemm_stream_kernel(GemmArgs a) {
  using D = Stream<WT, SDT, MT, S, NB, XR>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int xs_bytes = a.M * D::XSTRIDE * 2;
  uint8_t* const xs_base = smem;
  uint8_t* const xg_base = smem + 2 * xs_bytes;
  uint8_t* const sb_base = xg_base + 2 * D::XGF * 4;
  int* flag = reinterpret_cast<int*>(sb_base + 2 * D::STAGE_BYTES);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(tid >> 6));
  const int lane = tid & 63, l16 = lane & 15, h = lane >> 4;
  const int p = blockIdx.x;
  const int64_t b0 = unit_begin(p, a.U, a.P), b1 = unit_begin(p + 1, a.U, a.P);
  if (b0 >= b1) return;
  const int G = a.G;
  const int last = static_cast<int>(b1) - 1;
  const uint32_t nib_mask = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t magic = opaque_and(0x43004300u, 0xFFFFFFFFu);
  const uint32_t zsh = 4u * static_cast<uint32_t>(l16 & 7);  // tiles and strips start at multiples of 8 rows
  int arow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) arow[i] = (16 * i + l16) < a.M ? 16 * i + l16 : a.M - 1;

  BCur cur{static_cast<int>(b0), static_cast<int>(b0) / G, static_cast<int>(b0) % G};
  BCur wc = cur;  // the batch being fetched: b+2
  typename D::WRows wr;
  typename D::SRows sr;
  D::set_wrows(a, wr, wc.t, wave, lane);
  D::set_srows(a, sr, wc.t, tid);
  const typename D::Rsrc rs = D::make_rsrcs(a);
  uint32_t xo[D::XQ];
#pragma unroll
  for (int q = 0; q < D::XQ; ++q) xo[q] = D::x_off(a, q, tid);

  StW<WT, S> ring[2][NB];
  typename D::Stage st0, st1;
  // Fetch batch `wc` into ring half H and stage set `st`, then step wc.
  auto fetch_stage = [&](typename D::Stage& st) __attribute__((always_inline)) {
    D::load_x(rs, st.x, xo, wc.c * NB);
    D::load_sc(rs, st.s, sr, wc.c * NB);
  };
  auto advance_wc = [&]() __attribute__((always_inline)) {
    if (wc.advance(last, G)) {
      D::set_wrows(a, wr, wc.t, wave, lane);
      D::set_srows(a, sr, wc.t, tid);
    }
  };
  auto publish = [&](const typename D::Stage& st, int b) __attribute__((always_inline)) {
    D::store_x(a, reinterpret_cast<uint16_t*>(xs_base + b * xs_bytes),
               reinterpret_cast<float*>(xg_base + b * D::XGF * 4), st.x, tid);
    D::store_sc(sb_base + b * D::STAGE_BYTES, st.s, tid);
  };
  // Prologue: batches b0 and b0+1.
  fetch_stage(st0);
#pragma unroll
  for (int r = 0; r < NB; ++r) D::load_w(rs, ring[0][r], wr, wc.c * NB + r);
  advance_wc();
  fetch_stage(st1);
#pragma unroll
  for (int r = 0; r < NB; ++r) D::load_w(rs, ring[1][r], wr, wc.c * NB + r);
  advance_wc();
  publish(st0, 0);
  __syncthreads();

  f32x4_t acc[S][MT];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[s][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int buf = 0;
  // Split tiles of this range (at most its first and its last), settled
  // after the range so that no mid-range wait drains the weight pipeline.
  int pend0 = -1, pend1 = -1;

  // Batch `cur` (parity H): `mine` receives batch b+2, `other` holds batch
  // b+1 and is published at the end.  True when the range is done.
  auto step = [&](auto half, typename D::Stage& mine, const typename D::Stage& other) __attribute__((always_inline)) {
    constexpr int H = decltype(half)::value;
    fetch_stage(mine);
    const uint16_t* xs = reinterpret_cast<const uint16_t*>(xs_base + buf * xs_bytes);
    const float* xg = reinterpret_cast<const float*>(xg_base + buf * D::XGF * 4);
    typename D::LaneScales ls;
    D::read_scales(ls, sb_base + buf * D::STAGE_BYTES, wave, l16);
    const int wcol = wc.c * NB;
    // Software pipeline over the batch's chunks: iteration r refills the
    // ring slot of chunk r-1 (unpacked last iteration), reads the A
    // fragments of chunk r+1, unpacks and multiplies chunk r and folds the
    // products of chunk r-1, so LDS and MFMA latencies overlap other work.
    // fa[] holds chunks r and r+1, xgp the group sums of chunk r-1 (read
    // with its fragments, consumed by its fold one iteration later).
    typename D::AFrag fa[2];
    typename D::TOut to[2];
    f32x4_t xgp[MT];
    D::read_a(fa[0], xs, xg, 0, arow, h);
#pragma unroll
    for (int r = 0; r < NB; ++r) {
      if (r > 0) D::load_w(rs, ring[H][r - 1], wr, wcol + r - 1);
      if (r + 1 < NB) D::read_a(fa[(r + 1) & 1], xs, xg, r + 1, arow, h);
      typename D::BOp bo;
      D::unpack(bo, ring[H][r], nib_mask, magic);
      D::mfma(to[r & 1], fa[r & 1], bo);
      if (r > 0) D::fold(acc, to[(r - 1) & 1], xgp, ls, r - 1, zsh);
#pragma unroll
      for (int i = 0; i < MT; ++i) xgp[i] = fa[r & 1].xg[i];
      __builtin_amdgcn_sched_barrier(0);
    }
    D::load_w(rs, ring[H][NB - 1], wr, wcol + NB - 1);
    D::fold(acc, to[(NB - 1) & 1], xgp, ls, NB - 1, zsh);
    advance_wc();
    buf ^= 1;
    publish(other, buf);
    __syncthreads();
    const bool done = cur.lin == last;
    if (cur.c + 1 == G || done) {
      if (D::end_tile(a, acc, cur.t, p, b0, b1, tid)) (pend0 < 0 ? pend0 : pend1) = cur.t;
      if (done) return true;
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[s][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      cur.c = 0;
      ++cur.t;
    } else {
      ++cur.c;
    }
    ++cur.lin;
    return false;
  };
  for (;;) {
    if (step(std::integral_constant<int, 0>{}, st0, st1)) break;
    if (step(std::integral_constant<int, 1>{}, st1, st0)) break;
  }
  if (pend0 >= 0) D::settle(a, flag, pend0, pend1, tid);
}

template <int WT, int SDT, int MT, int S, int NB, int XR>
static hipError_t launch_stream_t(const GemmArgs& a, hipStream_t stream) {
  using D = Stream<WT, SDT, MT, S, NB, XR>;
  const size_t lds = D::lds_bytes(a.M);
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
  // Byte extents of every operand (with the tile overhang the kernel's
  // clamped row indices can reach) stay below the 32-bit buffer range.
  const int64_t lim = int64_t(1) << 31;
  const int64_t xb = (static_cast<int64_t>(a.M) * a.ldx + a.K) * 2;
  const int64_t wb = (static_cast<int64_t>(a.N) + 256) * a.ldw * (wt == W_INT4 ? 4 : 1);
  const int64_t sb = (static_cast<int64_t>(a.N) + 256) * a.lds * 4;
  const int64_t zb = (static_cast<int64_t>(a.N / 8) + 64) * a.ldz * 4;
  if (xb >= lim || wb >= lim || sb >= lim || zb >= lim) return false;
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
