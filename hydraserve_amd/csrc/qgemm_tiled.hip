// Decode-regime (1..64 activation rows) quantized weight GEMM over the
// load-time tiled weight copy, for gfx950.
//
// Replaces the Triton launches of hydraserve/kernels/awq.py:52-74
// (_awq_gemm_kernel, awq.py:82-142) and hydraserve/kernels/fp8.py:68-96
// (_fp8_gemm_kernel, fp8.py:104-168) when the weight carries a tiled copy
// (hydraserve_amd/kernels/tiles.py): tile (t, c) = rows 16t..16t+15 of the
// 128-wide K chunk c, stored contiguously (INT4: 16 rows x 64 bytes = 1 KiB;
// FP8: 16 rows x 128 bytes = 2 KiB, as two KiB halves of K 0..63 and
// 64..127, each lane's 16 bytes at 16 lane) at byte (c * N/16 + t) *
// tile_bytes, i.e.
// chunk-major: the tiles of one K chunk are adjacent, so the whole grid,
// walking K in step, reads one window of the weight at a time.  Every weight
// load instruction reads one contiguous KiB.  INT4 tile words keep their K
// range (word j of a row's chunk: K 8j .. 8j+7) with the nibbles paired for
// the MFMA operand: nibble i (i < 4) holds K 8j + 2i and nibble i + 4 holds
// K 8j + 2i + 1, so ((w >> 4i) & 0x000F000F) puts two consecutive-K weights
// in the two halves of a dword.
//
// Work split.  The N/16 tiles are cut into groups of `tpw` consecutive tiles
// and K into `splits` ranges of `cps` chunks; workgroup p takes tile group
// p / splits over K range p % splits.  Its waves own the group's tiles
// round-robin and walk the K range together, one chunk per step:
//   * each wave's weights go global -> registers through a ring of D chunks
//     unrolled by its depth (D-1 chunks in flight); the chunk's X rows go
//     global -> LDS by LDS-DMA in double-buffered rounds of R chunks with one
//     workgroup barrier per round; FP8 scales go by LDS-DMA per chunk, INT4
//     scales and zero points by one 16-byte LDS-DMA load per lane per round
//     of 8 chunks;
//   * weights are dequantised in registers and feed v_mfma_f32_16x16x32_bf16:
//     lane (n, p) = (lane % 16, lane / 16) supplies weight row n and X row n
//     of each 16-row block, K offsets 32p + 8s .. +8 at step s.  INT4 up to
//     32 rows: the group rewrite (128 + q as bf16, X sums from an all-ones
//     MFMA, acc += s (T - (128+z) Xg)); above, the reference's values
//     bf16_rne((q - z) * s) (awq.py:18-22, 136-137) via v_fma_mix on fp16
//     1024+q.  FP8: e4m3 -> bf16 exactly, the block scale applied to the
//     chunk's fp32 MFMA result;
//   * the loop body has no branches (skipped ring steps run after the loop,
//     each wave's code is specialised on its tile count, X loads past M are
//     out-of-range buffer loads), so the waits on loads in flight are exact.
// With one K range the workgroup stores bf16 Y directly.  With several, each
// workgroup writes an fp32 partial of its tile group, and the last of the
// group's workgroups to arrive sums the partials in K-range order
// (deterministic) and stores Y.
//
// LDS layout: X rows r = 0 .. 16*MB-1 of a chunk at 256r, the 16-byte K
// segment g at ((g ^ (r & 15)) * 16), so 16 consecutive rows' fragment reads
// hit distinct banks; per wave and 8-chunk round the INT4 scales (lane
// 16i + n: tile i's row n, 16 bytes per half of 4 chunks for fp32 scales)
// and zero-point words (lane 4i + 2h + half: tile i's word row h, chunks
// 4 half .. +3).
#include <cstdlib>
#include <type_traits>

#include "qgemm_ops.h"

namespace hsq {

constexpr int kTmLds = 160 * 1024;

struct TmRsrc {
  __amdgpu_buffer_rsrc_t x, w, s, z;
};

template <int WT, int MB, int TW, int NW>
struct Tm {
  static constexpr int TB = WT == W_INT4 ? 1024 : 2048;  // bytes of one tile
  static constexpr int LPT = TB / 1024;                  // 16-byte loads per lane per tile
  static constexpr int XB = MB * 4096;                   // X bytes of a chunk
  static constexpr int XI = XB / 1024;                   // 1 KiB X loads per chunk
  // D: chunks of the weight / scale ring (D-1 in flight; the weights of a
  // slot live in registers, TW * LPT * 4 VGPRs).  R: chunks per X round
  // (D a multiple of R); X rounds are double-buffered in LDS and the
  // workgroup meets at one barrier per round.
  // (FP8: a 4-deep ring measured faster than 6 or more at one row block,
  // gate_up M=1 30.9 -> 29.9 us, 9 deep 41.0, 12 deep 51.8: the fewer K
  // chunks the grid has in flight, the fewer DRAM pages it keeps open.)
  static constexpr int D = WT == W_INT4 ? 8 : 4;
  static constexpr int R = WT == W_INT4 ? (MB <= 2 ? 4 : 2) : 2;
  // R < D: the X of round 0 is issued inside the prologue, whose loads then
  // come in the same order as in every later round.
  static_assert(D % R == 0 && R < D, "X rounds tile the ring");
  static constexpr int XR = R * XB;                      // X bytes of a round
  static constexpr int LXR = (R * XI + NW - 1) / NW;     // X loads per wave per round
  // FP8: the chunk's scales (one per tile) in each ring slot.  INT4: the
  // scales and zero points of a whole ring round (D = 8 chunks) per wave,
  // double-buffered by round: MSB bytes per wave, scales at 0 (two 1 KiB
  // halves for fp32 scales, one for 16-bit ones), zero points at 2048.
  static constexpr int SB = WT == W_INT4 ? 0 : NW * 256;
  static constexpr int SLOTB = SB > 16 ? SB : 16;
  static constexpr int MSB = WT == W_INT4 ? 3072 : 0;
  static constexpr int MB2 = MSB > 0 ? 2 * NW * MSB : 16;
  static_assert(WT != W_INT4 || D == 8, "INT4 scale rounds are ring rounds of 8 chunks");
  static_assert(2 * XR + D * SLOTB + MB2 + 1024 + 256 <= kTmLds, "LDS");
  static constexpr int SLOT = NW * TW * MB * 256;  // floats of one workgroup's partial

  struct Smem {
    __attribute__((aligned(1024))) uint8_t xs[2][XR];
    __attribute__((aligned(1024))) uint8_t ring[D][SLOTB];
    __attribute__((aligned(1024))) uint8_t meta[MB2];
    uint8_t junk[1024];  // target of the X loads that carry no data
    int flag;
  };

  // Buffer accesses (kept out of the kernel's lambdas).
  static __device__ __forceinline__ void dma(__amdgpu_buffer_rsrc_t r, uint8_t* lds, int bytes, uint32_t voff,
                                             uint32_t soff) {
    if (bytes == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, soff, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 4, voff, soff, 0, 0);
  }
  // Weight loads: every weight byte is read once, and each load instruction
  // covers whole 128-byte lines; up to 16 rows they go with the non-temporal
  // policy (measured INT4 / FP8 gate_up M=1: 22.4 -> 21.5 / 34.0 -> 31.2 us;
  // at more rows it was slower for the split-K shapes).
  static constexpr int kWeightPolicy = MB == 1 ? 2 : 0;  // nt
  static __device__ __forceinline__ u32x4_t wload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kWeightPolicy));
  }
  static __device__ __forceinline__ u32x2_t wload8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
  }
};

// Steps t = r mod R among steps lo .. hi (may be negative).
constexpr int tm_steps_mod(int lo, int hi, int R, int r = 0) {
  int n = 0;
  for (int t = lo; t <= hi; ++t) n += (((t % R) + R) % R) == r;
  return n;
}

// KS (INT4, exact dequantisation): the waves pair up on the K16 steps of
// their tiles.  Wave w takes tile set w/2 (tiles w/2, w/2 + NW/2, ...) and
// K half w%2 (steps 2(w%2), 2(w%2)+1 of every chunk): each wave reads half of
// a chunk's X fragments from LDS and dequantises half of each of its tiles,
// and the two halves of a set run on different SIMDs.  The K-half-1 partial
// sums are added to the K-half-0 ones through LDS at the end.
// Fused SiLU-and-mul store of a tile group (a.silu_mul, INT4 gate_up with
// rows interleaved in 16-row blocks, so tile 2k holds gate rows and tile
// 2k + 1 the matching up rows; the plan keeps groups at an even tile count
// from an even first tile).  Every wave puts its final tile values into the
// freed X buffers at the tile's local index, then the owner of each gate
// tile reads the up values of the same (row, column) from the next local
// tile and stores bf16(g * sigmoid(g) * u), g and u rounded to bf16 first as
// the reference's unfused sequence does (hydraserve/model/runtime.py:1202-1210,
// silu_and_mul at hydraserve/kernels/activation.py:66-76), into y [M, N/2].
template <int MB, int TW, int NG>
__device__ __forceinline__ void tiled_silu_store(const GemmArgs& a, uint8_t* lds, const f32x4_t (&v)[TW][MB],
                                                 const int (&tt)[TW], int nto, int kg, int lane) {
  const int n = lane & 15, p4 = lane >> 4;
  f32x4_t* st = reinterpret_cast<f32x4_t*>(lds);
  __syncthreads();  // every wave is done with the X buffers
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    if (i >= nto) continue;
#pragma unroll
    for (int b = 0; b < MB; ++b) st[((kg + NG * i) * MB + b) * 64 + lane] = v[i][b];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    if (i >= nto || (tt[i] & 1) != 0) continue;
    const int col = 8 * tt[i] + n;  // output column 16 (tt / 2) + n
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const f32x4_t up = st[((kg + NG * i + 1) * MB + b) * 64 + lane];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int m = 16 * b + 4 * p4 + e2;
        if (m < a.M) {
          const float gv = bf16_to_f32(to_bf16_bits(v[i][b][e2]));
          const float uv = bf16_to_f32(to_bf16_bits(up[e2]));
          const float sig = 1.0f / (1.0f + expf(-gv));
          a.y[static_cast<int64_t>(m) * a.ldy + col] = to_bf16_bits(gv * sig * uv);
        }
      }
    }
  }
}

template <int WT, int SDT, int MB, int TW, int NW, bool KS = false>
__global__ __launch_bounds__(64 * NW, 1) void qgemm_tiled_kernel(GemmArgs a) {
  using C = Tm<WT, MB, TW, NW>;
  constexpr int D = C::D;
  constexpr int LPT = C::LPT;
  static_assert(!KS || (WT == W_INT4 && MB > 2 && NW % 2 == 0), "K halves: INT4 exact instances");
  constexpr int NG = KS ? NW / 2 : NW;  // tile sets
  __shared__ typename C::Smem sm;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = KS ? (wave >> 1) : wave;  // tile set
  const int kh = KS ? (wave & 1) : 0;      // K half
  const int lane = tid & 63, n = lane & 15, p4 = lane >> 4;
  const int NC = a.K >> 7;
  const int NT = a.N >> 4;
  const int g = blockIdx.x / a.splits, sp = blockIdx.x - g * a.splits;
  const int t0 = g * a.tpw;
  const int nt = (NT - t0) < a.tpw ? (NT - t0) : a.tpw;       // tiles of the group
  const int ntw = nt > kg ? (nt - kg + NG - 1) / NG : 0;      // of this wave (uniform)
  const int c0 = sp * a.cps;
  const int nk = (NC - c0) < a.cps ? (NC - c0) : a.cps;
  if (nt <= 0 || nk <= 0) return;

  TmRsrc rs;
  rs.x = make_rsrc(a.x, (static_cast<int64_t>(a.M - 1) * a.ldx + a.K) * 2);
  rs.w = make_rsrc(a.wtiles, static_cast<int64_t>(NT) * NC * C::TB);
  // FP8 instances read the scale dtype at run time.
  const int ses = WT == W_INT4 ? (SDT == SCALE_F32 ? 4 : 2) : (a.sdt == SCALE_F32 ? 4 : 2);
  const int64_t s_rows = WT == W_INT4 ? a.N : (a.N + 127) / 128;
  rs.s = make_rsrc(a.scale, (((s_rows - 1) * a.lds + ((a.K + 127) >> 7)) * ses + 3) & ~int64_t(3));
  rs.z = WT == W_INT4 ? make_rsrc(a.zero, ((static_cast<int64_t>(a.N + 7) >> 3) * a.ldz) * 4) : rs.w;

  // X load q of a round is the round's 1 KiB X load idx = wave + NW*q:
  // chunk idx / XI of the round, LDS bytes (idx % XI)*1024 + 16*lane of that
  // chunk's X, i.e. row r, K segment ((byte >> 4) & 15) ^ (r & 15).  Lanes of
  // rows at or past M read out of the buffer's range (no memory access; their
  // LDS bytes only reach output rows that are never stored).  Loads past the
  // round's X go to the junk area, entirely out of range, so every wave
  // issues LXR loads per round with no branches, which keeps the compiler's
  // count of loads in flight exact.
  constexpr uint32_t kOut = 0x80000000u;
  uint32_t xo[C::LXR];
  uint32_t xl[C::LXR];  // LDS byte offset of the load inside the X round (or ~0: junk)
#pragma unroll
  for (int q = 0; q < C::LXR; ++q) {
    const int idx = wave + NW * q;
    const int cr = idx / C::XI, blk = idx - cr * C::XI;
    const int b = 1024 * blk + 16 * lane;
    const int r = b >> 8;
    const int seg = ((b >> 4) & 15) ^ (r & 15);
    const bool on = idx < C::R * C::XI && r < a.M;
    xo[q] = on ? static_cast<uint32_t>(r * static_cast<uint32_t>(a.ldx) * 2u + cr * 256 + seg * 16) : kOut;
    xl[q] = idx < C::R * C::XI ? static_cast<uint32_t>(cr * C::XB + 1024 * blk) : 0xFFFFFFFFu;
  }
  // The wave's tiles; missing ones repeat tile t0 (loaded, never used).
  int tt[TW];
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    const int j = kg + NG * i;
    tt[i] = t0 + (j < nt ? j : 0);
  }
  // Weight byte offset of the lane's 16-byte load h of tile i at chunk 0.
  // INT4: row n, bytes 16p .. +16 (K 32p + 8s + e at step s), at 64n + 16p of
  // the tile.  FP8: row n, bytes 64h + 16p .. +16 (K 64(s/2) + 16p + 8(s%2)
  // + e at step s), stored at 1024h + 16 lane of the tile, so each of the two
  // loads reads one contiguous KiB.
  uint32_t wo[TW][LPT];
#pragma unroll
  for (int i = 0; i < TW; ++i)
#pragma unroll
    for (int h = 0; h < LPT; ++h) {
      // (KS: the K half's 8 bytes, words 2kh and 2kh+1)
      const uint32_t inner = WT == W_INT4 ? static_cast<uint32_t>(64 * n + 16 * p4 + 8 * kh)
                                          : static_cast<uint32_t>(1024 * h + 16 * lane);
      wo[i][h] = static_cast<uint32_t>(tt[i]) * C::TB + inner;
    }
  // Scale / zero-point source of lane 16i + n (tile i of the wave, row n) at chunk 0.
  const int li = (lane >> 4) < TW ? (lane >> 4) : TW - 1;
  int64_t se0;
  if constexpr (WT == W_INT4) se0 = static_cast<int64_t>(16 * tt[li] + n) * a.lds;
  else se0 = static_cast<int64_t>((16 * tt[li]) >> 7) * a.lds;
  // INT4 round loads (lane l, chunks c .. c+7 of a round at c = 0 mod 8):
  // scales of tile li, row n, 16 bytes per lane per 16-byte half (fp32: two
  // halves of four chunks); zero-point words of tile l/4, word row
  // (l/2) % 2 (tile rows 8h .. 8h+7), chunks 4 (l % 2) .. +3.
  const int zt = (lane >> 2) < TW ? (lane >> 2) : TW - 1;
  const uint32_t so0 = WT == W_INT4 ? static_cast<uint32_t>(se0 * ses) : 0u;
  const uint32_t zo0 = WT == W_INT4 ? static_cast<uint32_t>((2 * tt[zt] + ((lane >> 1) & 1)) * a.ldz) * 4u +
                                          static_cast<uint32_t>(lane & 1) * 16u
                                    : 0u;

  // INT4 group rewrite (128 + q as bf16, one v_and_or_b32 per two weights)
  // where the per-element correction stays cheaper than exact dequantisation.
  constexpr bool REW = WT == W_INT4 && MB <= 2;
  const uint32_t nib_mask = opaque_and(0x000F000Fu, 0xFFFFFFFFu);
  const uint32_t magic = opaque_and(0x64006400u, 0xFFFFFFFFu);
  const uint32_t magic_bf = opaque_and(0x43004300u, 0xFFFFFFFFu);
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

  f32x4_t acc[TW][MB];
#pragma unroll
  for (int i = 0; i < TW; ++i)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[i][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // The chunk loop for a wave with NTW real tiles (NTW uniform per wave):
  // no dummy tiles are loaded or computed, and the loop body has no branches,
  // so the compiler's own load-wait tracking stays exact across iterations.
  // A wave's vmcnt counts only its own loads, so waves with different NTW
  // (different loads per chunk) still meet at the same barriers.
  auto run = [&](auto ntc) __attribute__((always_inline)) {
    constexpr int NTW = decltype(ntc)::value;
    constexpr int R = C::R;
    // loads per wave per chunk: scales, (INT4) zero points, weights
    constexpr int Lc = (NTW > 0 && WT != W_INT4 ? 1 : 0) + NTW * LPT;
    // INT4 round loads (scales, zero points) of a wave, issued with the
    // weights of the round's first chunk.
    constexpr int Lm = WT == W_INT4 && NTW > 0 ? (SDT == SCALE_F32 ? 3 : 2) : 0;
    using WV = std::conditional_t<KS, u32x2_t, u32x4_t>;
    WV W[D][NTW > 0 ? NTW : 1][LPT];  // weight ring (registers)

    // X of round rho (chunks rho*R ..) into X buffer rho % 2; rounds past the
    // range read harmless in-range or out-of-range bytes that nothing uses.
    auto issue_x = [&](int rho) __attribute__((always_inline)) {
      uint8_t* base = &sm.xs[rho & 1][0];
      const int cf = c0 + (rho < 0 ? 0 : rho) * R;
      const uint32_t kx = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(cf) * 256u);
#pragma unroll
      for (int q = 0; q < C::LXR; ++q)
        C::dma(rs.x, (rho < 0 || xl[q] == 0xFFFFFFFFu) ? sm.junk : base + xl[q], 16, rho < 0 ? kOut : xo[q], kx);
    };
    // Scales, zero points and weights of chunk k (clamped) into ring slot J.
    // (J is a constant once the loops below are unrolled, so W[J] stays in
    // registers.)
    auto issue = [&](int J, int k) __attribute__((always_inline)) {
      if constexpr (NTW > 0) {
        if constexpr (WT == W_INT4) {
          if (J == 0) {
            // the round of chunks k .. k+7 (k = 0 mod 8; unclamped: a round
            // past the range reads bytes nobody uses)
            uint8_t* mb = &sm.meta[0] + ((k >> 3) & 1) * (NW * C::MSB) + wave * C::MSB;
            const uint32_t cs = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(c0 + k) * ses);
            C::dma(rs.s, mb, 16, so0, cs);
            if constexpr (SDT == SCALE_F32) C::dma(rs.s, mb + 1024, 16, so0 + 16u, cs);
            C::dma(rs.z, mb + 2048, 16, zo0, __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(c0 + k) * 4u));
          }
        }
        k = k < nk ? k : nk - 1;
        const int c = c0 + k;
        if constexpr (WT != W_INT4) {
          const uint32_t sb = static_cast<uint32_t>((se0 + c) * ses) & ~3u;
          C::dma(rs.s, &sm.ring[J][0] + wave * 256, 4, sb, 0);
        }
        const uint32_t kw = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(c) * static_cast<uint32_t>(NT) * C::TB);
#pragma unroll
        for (int i = 0; i < NTW; ++i)
#pragma unroll
          for (int h = 0; h < LPT; ++h) {
            if constexpr (KS) W[J][i][h] = C::wload8(rs.w, wo[i][h], kw);
            else W[J][i][h] = C::wload(rs.w, wo[i][h], kw);
          }
      }
    };

    // Chunk k from ring slot J.
    auto compute = [&](int J, int k) __attribute__((always_inline)) {
      if constexpr (NTW > 0) {
        const uint8_t* xchunk = &sm.xs[(k / R) & 1][0] + (J % R) * C::XB;
        const int c = c0 + k;
        uint32_t sd[NTW], zd[NTW];
        if constexpr (WT == W_INT4) {
          // chunk k = J mod 8 of its round
          const uint8_t* mb = &sm.meta[0] + ((k >> 3) & 1) * (NW * C::MSB) + wave * C::MSB;
#pragma unroll
          for (int i = 0; i < NTW; ++i) {
            if constexpr (SDT == SCALE_F32)
              sd[i] = *reinterpret_cast<const uint32_t*>(mb + (J >> 2) * 1024 + (16 * i + n) * 16 + (J & 3) * 4);
            else
              sd[i] = *reinterpret_cast<const uint16_t*>(mb + (16 * i + n) * 16 + J * 2);
            zd[i] = *reinterpret_cast<const uint32_t*>(mb + 2048 + 16 * (4 * i + 2 * (n >> 3) + (J >> 2)) + 4 * (J & 3));
          }
        } else {
          const uint8_t* sbase = &sm.ring[J][0] + wave * 256;
#pragma unroll
          for (int i = 0; i < NTW; ++i) {
            sd[i] = *reinterpret_cast<const uint32_t*>(sbase + (16 * i) * 4);
            zd[i] = 0u;
          }
        }
        constexpr int NST = KS ? 2 : 4;  // K16 steps of this wave per chunk
        bf16x8_t A[MB][NST];
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
          for (int st = 0; st < NST; ++st) {
            const int gseg = WT == W_INT4 ? 4 * p4 + (KS ? 2 * kh : 0) + st : 8 * (st >> 1) + 2 * p4 + (st & 1);
            A[b][st] = __builtin_bit_cast(
                bf16x8_t, *reinterpret_cast<const u32x4_t*>(xchunk + (16 * b + n) * 256 + ((gseg ^ n) * 16)));
          }
        // (all of the chunk's X fragments are read before the first use, so
        // their LDS latency is paid once per chunk)
        __builtin_amdgcn_sched_barrier(0);
        // Group rewrite: the per-row sums of X over the chunk, Xg, from an
        // all-ones MFMA (same layout as the results).
        f32x4_t xg[MB];
        if constexpr (REW) {
#pragma unroll
          for (int b = 0; b < MB; ++b) {
            xg[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st)
              xg[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[b][st], ones, xg[b], 0, 0, 0);
          }
        }
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
          const int t = tt[i];
          if constexpr (WT == W_INT4) {
            float s;
            if constexpr (SDT == SCALE_F32) s = __uint_as_float(sd[i]);
            else if constexpr (SDT == SCALE_BF16) s = __uint_as_float(sd[i] << 16);
            else s = __half2float(__ushort_as_half(static_cast<unsigned short>(sd[i])));
            const uint32_t z = (zd[i] >> ((n & 7) * 4)) & 0xFu;
            if constexpr (REW) {
              // acc += s * (sum x (128+q) - (128+z) * Xg)
              f32x4_t T[MB];
#pragma unroll
              for (int b = 0; b < MB; ++b) T[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int st = 0; st < 4; ++st) {
                const bf16x8_t B = int4_operand(W[J][i][0][st], nib_mask, magic_bf);
#pragma unroll
                for (int b = 0; b < MB; ++b)
                  T[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[b][st], B, T[b], 0, 0, 0);
              }
              const float zc = static_cast<float>(128u + z);
#pragma unroll
              for (int b = 0; b < MB; ++b)
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2)
                  acc[i][b][e2] = __builtin_fmaf(s, __builtin_fmaf(-zc, xg[b][e2], T[b][e2]), acc[i][b][e2]);
            } else {
              // exact: bf16_rne((q - z) * s), fp16 1024+q through v_fma_mix
              const float zp = static_cast<float>(1024u + z);
              const float cc = SDT == SCALE_F32 ? zp : -(zp * s);
#pragma unroll
              for (int st = 0; st < NST; ++st) {
                typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
                const uint32_t w = W[J][i][0][st];
                float f[8];
#pragma unroll
                for (int sh = 0; sh < 4; ++sh) {
                  const f16x2_t v = __builtin_bit_cast(f16x2_t, insert_nibbles(nib_mask, w >> (4 * sh), magic));
                  if constexpr (SDT == SCALE_F32) {
                    f[2 * sh] = (static_cast<float>(v[0]) - cc) * s;
                    f[2 * sh + 1] = (static_cast<float>(v[1]) - cc) * s;
                  } else {
                    f[2 * sh] = __builtin_fmaf(static_cast<float>(v[0]), s, cc);
                    f[2 * sh + 1] = __builtin_fmaf(static_cast<float>(v[1]), s, cc);
                  }
                }
                u32x4_t pb;
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) pb[e2] = pack_bf16x2(f[2 * e2], f[2 * e2 + 1]);
                const bf16x8_t B = __builtin_bit_cast(bf16x8_t, pb);
#pragma unroll
                for (int b = 0; b < MB; ++b)
                  acc[i][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[b][st], B, acc[i][b], 0, 0, 0);
              }
            }
          } else {
            const int64_t e = static_cast<int64_t>((16 * t) >> 7) * a.lds + c;
            float s;
            if (a.sdt == SCALE_F32) s = __uint_as_float(sd[i]);
            else if (a.sdt == SCALE_BF16) s = __uint_as_float((sd[i] >> ((e & 1) * 16)) << 16);
            else s = __half2float(__ushort_as_half(static_cast<unsigned short>(sd[i] >> ((e & 1) * 16))));
            f32x4_t T[MB];
#pragma unroll
            for (int b = 0; b < MB; ++b) T[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) {
              const u32x4_t& q = W[J][i][st >> 1];
              const bf16x8_t B = fp8_operand(q[2 * (st & 1)], q[2 * (st & 1) + 1]);
#pragma unroll
              for (int b = 0; b < MB; ++b)
                T[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[b][st], B, T[b], 0, 0, 0);
            }
#pragma unroll
            for (int b = 0; b < MB; ++b)
#pragma unroll
              for (int e2 = 0; e2 < 4; ++e2) acc[i][b][e2] = __builtin_fmaf(T[b][e2], s, acc[i][b][e2]);
          }
        }
      }
    };

    // Step J of the unrolled ring (chunk k = k0 + J, k0 a multiple of D).
    // Loads are issued in a fixed order: at a round start (J % R == 0) the X
    // of the next round, then at every step the chunk D-1 ahead.  The wait
    // before the step leaves in flight exactly the loads issued after the ones
    // it needs: chunk k's group, and at a round start also this round's X.
    auto step = [&](auto jc, int k) __attribute__((always_inline)) {
      constexpr int J = decltype(jc)::value;
      // (X rounds start at steps t = 0 mod R; INT4 round loads go out at
      // steps t = 1 mod D, with the weights of chunk t + D - 1 = 0 mod D.)
      constexpr int after_g = (D - 2) * Lc + C::LXR * tm_steps_mod(J - D + 2, J - 1, R) +
                              Lm * tm_steps_mod(J - D + 2, J - 1, D, 1);
      constexpr int after_x = R * Lc + Lm * tm_steps_mod(J - R, J - 1, D, 1);
      constexpr int later = (J % R == 0 && after_x < after_g) ? after_x : after_g;
      static_assert(later <= 63, "vmcnt range");
      __builtin_amdgcn_s_waitcnt((later & 15) | ((later >> 4) << 14) | 0x0F70);
      if constexpr (J % R == 0) {
        // This round's X (every wave's share) has landed, and every wave is
        // done with the previous round, whose buffer takes the next round.
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue_x(k / R + 1);
      }
      issue((J + D - 1) % D, k + D - 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(J, k);
      __builtin_amdgcn_sched_barrier(0);
    };

    // Prologue: the loads of steps -(D-1) .. -1 in steady-state order (X
    // rounds before round 0 carry no data).
#pragma unroll
    for (int t = -(D - 1); t < 0; ++t) {
      if (((t % R) + R) % R == 0) issue_x(t / R + 1);
      issue(t + D - 1, t + D - 1);
    }
    int k0 = 0;
    // Whole rounds of the ring: no branch inside the loop body.
    for (; k0 + D <= nk; k0 += D) {
#define HS_TM_STEP(J) if constexpr ((J) < D) step(std::integral_constant<int, (J)>{}, k0 + (J));
      HS_TM_STEP(0) HS_TM_STEP(1) HS_TM_STEP(2) HS_TM_STEP(3) HS_TM_STEP(4) HS_TM_STEP(5) HS_TM_STEP(6) HS_TM_STEP(7)
    }
    // The remaining chunks (fewer than D), after the loop.
#define HS_TM_REST(J) if constexpr ((J) < D - 1) { if (k0 + (J) < nk) step(std::integral_constant<int, (J)>{}, k0 + (J)); }
    HS_TM_REST(0) HS_TM_REST(1) HS_TM_REST(2) HS_TM_REST(3) HS_TM_REST(4) HS_TM_REST(5) HS_TM_REST(6)
#undef HS_TM_STEP
#undef HS_TM_REST
  };
  if (ntw >= TW) run(std::integral_constant<int, TW>{});
  else if (TW >= 3 && ntw == 2) run(std::integral_constant<int, (TW >= 3 ? 2 : 0)>{});
  else if (ntw == 1) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 0>{});
  // Drain the clamped prefetches before any exit.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  // K halves: half 1 hands its sums to half 0 of the same tile set, which
  // adds them (half 0 + half 1, a fixed order) and stores the tiles.
  int nto = ntw;  // tiles this wave stores
  if constexpr (KS) {
    __syncthreads();  // every wave is done with the X buffers
    static_assert(NG * TW * MB * 64 * 16 <= 2 * C::XR, "K-half sums fit the X buffers");
    f32x4_t* red = reinterpret_cast<f32x4_t*>(&sm.xs[0][0]);
    if (kh == 1) {
#pragma unroll
      for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int b = 0; b < MB; ++b) red[((kg * TW + i) * MB + b) * 64 + lane] = acc[i][b];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[i][b] += red[((kg * TW + i) * MB + b) * 64 + lane];
    } else {
      nto = 0;
    }
  }

  static_assert(NG * TW * MB * 64 * 16 <= 2 * C::XR, "a group's final tiles fit the X buffers");
  // Lane (n, p4), register e of block (i, b): row 16b + 4p4 + e, column 16 tt[i] + n.
  if (a.splits == 1) {
    if constexpr (WT == W_INT4) {
      if (a.silu_mul) {
        tiled_silu_store<MB, TW, NG>(a, &sm.xs[0][0], acc, tt, nto, kg, lane);
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < TW; ++i) {
      if (i >= nto) continue;
      const int col = 16 * tt[i] + n;
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int m = 16 * b + 4 * p4 + e2;
          if (m < a.M) a.y[static_cast<int64_t>(m) * a.ldy + col] = to_bf16_bits(acc[i][b][e2]);
        }
    }
    return;
  }
  const auto pr = partial_rsrc(a.partials);
  auto poff = [&](int pp, int i, int b) __attribute__((always_inline)) {
    return static_cast<uint32_t>((static_cast<int64_t>(pp) * C::SLOT / 4 + ((wave * TW + i) * MB + b) * 64 + lane) *
                                 16);
  };
  // Only the tiles this wave stores travel (uniform branches per wave).
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    if (i >= nto) continue;
#pragma unroll
    for (int b = 0; b < MB; ++b) store_partial4(pr, poff(blockIdx.x, i, b), acc[i][b]);
  }
  if (!arrive_last(a.counters, g, a.splits, &sm.flag)) return;
  f32x4_t sum[TW][MB];
#pragma unroll
  for (int i = 0; i < TW; ++i)
#pragma unroll
    for (int b = 0; b < MB; ++b) sum[i][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Contributors in K-range order, up to four (three-tile waves at 64 rows:
  // two) with all loads in flight (every load is a coherent round trip); a
  // slot past the last contributor re-reads the last one and adds zero.
  constexpr int QF = TW * MB > 8 ? 2 : 4;
  for (int q0 = 0; q0 < a.splits; q0 += QF) {
    f32x4_t v[QF][TW][MB];
#pragma unroll
    for (int u = 0; u < QF; ++u) {
      const int q = q0 + u < a.splits ? q0 + u : a.splits - 1;
#pragma unroll
      for (int i = 0; i < TW; ++i) {
        if (i >= nto) continue;
#pragma unroll
        for (int b = 0; b < MB; ++b) v[u][i][b] = load_partial4(pr, poff(g * a.splits + q, i, b));
      }
    }
#pragma unroll
    for (int u = 0; u < QF; ++u) {
      const float keep = q0 + u < a.splits ? 1.0f : 0.0f;
#pragma unroll
      for (int i = 0; i < TW; ++i) {
        if (i >= nto) continue;
#pragma unroll
        for (int b = 0; b < MB; ++b) sum[i][b] += v[u][i][b] * keep;
      }
    }
  }
  bool fused = false;
  if constexpr (WT == W_INT4) {
    if (a.silu_mul) {
      tiled_silu_store<MB, TW, NG>(a, &sm.xs[0][0], sum, tt, nto, kg, lane);
      fused = true;
    }
  }
  if (!fused) {
#pragma unroll
    for (int i = 0; i < TW; ++i) {
      if (i >= nto) continue;
      const int col = 16 * tt[i] + n;
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int m = 16 * b + 4 * p4 + e2;
          if (m < a.M) a.y[static_cast<int64_t>(m) * a.ldy + col] = to_bf16_bits(sum[i][b][e2]);
        }
    }
  }
  reset_counter(a.counters, g);
}

// Layout: eight waves (two per SIMD, so one wave's dequantisation overlaps
// the other's MFMAs and LDS latencies) of up to 2 tiles; FP8 above 32 rows
// keeps four waves of up to 3 tiles (eight would spill registers).
// Experiment switch: HS_TM_NW4=1 keeps four waves of up to 3 tiles above 32 rows.
bool tm_nw4() {
  static const bool v = [] {
    const char* e = std::getenv("HS_TM_NW4");
    return e != nullptr && e[0] == '1';
  }();
  return v;
}

// INT4 at 33..64 rows with one K range per tile group pairs the waves on the
// K halves of their tiles (measured gate_up 34816x5120 M=64: 43.4 against
// 45.3 us; with split K ranges, where the halves' partial sums travel too,
// it was 3-10 % slower, so those keep one wave per tile).  HS_TM_KS=0 turns
// it off.
bool tm_ks() {
  static const bool v = [] {
    const char* e = std::getenv("HS_TM_KS");
    return !(e != nullptr && e[0] == '0');
  }();
  return v;
}
int tm_mb(int M) { return M <= 16 ? 1 : (M <= 32 ? 2 : 4); }
int tm_nw(int wt, int M) { return M <= 32 || (wt == W_INT4 && !tm_nw4()) ? 8 : 4; }
constexpr int kTmKsMaxTpw = 12;  // four tile sets of up to three tiles
bool tm_use_ks(int wt, const GemmArgs& a) {
  return wt == W_INT4 && a.M > 32 && tm_nw(wt, a.M) == 8 && tm_ks() && a.splits == 1 && a.tpw <= kTmKsMaxTpw;
}
int tm_tw(int wt, int M) { return tm_nw(wt, M) == 8 ? 2 : 3; }
int tm_max_tpw(int wt, int M) { return tm_nw(wt, M) * tm_tw(wt, M); }
int tm_slot_floats(int wt, int M) { return tm_nw(wt, M) * tm_tw(wt, M) * tm_mb(M) * 256; }

// Tiled copy present, M <= 64, N a multiple of 16, K a multiple of 128, every
// buffer range below 2^31 bytes; INT4 scale rows 4-byte aligned.
bool tiled_ok(const GemmArgs& a, int wt) {
  if (a.wtiles == nullptr || a.M <= 0 || a.M > 64 || a.N % 16 != 0 || a.K % 128 != 0 || !a.xvec) return false;
  // fused SiLU: INT4, gate/up 16-row blocks in tile pairs
  if (a.silu_mul && (wt != W_INT4 || a.N % 32 != 0)) return false;
  if ((reinterpret_cast<uintptr_t>(a.scale) & 3) != 0 || (reinterpret_cast<uintptr_t>(a.wtiles) & 15) != 0) return false;
  if (wt == W_INT4) {
    // a round's scales and zero points go by 16-byte loads from 4-byte
    // aligned addresses (16-bit scales: even row strides; K ranges start at
    // even chunks)
    const int ses = a.sdt == SCALE_F32 ? 4 : 2;
    if ((a.lds * ses) % 4 != 0 || (reinterpret_cast<uintptr_t>(a.zero) & 3) != 0) return false;
  }
  const int64_t lim = int64_t(1) << 31;
  const int64_t tb = static_cast<int64_t>(a.N) * a.K / (wt == W_INT4 ? 2 : 1);
  const int64_t xb = (static_cast<int64_t>(a.M) * a.ldx + a.K) * 2;
  return tb < lim && xb < lim;
}

template <int WT, int SDT, int MB, int TW, int NW, bool KS = false>
static hipError_t launch_tiled_t(const GemmArgs& a, hipStream_t stream) {
  const int groups = (a.N / 16 + a.tpw - 1) / a.tpw;
  hipLaunchKernelGGL((qgemm_tiled_kernel<WT, SDT, MB, TW, NW, KS>), dim3(groups * a.splits), dim3(64 * NW), 0, stream,
                     a);
  return hipGetLastError();
}

template <int WT, int SDT>
static hipError_t launch_tiled_s(const GemmArgs& a, hipStream_t stream) {
  const int mb = tm_mb(a.M);
  if (mb == 1) return launch_tiled_t<WT, SDT, 1, 2, 8>(a, stream);
  if (mb == 2) return launch_tiled_t<WT, SDT, 2, 2, 8>(a, stream);
  if constexpr (WT == W_INT4) {
    if (tm_use_ks(WT, a)) return launch_tiled_t<WT, SDT, 4, 3, 8, true>(a, stream);
    if (!tm_nw4()) return launch_tiled_t<WT, SDT, 4, 2, 8>(a, stream);
  }
  return launch_tiled_t<WT, SDT, 4, 3, 4>(a, stream);
}

hipError_t launch_tiled(int wt, const GemmArgs& a, hipStream_t stream) {
  if (a.tpw <= 0 || a.tpw > tm_max_tpw(wt, a.M) || a.splits <= 0 || a.cps <= 0) return hipErrorInvalidValue;
  if (a.silu_mul && (wt != W_INT4 || a.tpw % 2 != 0 || a.N % 32 != 0)) return hipErrorInvalidValue;
  if (wt == W_INT4) {
    if (a.sdt == SCALE_BF16) return launch_tiled_s<W_INT4, SCALE_BF16>(a, stream);
    if (a.sdt == SCALE_F16) return launch_tiled_s<W_INT4, SCALE_F16>(a, stream);
    return launch_tiled_s<W_INT4, SCALE_F32>(a, stream);
  }
  // FP8 reads its scale dtype at run time (one scale per tile and chunk).
  return launch_tiled_s<W_FP8, SCALE_F32>(a, stream);
}

}  // namespace hsq
