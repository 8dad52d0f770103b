// C ABI of libhydraserve_amd.so (declared in include/hydraserve_amd.h).
//
// Host-side validation mirrors the checks the reference performs in Python
// before its Triton launches (hydraserve/kernels/awq.py:28-43,
// hydraserve/kernels/fp8.py:28-62) and returns an error code instead of
// launching on malformed input.  The launch plan (regime, tile shape, stream-K
// grid, workspace size) is a pure function of (kind, M, N, K, CU count), so
// hs_gemm_workspace_bytes and the GEMM entry points always agree.
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "qgemm_common.h"
#include "../../include/hydraserve_amd.h"

namespace hsq {
hipError_t launch_decode(int wt, const GemmArgs& a, int MT, int S, hipStream_t stream);
hipError_t launch_prefill(int wt, const GemmArgs& a, int BM, hipStream_t stream);
int decode_slot_floats(int MT, int S);
hipError_t launch_stream(int wt, const GemmArgs& a, int MT, int S, hipStream_t stream);
int stream_slot_floats(int MT, int S);
bool stream_ok(const GemmArgs& a, int wt, int NB);
bool decode_kfull(int K, int xvec, int wvec);
int prefill_slot_floats(int BM);
hipError_t launch_wide(int wt, const GemmArgs& a, hipStream_t stream);
hipError_t launch_mid(int wt, const GemmArgs& a, int bmi, int nj, int nw, hipStream_t stream);
int mid_slot_floats(int bmi, int nj, int nw);
bool mid_ok(const GemmArgs& a, int wt);
int wide_slot_floats();
bool wide_ok(const GemmArgs& a, int wt);
bool wide_tiles_ok(const GemmArgs& a, int wt);
bool rows_ok(const GemmArgs& a, int wt, int P, int* nblk_out, bool* xl_out, int* ms_out, int xl_pref);
hipError_t launch_rows(int wt, const GemmArgs& a, int nblk, bool xl, int ms, hipStream_t stream);
extern int rows_kw8;
bool gemv_ok(const GemmArgs& a, int wt, int P, int kw_pref, int* kw_out, int* rows_max);
hipError_t launch_gemv(int wt, const GemmArgs& a, int kw, hipStream_t stream);
extern int gemv_rd;
bool skinny_ok(const GemmArgs& a, int wt, int kc);
bool tiled_ok(const GemmArgs& a, int wt);
hipError_t launch_tiled(int wt, const GemmArgs& a, hipStream_t stream);
int tm_slot_floats(int wt, int M);
int tm_max_tpw(int wt, int M);
hipError_t launch_skinny(int wt, const GemmArgs& a, int s, int nb, int kc, bool xd, hipStream_t stream);
int skinny_slot_floats(int mt, int s, int nb);
int skinny_bt(int s, int nb);
int skinny_max_units(int s, int nb, int kc);
bool skinny_fits(int wt, int m, int s, int nb, int kc, bool xd);
hipError_t launch_int4_dequant(const uint32_t* packed, int64_t ldw, const void* scale, int64_t lds, int sdt,
                               const int32_t* zero, int64_t ldz, void* out, int64_t ldo, int odt, int N, int K,
                               int group, hipStream_t stream);
hipError_t launch_fp8_dequant(const uint8_t* w, int64_t ldw, const void* scale, int64_t lds, int sdt, void* out,
                              int64_t ldo, int odt, int N, int K, hipStream_t stream);

namespace {

constexpr int kMaxDevices = 64;
constexpr int kDecodeMaxM = 64;
// Arrival counters live at a fixed offset and size in every workspace, so the
// region never overlaps the (dirty) partial tiles of a call with another shape.
constexpr int64_t kMaxTiles = 1 << 18;
constexpr int64_t kCounterBytes = kMaxTiles * 4;

struct Tuning {
  int rows_off = 0;        // 1: never use the row-partitioned decode kernel
  int rows_wg = 0;         // its workgroups per CU (0 = 1)
  int rows_xl = 1;         // 0: never stage X in LDS (read A fragments from global memory)
  int rows_force = 0;      // 1: use it whenever it can run
  int gemv_off = 0;        // 1: never use the block-major kernel
  int gemv_kw = 0;         // its wavefronts per workgroup (0 = 8)
  int gemv_wg = 0;         // its workgroups per CU (0 = 1)
  int st_off = 0;          // 1: never use the streaming decode kernel
  int st_s = 0;            // its strips of 16 rows per wave (0 = heuristic)
  int st_wg = 0;           // its workgroups per CU
  int st_nb = 0;           // its chunks per batch (0 = heuristic)
  int decode_s = 0;        // strips of 16 rows per wave (0 = heuristic)
  int decode_wg_per_cu = 0;
  int prefill_bm = 0;
  int wide_off = 0;         // 1: never use the 256x256-tile prefill kernel
  int wide_min_m = 0;      // smallest M for it (0 = 129)
  int wide_tiles_off = 0;  // 1: it reads the row-major weight even when a tiled copy is given
  int tune = 0;            // GemmArgs::tune experiment bits
  int mid_off = 0;         // 1: never use the LDS-DMA streaming kernel for 17..64 rows
  int mid_min_m = 0;       // smallest M for it (0 = 17)
  int mid_nj = 0;          // its 32-column blocks per wave (0 = heuristic)
  int rows_ms2_off = 0;    // 1: the row-partitioned kernel only up to 16 rows
  int prefill_wg_per_cu = 0;
  int skinny = 0;          // register-streamed decode kernel: 0 = where measured faster, 1 = always (M <= 64), 2 = never
  int skinny_layout = -1;  // its (S, NB, KC) layout index (-1 = heuristic)
  int skinny_wg = 0;       // its workgroups per CU (0 = 1)
  int skinny_xd = -1;      // its largest M loading X fragments per wave (-1 = none)
  int row_split_off = 0;   // 1: no two-pass row split at 129..256 rows on narrow outputs
  int tm_off = 0;          // 1: never use the tiled decode kernel
  int tm_min_m = 0;        // smallest M for it (0 = default)
  int tm_tpw = 0;          // its tiles per workgroup (0 = heuristic)
  int tm_s = 0;            // its K ranges (0 = heuristic)
};

int env_int(const char* name) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : 0;
}

// Optional overrides for tuning sweeps, read once per process.
const Tuning& tuning() {
  static Tuning t = [] {
    Tuning r;
    r.rows_off = env_int("HS_ROWS_OFF");
    r.rows_wg = env_int("HS_ROWS_WG");
    if (std::getenv("HS_ROWS_XL") != nullptr) r.rows_xl = env_int("HS_ROWS_XL");
    r.rows_force = env_int("HS_ROWS_FORCE");
    rows_kw8 = env_int("HS_ROWS_KW8");
    r.gemv_off = env_int("HS_GEMV_OFF");
    r.gemv_kw = env_int("HS_GEMV_KW");
    r.gemv_wg = env_int("HS_GEMV_WG");
    gemv_rd = env_int("HS_GEMV_RD");
    r.st_off = env_int("HS_ST_OFF");
    r.st_s = env_int("HS_ST_S");
    r.st_wg = env_int("HS_ST_WG");
    r.st_nb = env_int("HS_ST_NB");
    r.decode_s = env_int("HS_DECODE_S");
    r.decode_wg_per_cu = env_int("HS_DECODE_WG_PER_CU");
    r.prefill_bm = env_int("HS_PREFILL_BM");
    r.wide_off = env_int("HS_WIDE_OFF");
    r.wide_min_m = env_int("HS_WIDE_MIN_M");
    r.wide_tiles_off = env_int("HS_WIDE_TILES_OFF");
    r.tune = env_int("HS_TUNE");
    r.mid_off = env_int("HS_MID_OFF");
    r.mid_min_m = env_int("HS_MID_MIN_M");
    r.mid_nj = env_int("HS_MID_NJ");
    r.rows_ms2_off = env_int("HS_ROWS_MS2_OFF");
    r.prefill_wg_per_cu = env_int("HS_PREFILL_WG_PER_CU");
    r.skinny = env_int("HS_SKINNY");
    if (std::getenv("HS_SKINNY_LAYOUT") != nullptr) r.skinny_layout = env_int("HS_SKINNY_LAYOUT");
    r.skinny_wg = env_int("HS_SKINNY_WG");
    if (std::getenv("HS_SKINNY_XD") != nullptr) r.skinny_xd = env_int("HS_SKINNY_XD");
    r.row_split_off = env_int("HS_ROW_SPLIT_OFF");
    r.tm_off = env_int("HS_TM_OFF");
    r.tm_min_m = env_int("HS_TM_MIN_M");
    r.tm_tpw = env_int("HS_TM_TPW");
    r.tm_s = env_int("HS_TM_S");
    return r;
  }();
  return t;
}

int device_cus() {
  static int cus[kMaxDevices] = {0};
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

struct Plan {
  bool stream = false;  // streaming decode kernel (fast path)
  bool decode = true;
  bool wide = false;    // 256x256-tile prefill kernel
  bool mid = false;     // LDS-DMA streaming kernel, 32-row MFMA blocks
  bool skinny = false;  // register-streamed decode kernel
  int SS = 1, SNB = 2, SKC = 4;
  int BMI = 1, NJ = 1, NW = 4;
  int MT = 1, S = 1, BM = 256, NB = 1;
  int T = 0, TM = 1, G = 0;
  int64_t U = 0;
  int P = 0;
  int64_t slot_floats = 0;
  int64_t counter_bytes = 0;
  int64_t ws_bytes = 0;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int stream_nb(int M) { return M <= 16 ? 8 : (M <= 32 ? 4 : 2); }

// Tiled decode kernel: tile groups of `tpw` 16-row tiles over `splits` K
// ranges of `cps` chunks, one workgroup each, at most one per CU.  The
// estimate per chunk step is the larger of the CU's HBM bytes (its tiles plus
// a share for the X chunk, an L2 hit) and the busiest wave's dequant + MFMA
// work in byte equivalents; split groups add a settle.
struct TmPlan {
  int tpw = 0, splits = 0, cps = 0, P = 0;
  int64_t ws_bytes = 0;
};

// silu: the fused SiLU store pairs tiles 2k and 2k+1 inside one group, so
// groups hold an even number of tiles.
TmPlan tm_plan(int wt, int M, int N, int K, bool silu = false) {
  TmPlan best;
  const int cus = device_cus();
  const Tuning& tn = tuning();
  const int64_t NT = N / 16, NC = K / 128;
  const int mb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const double tb = wt == W_INT4 ? 1024.0 : 2048.0;
  // per-SIMD compute of one tile and chunk, in the units of the memory term:
  // INT4 at 33..64 rows dequantises exactly and runs four MFMA row blocks
  // (measured at 64 rows: down 17408->5120 31.8 us at 6 K ranges of 8-tile
  // groups against 33.7 at 8 of 10-tile groups, whose busiest SIMD holds 3)
  const double comp = wt == W_INT4 ? (mb >= 4 ? 8000.0 : 2600.0) : 1000.0 + 250.0 * mb;
  double best_est = 1e30;
  const int cand[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32};
  for (int s0 : cand) {
    if (tn.tm_s > 0 && s0 != tn.tm_s) continue;
    if (s0 > NC) break;
    // INT4 K ranges start at even chunks (4-byte aligned 16-bit scale loads)
    const int cps = wt == W_INT4 ? static_cast<int>(2 * cdiv(cdiv(NC, s0), 2)) : static_cast<int>(cdiv(NC, s0));
    const int S = static_cast<int>(cdiv(NC, cps));
    int tpw = tn.tm_tpw > 0 ? tn.tm_tpw : static_cast<int>(cdiv(NT * S, cus));
    if (tpw < 1) tpw = 1;
    if (silu && tpw % 2 != 0) {
      if (tn.tm_tpw > 0) continue;
      ++tpw;
    }
    if (tpw > tm_max_tpw(wt, M)) continue;
    const int64_t groups = cdiv(NT, tpw);
    const int64_t P = groups * S;
    if (P > 4 * cus || groups > kMaxTiles) continue;
    const double waves_per_cu = P > cus ? static_cast<double>(cdiv(P, cus)) : 1.0;
    const int tw = (tpw + 3) / 4;  // tiles per SIMD
    // At one row block a wave streams its tiles at ~1/6 of what the
    // workgroup's eight waves stream together, so the busiest wave's tile
    // count bounds the workgroup's pace too, and each K range pays its ring
    // fill (~3 INT4 / 2 FP8 chunks) once.  Fitted to the best of a measured
    // sweep at 1..16 rows: down 17408->5120 at 6 K ranges of 8-tile groups
    // (INT4 15.8-16.1 us against 16.7-17.0 at 8 ranges of 10-tile groups,
    // where two waves hold two tiles); qkv 5120->10240 INT4 at 3 ranges, 12.2
    // against 13.6 us at 5 ranges of 8 chunks.
    double wbytes = tpw * tb;
    double fill = 0.0;
    if (mb == 1) {
      const double wave_bound = ((tpw + 7) / 8) * 6.0 * tb;
      wbytes = wave_bound > wbytes ? wave_bound : wbytes;
      fill = wt == W_INT4 ? 3.0 : 2.0;
    }
    const double mem = wbytes + 0.5 * mb * 4096.0;
    const double cmp = tw * comp;
    // a split group settles after its last K range: partial stores, the
    // arrival, then coherent loads of four contributors per round trip; the
    // partials grow with the row blocks (measured at 64 rows: o_proj
    // 8192->5120 19.2 us at 4 K ranges against 22.9 at 8)
    const double settle = S > 1 ? (30000.0 + 20000.0 * ((S + 3) / 4)) * mb : 0.0;
    const double est = waves_per_cu * (cps + fill) * (mem > cmp ? mem : cmp) + settle;
    if (est < best_est) {
      best_est = est;
      best.tpw = tpw;
      best.splits = S;
      best.cps = cps;
      best.P = static_cast<int>(P);
    }
  }
  if (best.P > 0)
    best.ws_bytes = kCounterBytes + static_cast<int64_t>(best.P) * tm_slot_floats(wt, M) * 4;
  return best;
}

// Measured on MI355X (gate_up 5120->34816, down 17408->5120, qkv): with the
// scale rounds the tiled kernel is faster at every row count for INT4 too
// (gate_up M=1 / 4: 22.8 / 21.8 us against 28.3 / 26.2 on the row-major
// kernels; down M=1 / 4: 16.7 / 16.7 against 19.8 / 21.5).
// Small weights stay row-major: the tiled kernel's ring fill and drain cost
// ~5 us a launch (INT4 4096x4096 at M=8: 9.2 vs 7.7 us).
bool tm_min_ok(int wt, int M, int N, int K) {
  const Tuning& tn = tuning();
  if (tn.tm_off) return false;
  if (tn.tm_min_m > 0) return M >= tn.tm_min_m;
  (void)wt;
  return M >= 1 && static_cast<int64_t>(N) * K >= (int64_t{32} << 20);
}

// Register-streamed decode kernel layouts: S 16-row blocks per wave, NB
// block groups, KC K phases (NB * KC = 8 wavefronts).
struct SkinnyLayout {
  int s, nb, kc;
};
constexpr SkinnyLayout kSkinnyLayouts[] = {{1, 2, 4}, {1, 4, 2}, {2, 2, 4}, {1, 8, 1}, {2, 4, 2}, {2, 1, 8}};
constexpr int kSkinnyLayoutCount = 6;

bool skinny_xd(int M) {
  const Tuning& tn = tuning();
  return M <= (tn.skinny_xd >= 0 ? tn.skinny_xd : 0);
}

SkinnyLayout skinny_layout(int wt, int M, int K) {
  const Tuning& tn = tuning();
  int i = tn.skinny_layout;
  // Measured on MI355X (17408 -> 5120, 8192 -> 5120): two row blocks per
  // wave over four K phases up to 16 rows (INT4), one 128-row tile over one
  // phase above.
  if (i < 0 || i >= kSkinnyLayoutCount) i = (wt == W_INT4 && M <= 16) ? 2 : 3;
  const auto usable = [&](int j) {
    const SkinnyLayout& l = kSkinnyLayouts[j];
    return K % (128 * l.kc) == 0 && (l.s == 1 || M <= 32) && skinny_fits(wt, M, l.s, l.nb, l.kc, skinny_xd(M));
  };
  // Fall back to fewer K phases (or one row block per wave) when the layout
  // does not divide K or does not fit LDS.
  if (!usable(i)) i = 1;
  if (!usable(i)) i = 3;
  return kSkinnyLayouts[i];
}

// `fast`: the streaming kernel can run this problem (see stream_ok); `wide`:
// the 256x256-tile prefill kernel can (see wide_ok).
Plan make_plan(int wt, int M, int N, int K, bool kfull, bool fast, bool wide, bool mid, bool skinny) {
  Plan p;
  const int cus = device_cus();
  const Tuning& tn = tuning();
  if (skinny && M <= 64) {
    p.skinny = true;
    p.decode = false;
    const SkinnyLayout l = skinny_layout(wt, M, K);
    p.SS = l.s;
    p.SNB = l.nb;
    p.SKC = l.kc;
    p.T = static_cast<int>(cdiv(N, skinny_bt(p.SS, p.SNB)));
    p.G = K / (128 * p.SKC);
    p.U = static_cast<int64_t>(p.T) * p.G;
    int64_t wgs = static_cast<int64_t>(cus) * (tn.skinny_wg > 0 ? tn.skinny_wg : 1);
    // Each workgroup stages the scales of all its units in LDS: at most
    // skinny_max_units() of them.
    const int64_t need = cdiv(p.U, skinny_max_units(p.SS, p.SNB, p.SKC));
    wgs = wgs > need ? wgs : need;
    p.P = static_cast<int>(p.U < wgs ? p.U : wgs);
    p.slot_floats = skinny_slot_floats((M + 15) / 16, p.SS, p.SNB);
    p.counter_bytes = kCounterBytes;
    p.ws_bytes = p.counter_bytes + static_cast<int64_t>(p.P) * 2 * p.slot_floats * 4;
    return p;
  }
  if (mid && !tn.mid_off && M >= (tn.mid_min_m > 0 ? tn.mid_min_m : 17) && M <= 128) {
    p.mid = true;
    p.BMI = static_cast<int>(cdiv(M, 32));
    // Wide outputs: 256 weight rows per tile; narrow ones 128, so that
    // enough tiles exist and fewer of them are split across workgroups.
    p.NJ = tn.mid_nj == 1 || tn.mid_nj == 2 ? tn.mid_nj : (N >= 16384 ? 2 : 1);
    if ((wt != W_INT4 && p.BMI > 2) || p.BMI > 3) p.NJ = 1;
    p.NW = 4;
    p.T = static_cast<int>(cdiv(N, 32 * p.NJ * p.NW));
    p.G = K / 64;
    p.U = static_cast<int64_t>(p.T) * p.G;
    p.P = static_cast<int>(p.U < cus ? p.U : cus);
    p.slot_floats = mid_slot_floats(p.BMI, p.NJ, p.NW);
    p.counter_bytes = kCounterBytes;
    p.ws_bytes = p.counter_bytes + static_cast<int64_t>(p.P) * 2 * p.slot_floats * 4;
    return p;
  }
  if (M <= kDecodeMaxM && fast && !tn.st_off) {
    p.stream = true;
    p.MT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    int S = tn.st_s;
    // Above 16 rows, two 16-row strips per wave halve the activation re-reads
    // from LDS (measured INT4 34816x5120 at 64 rows: 137 -> 94 us); only FP8
    // on narrow outputs at up to 32 rows keeps one strip (31 vs 35 us).
    if (S != 1 && S != 2)
      S = (M > 16 && (wt == W_INT4 || M > 32 || N >= 2 * K)) ? 2 : 1;
    p.S = S;
    p.NB = tn.st_nb > 0 ? tn.st_nb : stream_nb(M);
    p.T = static_cast<int>(cdiv(N, 64 * S));
    p.G = K / (128 * p.NB);
    const int occ = tn.st_wg > 0 ? tn.st_wg : 1;
    p.U = static_cast<int64_t>(p.T) * p.G;
    const int64_t wgs = static_cast<int64_t>(cus) * occ;
    p.P = static_cast<int>(p.U < wgs ? p.U : wgs);
    p.slot_floats = stream_slot_floats(p.MT, S);
  } else if (M <= kDecodeMaxM) {
    p.decode = true;
    p.MT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    int S = tn.decode_s;
    if (S != 1 && S != 2 && S != 4) S = 1;
    p.S = S;
    p.T = static_cast<int>(cdiv(N, 64 * S));
    p.TM = 1;
    p.NB = kfull ? 4 : 1;
    p.G = static_cast<int>(cdiv(K, 128)) / p.NB;
    const int occ = tn.decode_wg_per_cu > 0 ? tn.decode_wg_per_cu : 4;
    p.U = static_cast<int64_t>(p.T) * p.G;
    p.P = static_cast<int>(p.U < static_cast<int64_t>(cus) * occ ? p.U : static_cast<int64_t>(cus) * occ);
    p.slot_floats = decode_slot_floats(p.MT, p.S);
  } else if (wide && !tn.wide_off && M >= (tn.wide_min_m > 0 ? tn.wide_min_m : 129)) {
    // With coherent 16-byte partial loads the 256x256 tiles win even where
    // few tiles exist and most are split (down 17408->5120 at 512 rows:
    // 139 us vs 218 us for 128-row tiles).
    p.decode = false;
    p.wide = true;
    p.TM = static_cast<int>(cdiv(M, 256));
    p.T = p.TM * static_cast<int>(cdiv(N, 256));
    p.G = K / 128;  // stream-K unit: one 128-K group
    p.U = static_cast<int64_t>(p.T) * p.G;
    p.P = static_cast<int>(p.U < cus ? p.U : cus);
    p.slot_floats = wide_slot_floats();
  } else {
    p.decode = false;
    int bm = tn.prefill_bm;
    if (bm != 64 && bm != 128 && bm != 256) bm = 128;
    p.BM = bm;
    p.TM = static_cast<int>(cdiv(M, bm));
    p.T = p.TM * static_cast<int>(cdiv(N, 256));
    p.G = static_cast<int>(cdiv(K, 64));
    const int occ = tn.prefill_wg_per_cu > 0 ? tn.prefill_wg_per_cu : 1;
    p.U = static_cast<int64_t>(p.T) * p.G;
    p.P = static_cast<int>(p.U < static_cast<int64_t>(cus) * occ ? p.U : static_cast<int64_t>(cus) * occ);
    p.slot_floats = prefill_slot_floats(bm);
  }
  p.counter_bytes = kCounterBytes;
  p.ws_bytes = p.counter_bytes + static_cast<int64_t>(p.P) * 2 * p.slot_floats * 4;
  return p;
}

int hip_code(hipError_t e) { return e == hipSuccess ? HS_OK : HS_EHIP + static_cast<int>(e); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool valid_dt(int dt) { return dt == HS_DT_BF16 || dt == HS_DT_F16 || dt == HS_DT_F32; }

// Every kernel addresses its operands through buffer resources whose range
// and per-lane offsets are 32-bit.  An operand spanning 2^31 bytes or more
// would get a wrapped range, and out-of-range buffer loads read zero without
// a fault, so such calls are refused here instead of computing wrong values.
bool extents_ok(int wt, const GemmArgs& a, int y_cols) {
  constexpr int64_t lim = int64_t(1) << 31;
  const int64_t groups = (a.K + 127) / 128;
  const int64_t ses = a.sdt == HS_DT_F32 ? 4 : 2;
  const int64_t xb = ((a.M - 1) * a.ldx + a.K) * 2;
  const int64_t yb = ((a.M - 1) * a.ldy + y_cols) * 2;
  int64_t wb, sb, zb = 0;
  if (wt == W_INT4) {
    wb = ((a.N - 1) * a.ldw + (a.K + 7) / 8) * 4;
    sb = ((a.N - 1) * a.lds + groups) * ses;
    zb = (((a.N + 7) / 8 - 1) * a.ldz + groups) * 4;
  } else {
    wb = (a.N - 1) * a.ldw + a.K;
    sb = (((a.N + 127) / 128 - 1) * a.lds + groups) * ses;
  }
  return xb < lim && yb < lim && wb < lim && sb < lim && zb < lim;
}

int run_gemm(int wt, GemmArgs& a, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if (!extents_ok(wt, a, a.N)) return HS_EUNSUPPORTED;
  a.xvec = aligned16(a.x) && (a.ldx % 8 == 0);
  const Tuning& tn = tuning();
  // Tiled weight copy: the tiled decode kernel (contiguous KiB weight loads);
  // every other kernel reads the row-major weight.
  if (a.wtiles != nullptr && tm_min_ok(wt, a.M, a.N, a.K) && tiled_ok(a, wt)) {
    const TmPlan tp = tm_plan(wt, a.M, a.N, a.K);
    if (tp.P > 0) {
      if (tp.splits > 1 && (workspace == nullptr || workspace_bytes < tp.ws_bytes)) return HS_EWORKSPACE;
      a.tpw = tp.tpw;
      a.splits = tp.splits;
      a.cps = tp.cps;
      a.counters = reinterpret_cast<int*>(workspace);
      a.partials = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + kCounterBytes);
      return hip_code(launch_tiled(wt, a, stream));
    }
  }
  // Narrow outputs (N < K) at 129..256 rows: too few 256x256 tiles to fill
  // the chip (20 on a 5120-row output), so two passes of the 17..128-row
  // streaming kernel over row halves measured faster (INT4 / FP8 down
  // 17408->5120 at M=256: 102 / 100 us against 108 / 111 us; M=160: 80 vs
  // 106 us).  Sequential on the stream, so they share the workspace.
  // With a tiled weight copy and at most 64 rows in the upper half, wide
  // outputs split too: the upper half goes to the tiled decode kernel (INT4 /
  // FP8 qkv 12288x5120 at M=192: 60 / 64 us against 73 / 76 us in one pass).
  if (!tn.row_split_off && a.M > 128 && a.M <= 256 && (a.N < a.K || (a.wtiles != nullptr && a.M <= 192)) &&
      a.silu_mul == 0) {
    GemmArgs lo = a, hi = a;
    lo.M = 128;
    hi.M = a.M - 128;
    hi.x = a.x + 128 * a.ldx;
    hi.y = a.y + 128 * a.ldy;
    lo.xvec = hi.xvec = a.xvec && aligned16(hi.x);
    if (lo.xvec && mid_ok(lo, wt)) {
      const int rc = run_gemm(wt, lo, workspace, workspace_bytes, stream);
      if (rc != HS_OK) return rc;
      return run_gemm(wt, hi, workspace, workspace_bytes, stream);
    }
  }
  // Decode with at most 16 activation rows: row-partitioned kernels, one
  // partition per workgroup, no workspace.  Block-major when X fits in LDS.
  // The register-streamed kernel wins on narrow outputs (N < K) from 5
  // (INT4) / 9 (FP8) activation rows; the row-partitioned kernels below keep
  // fewer rows and the wide outputs.  Of the kernels below only the 256x256
  // prefill kernel reads tiles.
  const void* const tiles = a.wtiles;
  a.wtiles = nullptr;
  const bool skinny_auto = a.N < a.K && a.M >= (wt == W_INT4 ? 5 : 9);
  const bool use_skinny = tn.skinny != 2 && (tn.skinny == 1 || skinny_auto) && a.M <= 64 &&
                          skinny_ok(a, wt, skinny_layout(wt, a.M, a.K).kc);
  // Up to 8 (INT4) / 4 (FP8) rows with at most two 16-row blocks per
  // workgroup (narrow outputs such as 5120 or 4096 rows): the chunk-major
  // kernel below measured faster (INT4 4096x4096, M=1..8: 8.1 vs 9.4 us;
  // FP8 5120x17408, M=4: 26.7 vs 29.8 us; FP8 4096x4096, M=1: 9.2 vs 10.9 us).
  const bool gemv_narrow = a.M <= (wt == W_INT4 ? 8 : 4) &&
                           (a.N + device_cus() - 1) / device_cus() <= 32 && !tn.rows_off;
  if (!use_skinny && !tn.gemv_off && a.M <= 16 && !gemv_narrow) {
    const int P = device_cus() * (tn.gemv_wg > 0 ? tn.gemv_wg : 1);
    int kw = 0, rows_max = 0;
    if (gemv_ok(a, wt, P, tn.gemv_kw > 0 ? tn.gemv_kw : 8, &kw, &rows_max)) {
      a.P = P;
      a.T = a.K / 128;
      a.G = rows_max;
      return hip_code(launch_gemv(wt, a, kw, stream));
    }
  }
  if (!use_skinny && !tn.rows_off && a.M <= (tn.rows_ms2_off ? 16 : 32)) {
    const int P = device_cus() * (tn.rows_wg > 0 ? tn.rows_wg : 1);
    int nblk = 0, ms = 1;
    bool xl = false;
    // Above 4 rows (8 for INT4) with narrow partitions (1-2 blocks of 16
    // weight rows per workgroup) the streaming kernel below is faster;
    // 17..32 rows take two 16-row strips and need 3+ row blocks.
    if (rows_ok(a, wt, P, &nblk, &xl, &ms, tn.rows_xl) &&
        (tn.rows_force || a.M <= 4 || (a.M <= 8 && wt == W_INT4) || nblk >= 3)) {
      a.P = P;
      a.T = a.K / 128;
      return hip_code(launch_rows(wt, a, nblk, xl, ms, stream));
    }
  }
  const int nb = tn.st_nb > 0 ? tn.st_nb : stream_nb(a.M);
  const Plan p = make_plan(wt, a.M, a.N, a.K, decode_kfull(a.K, a.xvec, a.wvec), stream_ok(a, wt, nb),
                           wide_ok(a, wt), mid_ok(a, wt), use_skinny);
  if (p.T > kMaxTiles) return HS_EUNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < p.ws_bytes) return HS_EWORKSPACE;
  a.G = p.G;
  a.NB = p.NB;
  a.T = p.T;
  a.TM = p.TM;
  a.U = p.U;
  a.P = p.P;
  a.counters = reinterpret_cast<int*>(workspace);
  a.partials = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + p.counter_bytes);
  if (p.wide && !tn.wide_tiles_off) {
    a.wtiles = tiles;
    if (!wide_tiles_ok(a, wt)) a.wtiles = nullptr;
  }
  hipError_t e = p.skinny   ? launch_skinny(wt, a, p.SS, p.SNB, p.SKC, skinny_xd(a.M), stream)
                 : p.mid    ? launch_mid(wt, a, p.BMI, p.NJ, p.NW, stream)
                 : p.stream ? launch_stream(wt, a, p.MT, p.S, stream)
                 : p.decode ? launch_decode(wt, a, p.MT, p.S, stream)
                 : p.wide   ? launch_wide(wt, a, stream)
                            : launch_prefill(wt, a, p.BM, stream);
  return hip_code(e);
}

// ---- fixed scratch for callers that cannot allocate (hs_int4_gemm_noalloc) --
// One file-scope device array per GPU holds the split-K workspace: arrival
// counters first (which every kernel returns to zero when it finishes), then
// the partial tiles.  Host code never uses the array's name as an address:
// the device address comes from hipGetSymbolAddress, once per device, with
// that device current.
constexpr int64_t kScratchBytes = int64_t(40) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

struct ScratchSlot {
  void* ptr = nullptr;
  bool cleared = false;
};
ScratchSlot g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

__global__ void clear_words_kernel(uint32_t* p, int64_t words) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride) p[i] = 0u;
}

// Device address of this device's scratch array; on the first call per device
// the counter block is cleared with a fill kernel on `stream` (no memset node,
// so the call may be captured).  The clear is repeated until it has run on a
// stream that was not capturing, so a captured-but-never-replayed first call
// cannot leave the counters uncleared.
int scratch_for_device(hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_code(e);
  if (dev < 0 || dev >= kMaxDevices) return HS_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot& slot = g_scratch[dev];
  if (slot.ptr == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_code(e);
    if (ptr == nullptr) return HS_EHIP + static_cast<int>(hipErrorInvalidSymbol);
    slot.ptr = ptr;
  }
  if (!slot.cleared) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return hip_code(e);
    hipLaunchKernelGGL(clear_words_kernel, dim3(256), dim3(256), 0, stream, static_cast<uint32_t*>(slot.ptr),
                       kCounterBytes / 4);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_code(e);
    slot.cleared = cs == hipStreamCaptureStatusNone;
  }
  *out = slot.ptr;
  return HS_OK;
}

}  // namespace
}  // namespace hsq

extern "C" {

int hs_abi_version(void) { return 1; }

const char* hs_error_string(int code) {
  switch (code) {
    case HS_OK: return "success";
    case HS_EINVAL: return "invalid argument (shape, stride, pointer or dtype code)";
    case HS_EWORKSPACE: return "workspace missing or smaller than hs_gemm_workspace_bytes()";
    case HS_EUNSUPPORTED: return "unsupported configuration";
    case HS_ESCRATCH: return "problem needs more split-K workspace than the fixed scratch array holds (hs_int4_gemm_noalloc)";
    default: break;
  }
  if (code >= HS_EHIP) return hipGetErrorString(static_cast<hipError_t>(code - HS_EHIP));
  return "unknown error";
}

int64_t hs_gemm_workspace_bytes(int kind, int M, int N, int K) {
  if ((kind != HS_KIND_INT4 && kind != HS_KIND_FP8) || M <= 0 || N <= 0 || K <= 0) return 0;
  // The bound covers every variant the call may pick for this shape.
  int64_t best = 0;
  for (int kfull = 0; kfull < 2; ++kfull)
    for (int fast = 0; fast < 2; ++fast)
      for (int wide = 0; wide < 2; ++wide)
        for (int mid = 0; mid < 2; ++mid)
          for (int sk = 0; sk < 2; ++sk) {
            const int64_t b =
                hsq::make_plan(kind, M, N, K, kfull != 0, fast != 0, wide != 0, mid != 0, sk != 0).ws_bytes;
            best = b > best ? b : best;
          }
  // the tiled decode kernel (calls that pass a tiled copy)
  if (M <= 64 && N % 16 == 0 && K % 128 == 0) {
    for (int silu = 0; silu < 2; ++silu) {
      const int64_t b = hsq::tm_plan(kind, M, N, K, silu != 0).ws_bytes;
      best = b > best ? b : best;
    }
  }
  // the two row halves of the narrow-output split at 129..256 rows
  if (M > 128 && M <= 256 && (N < K || M <= 192)) {
    const int64_t lo = hs_gemm_workspace_bytes(kind, 128, N, K), hi = hs_gemm_workspace_bytes(kind, M - 128, N, K);
    best = lo > best ? lo : best;
    best = hi > best ? hi : best;
  }
  return best;
}

static int int4_gemm_impl(const void* x, int64_t ldx, const int32_t* packed, int64_t ld_packed, const void* scale,
                          int64_t ld_scale, int scale_dtype, const int32_t* zero_point, int64_t ld_zero,
                          const int32_t* tiles, void* y, int64_t ldy, int M, int N, int K, int group, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  if (M < 0 || N < 0 || K < 0) return HS_EINVAL;
  if (group != 128) return HS_EUNSUPPORTED;
  if (M == 0 || N == 0) return HS_OK;
  if (K == 0) return HS_EUNSUPPORTED;
  const int64_t kw = (K + 7) / 8, groups = (K + 127) / 128;
  if (!x || !packed || !scale || !zero_point || !y) return HS_EINVAL;
  if (ldx < K || ld_packed < kw || ld_scale < groups || ld_zero < groups || ldy < N) return HS_EINVAL;
  if (!hsq::valid_dt(scale_dtype)) return HS_EINVAL;
  hsq::GemmArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = packed;
  a.ldw = ld_packed;
  a.scale = scale;
  a.lds = ld_scale;
  a.sdt = scale_dtype;
  a.zero = zero_point;
  a.ldz = ld_zero;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.wvec = hsq::aligned16(packed) && (ld_packed % 4 == 0);
  a.tune = hsq::tuning().tune;
  a.wtiles = tiles != nullptr && hsq::aligned16(tiles) && K % 128 == 0 && N % 16 == 0 ? tiles : nullptr;
  return hsq::run_gemm(hsq::W_INT4, a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int hs_int4_gemm(const void* x, int64_t ldx, const int32_t* packed, int64_t ld_packed, const void* scale,
                 int64_t ld_scale, int scale_dtype, const int32_t* zero_point, int64_t ld_zero, void* y, int64_t ldy,
                 int M, int N, int K, int group, void* workspace, int64_t workspace_bytes, void* stream) {
  return int4_gemm_impl(x, ldx, packed, ld_packed, scale, ld_scale, scale_dtype, zero_point, ld_zero, nullptr, y, ldy, M,
                        N, K, group, workspace, workspace_bytes, stream);
}

int hs_int4_gemm_tiled(const void* x, int64_t ldx, const int32_t* packed, int64_t ld_packed, const int32_t* tiles,
                       const void* scale, int64_t ld_scale, int scale_dtype, const int32_t* zero_point,
                       int64_t ld_zero, void* y, int64_t ldy, int M, int N, int K, int group, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  if (tiles == nullptr) return HS_EINVAL;
  return int4_gemm_impl(x, ldx, packed, ld_packed, scale, ld_scale, scale_dtype, zero_point, ld_zero, tiles, y, ldy, M,
                        N, K, group, workspace, workspace_bytes, stream);
}

int hs_int4_gemm_noalloc(const void* x, int64_t ldx, const int32_t* packed, int64_t ld_packed, const void* scale,
                         int64_t ld_scale, int scale_dtype, const int32_t* zero_point, int64_t ld_zero, void* y,
                         int64_t ldy, int M, int N, int K, int group, void* stream) {
  if (M < 0 || N < 0 || K < 0) return HS_EINVAL;
  if (group != 128) return HS_EUNSUPPORTED;
  if (M == 0 || N == 0) return HS_OK;
  // Argument checks first, so a rejected call touches no device state.
  if (K == 0) return HS_EUNSUPPORTED;
  if (x == nullptr || packed == nullptr || scale == nullptr || zero_point == nullptr || y == nullptr) return HS_EINVAL;
  if (ldx < K || ld_packed < (K + 7) / 8 || ld_scale < (K + 127) / 128 || ld_zero < (K + 127) / 128 || ldy < N)
    return HS_EINVAL;
  if (!hsq::valid_dt(scale_dtype)) return HS_EINVAL;
  void* ws = nullptr;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc0 = hsq::scratch_for_device(s, &ws);
  if (rc0 != HS_OK) return rc0;
  const int rc = hs_int4_gemm(x, ldx, packed, ld_packed, scale, ld_scale, scale_dtype, zero_point, ld_zero, y, ldy, M,
                              N, K, group, ws, hsq::kScratchBytes, stream);
  return rc == HS_EWORKSPACE ? HS_ESCRATCH : rc;
}

static int int4_silu_impl(const void* x, int64_t ldx, const int32_t* packed, int64_t ld_packed,
                          const int32_t* tiles, const void* scale, int64_t ld_scale, int scale_dtype,
                          const int32_t* zero_point, int64_t ld_zero, void* y, int64_t ldy, int M, int N, int K,
                          int group, void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || N < 0 || K < 0) return HS_EINVAL;
  if (group != 128) return HS_EUNSUPPORTED;
  if (N % 32 != 0) return HS_EINVAL;
  if (M == 0 || N == 0) return HS_OK;
  if (K == 0) return HS_EUNSUPPORTED;
  const int64_t kw = (K + 7) / 8, groups = (K + 127) / 128;
  if (!x || !packed || !scale || !zero_point || !y) return HS_EINVAL;
  if (ldx < K || ld_packed < kw || ld_scale < groups || ld_zero < groups || ldy < N / 2) return HS_EINVAL;
  if (!hsq::valid_dt(scale_dtype)) return HS_EINVAL;
  hsq::GemmArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = packed;
  a.ldw = ld_packed;
  a.scale = scale;
  a.lds = ld_scale;
  a.sdt = scale_dtype;
  a.zero = zero_point;
  a.ldz = ld_zero;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.xvec = hsq::aligned16(x) && (ldx % 8 == 0);
  a.wvec = hsq::aligned16(packed) && (ld_packed % 4 == 0);
  a.tune = hsq::tuning().tune;
  a.silu_mul = 1;
  if (!hsq::extents_ok(hsq::W_INT4, a, N / 2)) return HS_EUNSUPPORTED;
  // Tiled copy of the interleaved weight: the tiled decode kernel's store
  // carries the epilogue up to 64 rows, the 256x256 prefill kernel reads the
  // tiles from 129 rows; 17..128 rows and every other case use the kernels
  // below on the row-major weight.
  const int32_t* const tl = tiles != nullptr && hsq::aligned16(tiles) && K % 128 == 0 && N % 16 == 0 ? tiles : nullptr;
  if (tl != nullptr) {
    a.wtiles = tl;
    if (hsq::tm_min_ok(hsq::W_INT4, M, N, K) && hsq::tiled_ok(a, hsq::W_INT4)) {
      const hsq::TmPlan tp = hsq::tm_plan(hsq::W_INT4, M, N, K, true);
      if (tp.P > 0) {
        if (tp.splits > 1 && (workspace == nullptr || workspace_bytes < tp.ws_bytes)) return HS_EWORKSPACE;
        a.tpw = tp.tpw;
        a.splits = tp.splits;
        a.cps = tp.cps;
        a.counters = reinterpret_cast<int*>(workspace);
        a.partials = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + hsq::kCounterBytes);
        return hsq::hip_code(hsq::launch_tiled(hsq::W_INT4, a, static_cast<hipStream_t>(stream)));
      }
    }
    a.wtiles = nullptr;
  }
  // The fused epilogue is in the block-major GEMV kernel (1..16 rows, X in
  // LDS) and in the 17..128-row LDS-DMA kernel.
  if (M <= 16) {
    const hsq::Tuning& tn = hsq::tuning();
    const int P = hsq::device_cus() * (tn.gemv_wg > 0 ? tn.gemv_wg : 1);
    int kw = 0, rows_max = 0;
    if (!tn.gemv_off && hsq::gemv_ok(a, hsq::W_INT4, P, tn.gemv_kw > 0 ? tn.gemv_kw : 8, &kw, &rows_max)) {
      a.P = P;
      a.T = K / 128;
      a.G = rows_max;
      return hsq::hip_code(hsq::launch_gemv(hsq::W_INT4, a, kw, static_cast<hipStream_t>(stream)));
    }
    // X too large for the block-major kernel's LDS: the row-partitioned
    // kernel (X in LDS when it fits, else A fragments from global memory).
    const int Pr = hsq::device_cus() * (tn.rows_wg > 0 ? tn.rows_wg : 1);
    int nblk = 0, ms = 1;
    bool xl = false;
    if (tn.rows_off || !hsq::rows_ok(a, hsq::W_INT4, Pr, &nblk, &xl, &ms, tn.rows_xl)) return HS_EUNSUPPORTED;
    a.P = Pr;
    a.T = K / 128;
    return hsq::hip_code(hsq::launch_rows(hsq::W_INT4, a, nblk, xl, ms, static_cast<hipStream_t>(stream)));
  }
  if (M > 128) {
    // Prefill: the 256x256-tile kernel's store carries the epilogue.
    if (!hsq::wide_ok(a, hsq::W_INT4)) return HS_EUNSUPPORTED;
    if (tl != nullptr && !hsq::tuning().wide_tiles_off) {
      a.wtiles = tl;
      if (!hsq::wide_tiles_ok(a, hsq::W_INT4)) a.wtiles = nullptr;
    }
    const hsq::Plan p = hsq::make_plan(hsq::W_INT4, M, N, K, false, false, true, false, false);
    if (!p.wide || p.T > hsq::kMaxTiles) return HS_EUNSUPPORTED;
    if (workspace == nullptr || workspace_bytes < p.ws_bytes) return HS_EWORKSPACE;
    a.G = p.G;
    a.NB = p.NB;
    a.T = p.T;
    a.TM = p.TM;
    a.U = p.U;
    a.P = p.P;
    a.counters = reinterpret_cast<int*>(workspace);
    a.partials = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + p.counter_bytes);
    return hsq::hip_code(hsq::launch_wide(hsq::W_INT4, a, static_cast<hipStream_t>(stream)));
  }
  if (!hsq::mid_ok(a, hsq::W_INT4)) return HS_EUNSUPPORTED;
  const hsq::Plan p = hsq::make_plan(hsq::W_INT4, M, N, K, false, false, false, true, false);
  if (!p.mid) return HS_EUNSUPPORTED;
  if (p.T > hsq::kMaxTiles) return HS_EUNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < p.ws_bytes) return HS_EWORKSPACE;
  a.G = p.G;
  a.NB = p.NB;
  a.T = p.T;
  a.TM = p.TM;
  a.U = p.U;
  a.P = p.P;
  a.counters = reinterpret_cast<int*>(workspace);
  a.partials = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + p.counter_bytes);
  return hsq::hip_code(hsq::launch_mid(hsq::W_INT4, a, p.BMI, p.NJ, p.NW, static_cast<hipStream_t>(stream)));
}

int hs_int4_gemm_silu_mul(const void* x, int64_t ldx, const int32_t* packed, int64_t ld_packed, const void* scale,
                          int64_t ld_scale, int scale_dtype, const int32_t* zero_point, int64_t ld_zero, void* y,
                          int64_t ldy, int M, int N, int K, int group, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  return int4_silu_impl(x, ldx, packed, ld_packed, nullptr, scale, ld_scale, scale_dtype, zero_point, ld_zero, y, ldy,
                        M, N, K, group, workspace, workspace_bytes, stream);
}

int hs_int4_gemm_silu_mul_tiled(const void* x, int64_t ldx, const int32_t* packed, int64_t ld_packed,
                                const int32_t* tiles, const void* scale, int64_t ld_scale, int scale_dtype,
                                const int32_t* zero_point, int64_t ld_zero, void* y, int64_t ldy, int M, int N, int K,
                                int group, void* workspace, int64_t workspace_bytes, void* stream) {
  return int4_silu_impl(x, ldx, packed, ld_packed, tiles, scale, ld_scale, scale_dtype, zero_point, ld_zero, y, ldy,
                        M, N, K, group, workspace, workspace_bytes, stream);
}

static int fp8_gemm_impl(const void* x, int64_t ldx, const uint8_t* data, int64_t ld_data, const uint8_t* tiles,
                         const void* scale_inv, int64_t ld_scale, int scale_dtype, void* y, int64_t ldy, int M, int N,
                         int K, void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || N < 0 || K < 0) return HS_EINVAL;
  if (M == 0 || N == 0) return HS_OK;
  if (K == 0) return HS_EUNSUPPORTED;
  const int64_t kb = (K + 127) / 128;
  if (!x || !data || !scale_inv || !y) return HS_EINVAL;
  if (ldx < K || ld_data < K || ld_scale < kb || ldy < N) return HS_EINVAL;
  if (!hsq::valid_dt(scale_dtype)) return HS_EINVAL;
  hsq::GemmArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = data;
  a.ldw = ld_data;
  a.scale = scale_inv;
  a.lds = ld_scale;
  a.sdt = scale_dtype;
  a.zero = nullptr;
  a.ldz = 0;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.wvec = hsq::aligned16(data) && (ld_data % 16 == 0);
  a.tune = hsq::tuning().tune;
  a.wtiles = tiles != nullptr && hsq::aligned16(tiles) && K % 128 == 0 && N % 16 == 0 ? tiles : nullptr;
  return hsq::run_gemm(hsq::W_FP8, a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int hs_fp8_gemm(const void* x, int64_t ldx, const uint8_t* data, int64_t ld_data, const void* scale_inv,
                int64_t ld_scale, int scale_dtype, void* y, int64_t ldy, int M, int N, int K, void* workspace,
                int64_t workspace_bytes, void* stream) {
  return fp8_gemm_impl(x, ldx, data, ld_data, nullptr, scale_inv, ld_scale, scale_dtype, y, ldy, M, N, K, workspace,
                       workspace_bytes, stream);
}

int hs_fp8_gemm_tiled(const void* x, int64_t ldx, const uint8_t* data, int64_t ld_data, const uint8_t* tiles,
                      const void* scale_inv, int64_t ld_scale, int scale_dtype, void* y, int64_t ldy, int M, int N,
                      int K, void* workspace, int64_t workspace_bytes, void* stream) {
  if (tiles == nullptr) return HS_EINVAL;
  return fp8_gemm_impl(x, ldx, data, ld_data, tiles, scale_inv, ld_scale, scale_dtype, y, ldy, M, N, K, workspace,
                       workspace_bytes, stream);
}

int hs_int4_dequant(const int32_t* packed, int64_t ld_packed, const void* scale, int64_t ld_scale, int scale_dtype,
                    const int32_t* zero_point, int64_t ld_zero, void* out, int64_t ld_out, int out_dtype, int N, int K,
                    int group, void* stream) {
  if (N < 0 || K < 0 || group <= 0) return HS_EINVAL;
  if (N == 0 || K == 0) return HS_OK;
  const int64_t kw = (K + 7) / 8, groups = (K + group - 1) / group;
  if (!packed || !scale || !zero_point || !out) return HS_EINVAL;
  if (ld_packed < kw || ld_scale < groups || ld_zero < groups || ld_out < K) return HS_EINVAL;
  if (!hsq::valid_dt(scale_dtype) || !hsq::valid_dt(out_dtype)) return HS_EINVAL;
  return hsq::hip_code(hsq::launch_int4_dequant(reinterpret_cast<const uint32_t*>(packed), ld_packed, scale, ld_scale,
                                                scale_dtype, zero_point, ld_zero, out, ld_out, out_dtype, N, K, group,
                                                static_cast<hipStream_t>(stream)));
}

int hs_fp8_dequant(const uint8_t* data, int64_t ld_data, const void* scale_inv, int64_t ld_scale, int scale_dtype,
                   void* out, int64_t ld_out, int out_dtype, int N, int K, void* stream) {
  if (N < 0 || K < 0) return HS_EINVAL;
  if (N == 0 || K == 0) return HS_OK;
  const int64_t kb = (K + 127) / 128;
  if (!data || !scale_inv || !out) return HS_EINVAL;
  if (ld_data < K || ld_scale < kb || ld_out < K) return HS_EINVAL;
  if (!hsq::valid_dt(scale_dtype) || !hsq::valid_dt(out_dtype)) return HS_EINVAL;
  return hsq::hip_code(hsq::launch_fp8_dequant(data, ld_data, scale_inv, ld_scale, scale_dtype, out, ld_out, out_dtype,
                                               N, K, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
