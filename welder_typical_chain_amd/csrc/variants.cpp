// variants.cpp -- the variant table and the calibrated cost model
// (declarations and the role of each in variants.h).
#include "variants.h"

#include <algorithm>
#include <cmath>

#include "wtc/wtc_hip.h"

namespace wtc {

namespace {

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int in_bytes(int dt) { return dt == WTC_DTYPE_F32 ? 4 : (dt == WTC_DTYPE_FP8_E4M3 ? 1 : 2); }
int out_bytes(int dt) { return dt == WTC_DTYPE_F32 ? 4 : 2; }
bool valid_in(int dt) { return dt >= WTC_DTYPE_F32 && dt <= WTC_DTYPE_FP8_E4M3; }

constexpr unsigned bit(int path) { return 1u << path; }
constexpr unsigned kTilePaths = bit(WTC_PATH_EXCHANGE) | bit(WTC_PATH_SPLIT) | bit(WTC_PATH_UNFUSED);
constexpr unsigned kSplitPaths = bit(WTC_PATH_SPLIT) | bit(WTC_PATH_UNFUSED);

// ---- calibration -------------------------------------------------------------
// The model: a call costs its kernels' back-to-back launch time, plus the
// tile kernel's waves times one tile's cycles at the clock the chip holds
// under that load, plus the passes that stream the output (split: the
// rescale; unfused: four f32 row passes), plus the row exchange (a fixed
// part and a part per column tile of a row block).  The full waves (every
// CU busy) and the last, partial one are priced separately.  One tile's
// cycles are a fixed part (first loads and epilogue) and, per 128 bytes of
// K, the variant's own cycles plus the cycles its A and B bytes add as they
// stream in (bytes of every active tile over a chip-wide rate).
//
// The constants were fitted (least squares on the log of the time) to
// back-to-back timings of every variant on every path over the 60 shapes
// of calibrate.py on MI355X.  Fitted on three of its four shape sets and
// scored on the fourth, in turn, the fused ranking lost 0.84 % on average
// against the measured fastest choice (the hand-written rules it replaces:
// 5.3 %).
struct TileCal {
  double kt_cyc;        // own cycles per k-tile
  double fixed_cyc[3];  // per tile: exchange, split, logits epilogues
};
// [tile variant][0: 16-bit, 1: fp8, 2: f32]; fixed parts shared across input
// types.  Rows: kVarTile128, kVarTile128Loaders, kVarTile256, kVarTile256x256.
const TileCal kTileCal[4][3] = {
    /* kVarTile128 */ {{635.87, {3678.9, 5946.6, 0}}, {617.19, {3678.9, 5946.6, 0}}, {4521.3, {3678.9, 5946.6, 0}}},
    /* kVarTile128Loaders */ {{562.07, {4068.6, 6487.6, 254}}, {530.85, {4068.6, 6487.6, 254}}, {0, {0, 0, 0}}},
    /* kVarTile256 */ {{1142.1, {0, 11628.2, 0}}, {1286.6, {0, 11628.2, 0}}, {0, {0, 0, 0}}},
    /* kVarTile256x256 */ {{1973.6, {0, 20944.0, 6164}}, {1635.5, {0, 20944.0, 6164}}, {0, {0, 0, 0}}},
};
int cal_row(int id) { return id == kVarTile256x256 ? 3 : id; }
// Rows kernel, cycles per row block: a fixed part, and per 128-column tile
// (both passes) a fixed part and a part per 16-wide k-step.
constexpr double kRowsBlockCyc = 1983.1, kRowsTileCyc = 4932.5, kRowsKstepCyc = 102.19;
// Back-to-back launch cost of one kernel (us); the row exchange after the
// last tile of a row block: fixed (us) and per column tile (us); the HBM
// rate of the fused paths' streaming passes and the chip-wide rate that
// prices k-tile bytes (GB/s).
constexpr double kLaunchUs = 3.6597, kExchangeUs = 0.2592, kExchangePerTileUs = 0.08580;
constexpr double kHbmGBs = 7919.8, kFeedGBs = 83312.1;
// Unfused row passes (one 256-thread workgroup per row, eight per CU): HBM
// rate, and the rate one workgroup streams its row at (GB/s).
constexpr double kRowPassHbmGBs = 5293.0, kRowPassWgGBs = 5.573;

// Core clock under load, from the call's mean share of busy CUs: 1.5 GHz
// with every CU busy throughout, ~2.1 with half of them or fewer (the chip's
// power limit, not the workload, sets it).
double clock_ghz(double busy) {
  busy = std::min(1.0, std::max(0.0, busy));
  return busy <= 0.5 ? 2.1 : 2.1 - 1.2 * (busy - 0.5);
}

int in_class(int in_dt) {
  return in_dt == WTC_DTYPE_FP8_E4M3 ? 1 : (in_dt == WTC_DTYPE_F32 ? 2 : 0);
}

}  // namespace

static std::vector<VariantDesc> make_variants(int in_dt) {
  std::vector<VariantDesc> v;
  if (!valid_in(in_dt)) return v;
  const int64_t tk = 128 / in_bytes(in_dt);
  if (in_dt == WTC_DTYPE_F32) {
    v.push_back({kVarTile128, "tile128x128_wave64x64", 128, 128, tk, 2, 32, 128, 0, kTilePaths});
    return v;
  }
  v.push_back({kVarTile128, "tile128x128_wave64x32", 128, 128, tk, 2, 16, 128, 0, kTilePaths});
  v.push_back({kVarTile128Loaders, "tile128x128_wave64x64_loaders", 128, 128, tk, 2, 32, 128, 1,
               kTilePaths});
  v.push_back({kVarTile256, "tile256x128_wave64x64", 256, 128, tk, 2, 32, 256, 0, kSplitPaths});
  if (in_dt == WTC_DTYPE_F16 || in_dt == WTC_DTYPE_BF16)
    v.push_back({kVarRows, "rows128_wave64x32_k128", 128, 128, kRowsMaxK, 2, 16, 128, 0,
                 bit(WTC_PATH_ROWS)});
  // tile_k: one 64-byte k-slab per ring stage
  v.push_back({kVarTile256x256, "tile256x256_wave128x128", 256, 256, tk / 2, 4, 64, 256, 0,
               kSplitPaths});
  return v;
}

const std::vector<VariantDesc>& variants_for(int in_dt) {
  static const std::vector<VariantDesc> tables[5] = {
      make_variants(WTC_DTYPE_F32), make_variants(WTC_DTYPE_F16), make_variants(WTC_DTYPE_BF16),
      make_variants(WTC_DTYPE_FP8_E4M3), {}};
  return tables[valid_in(in_dt) ? in_dt : 4];
}

bool find_variant(int in_dt, int64_t tm, int64_t tn, int64_t tk, int64_t ttm, int64_t ttn,
                  VariantDesc* out) {
  for (const VariantDesc& v : variants_for(in_dt))
    if (v.tile_m == tm && v.tile_n == tn && v.tile_k == tk && v.thread_tile_m == ttm &&
        v.thread_tile_n == ttn) {
      if (out) *out = v;
      return true;
    }
  return false;
}

bool variant_by_id(int in_dt, int id, VariantDesc* out) {
  for (const VariantDesc& v : variants_for(in_dt))
    if (v.id == id) {
      if (out) *out = v;
      return true;
    }
  return false;
}

bool feasible(const VariantDesc& v, int path, const Problem& p) {
  if (path < WTC_PATH_EXCHANGE || path > WTC_PATH_ROWS || !(v.paths & bit(path))) return false;
  const int64_t nT = cdiv(p.n, v.tile_n);
  switch (path) {
    case WTC_PATH_EXCHANGE: {
      const int64_t tiles = p.batch * cdiv(p.m, v.tile_rows) * nT;
      return tiles <= (int64_t)p.cu_count * std::max(1, p.xch_per_cu) &&
             nT <= kExchangeMaxColTiles && tiles <= kExchangeMaxTiles;
    }
    case WTC_PATH_SPLIT:
      return nT <= kSplitMaxColTiles;
    case WTC_PATH_ROWS:
      return p.k <= kRowsMaxK;
    default:
      return true;
  }
}

std::string infeasible_reason(const VariantDesc& v, int path, const Problem& p) {
  static const char* const kPathNames[] = {"auto", "exchange", "split", "unfused", "rows"};
  if (path < WTC_PATH_EXCHANGE || path > WTC_PATH_ROWS) return "unknown path";
  if (!(v.paths & bit(path)))
    return path == WTC_PATH_ROWS ? "rows path needs 16-bit inputs and k <= 128"
                                 : std::string("variant ") + v.name + " does not run the " +
                                       kPathNames[path] + " path";
  const int64_t nT = cdiv(p.n, v.tile_n);
  switch (path) {
    case WTC_PATH_EXCHANGE: {
      const int64_t tiles = p.batch * cdiv(p.m, v.tile_rows) * nT;
      const int64_t resident = (int64_t)p.cu_count * std::max(1, p.xch_per_cu);
      if (tiles > resident)
        return "exchange path needs every tile co-resident: " + std::to_string(tiles) + " tiles > " +
               std::to_string(resident) + " resident workgroups";
      if (nT > kExchangeMaxColTiles || tiles > kExchangeMaxTiles)
        return "exchange path supports n <= 8192 and <= " + std::to_string(kExchangeMaxTiles) +
               " tiles";
      return "";
    }
    case WTC_PATH_SPLIT:
      return nT > kSplitMaxColTiles
                 ? "split path supports n <= " + std::to_string(kSplitMaxColTiles * v.tile_n) +
                       " with " + std::to_string(v.tile_n) + "-column tiles"
                 : "";
    case WTC_PATH_ROWS:
      return p.k > kRowsMaxK ? "rows path needs 16-bit inputs and k <= 128" : "";
    default:
      return "";
  }
}

int64_t variant_grid(const VariantDesc& v, int path, const Problem& p) {
  if (path == WTC_PATH_ROWS) return p.batch * cdiv(p.m, 128);
  return p.batch * cdiv(p.m, v.tile_rows) * cdiv(p.n, v.tile_n);
}

double estimate_us(const VariantDesc& v, int path, const Problem& p) {
  const double cu = std::max(1, p.cu_count);
  const double isz = in_bytes(p.in_dt), osz = out_bytes(p.out_dt);
  const double elems = (double)p.batch * (double)p.m * (double)p.n;
  const double ab_bytes = (double)p.batch * ((double)p.m * p.k + (double)p.k * p.n) * isz;
  const double us_per_byte = 1e6 / (kHbmGBs * 1e9);
  const double nT = (double)cdiv(p.n, path == WTC_PATH_ROWS ? 128 : v.tile_n);
  if (path == WTC_PATH_ROWS) {
    const double blocks = (double)variant_grid(v, path, p);
    const double waves = std::ceil(blocks / cu);
    const double f = clock_ghz(blocks / (waves * cu));
    const double cyc = kRowsBlockCyc + nT * (kRowsTileCyc + kRowsKstepCyc * (double)cdiv(p.k, 16));
    const double t_blocks = waves * cyc / (f * 1e3);
    const double t_hbm = (ab_bytes + elems * osz) * us_per_byte;
    return kLaunchUs + std::max(t_blocks, t_hbm);
  }
  const TileCal& cal = kTileCal[cal_row(v.id)][in_class(p.in_dt)];
  const int epi = path == WTC_PATH_EXCHANGE ? 0 : (path == WTC_PATH_SPLIT ? 1 : 2);
  const double tiles = (double)variant_grid(v, path, p);
  const double waves = std::ceil(tiles / cu);
  const double f = clock_ghz(tiles / (waves * cu));
  const double nk = (double)cdiv(p.k * in_bytes(p.in_dt), 128);
  const double kt_bytes = (double)(v.tile_rows + v.tile_n) * 128.0;  // A and B per 128 bytes of K
  auto wave_us = [&](double active) {
    const double kt = cal.kt_cyc + kt_bytes * active * f / kFeedGBs;
    return (cal.fixed_cyc[epi] + nk * kt) / (f * 1e3);
  };
  const double full = std::floor(tiles / cu), rem = tiles - full * cu;
  const double t_tiles = full * wave_us(cu) + (rem > 0 ? wave_us(rem) : 0.0);
  if (path == WTC_PATH_EXCHANGE) {
    const double t_hbm = (ab_bytes + elems * osz) * us_per_byte;
    const double t_xch = p.n > 128 ? kExchangeUs + kExchangePerTileUs * nT : 0.0;
    return kLaunchUs + std::max(t_tiles, t_hbm) + t_xch;
  }
  if (path == WTC_PATH_SPLIT) {
    // the tile pass writes the output and the row statistics; the rescale
    // pass reads and rewrites the output
    const double stats = (double)p.batch * (double)p.m * nT * 8.0;
    const double t_hbm = (ab_bytes + elems * osz + stats) * us_per_byte;
    const double t_rescale = (2.0 * elems * osz + stats) * us_per_byte;
    return 2 * kLaunchUs + std::max(t_tiles, t_hbm) + t_rescale;
  }
  // unfused: f32 logits, then max, exp, sum and divide passes over them,
  // each at the HBM rate or, with few rows, at the rate of its workgroups
  const double row_us_per_byte = 1e6 / (kRowPassHbmGBs * 1e9);
  double t = 5 * kLaunchUs + std::max(t_tiles, (ab_bytes + elems * 4.0) * row_us_per_byte);
  const double row_waves = std::ceil((double)p.batch * (double)p.m / (cu * 8));
  for (const double bpe : {4.0, 8.0, 4.0, 4.0 + osz})
    t += std::max(elems * bpe * row_us_per_byte,
                  row_waves * (double)p.n * bpe * 1e6 / (kRowPassWgGBs * 1e9));
  return t;
}

std::vector<Choice> rank_choices(const Problem& p, int path, int variant) {
  std::vector<Choice> out;
  for (const VariantDesc& v : variants_for(p.in_dt)) {
    if (variant >= 0 && v.id != variant) continue;
    for (int q = WTC_PATH_EXCHANGE; q <= WTC_PATH_ROWS; ++q) {
      if (path == WTC_PATH_AUTO ? q == WTC_PATH_UNFUSED : q != path) continue;
      if (!feasible(v, q, p)) continue;
      out.push_back({v, q, estimate_us(v, q, p)});
    }
  }
  std::stable_sort(out.begin(), out.end(),
                   [](const Choice& a, const Choice& b) { return a.est_us < b.est_us; });
  return out;
}

bool best_choice(const Problem& p, int path, int variant, Choice* out) {
  bool found = false;
  for (const VariantDesc& v : variants_for(p.in_dt)) {
    if (variant >= 0 && v.id != variant) continue;
    for (int q = WTC_PATH_EXCHANGE; q <= WTC_PATH_ROWS; ++q) {
      if (path == WTC_PATH_AUTO ? q == WTC_PATH_UNFUSED : q != path) continue;
      if (!feasible(v, q, p)) continue;
      const double est = estimate_us(v, q, p);
      if (!found || est < out->est_us) {  // ties keep the earlier pair, as the stable sort does
        *out = Choice{v, q, est};
        found = true;
      }
    }
  }
  return found;
}

}  // namespace wtc
