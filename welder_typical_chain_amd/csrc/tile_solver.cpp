// tile_solver.cpp -- the search boundary: gfx950 tile variants, best.json I/O,
// the cost model, and welder_solver_solve_typical_chain.
//
// Replaces the Welder solver behind the same C symbol
// (backend/welder/compiler/solver/WelderSolverCAPI.cpp:104-196).  The
// reference searches a large tile space with an analytic traffic model
// (solveGeneric, solver/WelderSolverSolveEntrypoints.h:157-265) because it
// generates code for any tile; here the kernels are hand-written, so the space
// is the set of instantiated variants and the model is MI355X's roofline.
#include <algorithm>
#include <cmath>
#include <filesystem>
#include <fstream>
#include <regex>
#include <sstream>

#include "chain_spec.h"
#include "wtc/welder_solver_capi.h"
#include "wtc/wtc_hip.h"

namespace wtc {

// The kernel library's variants: a 128x128 output tile per workgroup, one
// 128-byte k-tile per pipeline step.  16-bit and fp8 inputs run 8 waves of
// 64x32 (each lane: 2 output rows x 16 columns of accumulators), f32 runs 4
// waves of 64x64 (2 rows x 32 columns).
std::vector<Variant> supported_variants(Elem in) {
  const int64_t tk = elem_bytes(in) ? 128 / elem_bytes(in) : 0;
  if (tk == 0) return {};
  if (in == Elem::F32) return {Variant{TileParams{128, 128, tk, 2, 32}, "tile128x128_wave64x64"}};
  return {Variant{TileParams{128, 128, tk, 2, 16}, "tile128x128_wave64x32"}};
}

bool is_supported(const TileParams& t, Elem in) {
  for (const Variant& v : supported_variants(in))
    if (v.tiles.tile_m == t.tile_m && v.tiles.tile_n == t.tile_n && v.tiles.tile_k == t.tile_k &&
        v.tiles.thread_tile_m == t.thread_tile_m && v.tiles.thread_tile_n == t.thread_tile_n)
      return true;
  return false;
}

// Regex reader of the five integer keys: first match wins, so a
// best_summary.json with a nested "best" object parses too
// (compiler/scheduler/Search.cpp:12-20,35-60).
static bool extract_int64(const std::string& text, const char* key, int64_t& value) {
  const std::regex re(std::string("\"") + key + "\"\\s*:\\s*(-?[0-9]+)");
  std::smatch m;
  if (!std::regex_search(text, m, re)) return false;
  value = std::stoll(m[1].str());
  return true;
}

bool load_best_json(const std::string& path, TileParams& t, std::string& diag) {
  if (path.empty()) {
    diag = "json path is empty";
    return false;
  }
  std::string text;
  if (!read_file(path, text) || text.empty()) {
    diag = "failed to read json: " + path;
    return false;
  }
  TileParams p;
  if (!extract_int64(text, "tileM", p.tile_m) || !extract_int64(text, "tileN", p.tile_n) ||
      !extract_int64(text, "tileK", p.tile_k) || !extract_int64(text, "threadTileM", p.thread_tile_m) ||
      !extract_int64(text, "threadTileN", p.thread_tile_n)) {
    diag = "failed to parse tile fields from " + path;
    return false;
  }
  t = p;
  diag.clear();
  return true;
}

// Same five keys and layout as compiler/scheduler/Search.cpp:62-86.
bool write_best_json(const TileParams& t, const std::string& path, std::string& diag) {
  if (path.empty()) {
    diag = "json path is empty";
    return false;
  }
  std::error_code ec;
  const auto parent = std::filesystem::path(path).parent_path();
  if (!parent.empty()) std::filesystem::create_directories(parent, ec);
  std::ostringstream o;
  o << "{\n"
    << "  \"tileM\": " << t.tile_m << ",\n"
    << "  \"tileN\": " << t.tile_n << ",\n"
    << "  \"tileK\": " << t.tile_k << ",\n"
    << "  \"threadTileM\": " << t.thread_tile_m << ",\n"
    << "  \"threadTileN\": " << t.thread_tile_n << "\n"
    << "}\n";
  if (!write_file(path, o.str())) {
    diag = "failed to open json for write: " + path;
    return false;
  }
  diag.clear();
  return true;
}

// ---------------------------------------------------------------------------
// cost model
// ---------------------------------------------------------------------------
// Dense MFMA FLOP per clock per CU on gfx950 (f16/bf16 4096, fp8 8192,
// f32 256).
static double mfma_flop_per_clk_cu(Elem in) {
  switch (in) {
    case Elem::F16:
    case Elem::BF16: return 4096.0;
    case Elem::F8E4M3FN: return 8192.0;
    case Elem::F32: return 256.0;
    default: return 0.0;
  }
}

std::vector<Candidate> solve(const ChainSpec& s, int64_t /*max_connect_level*/,
                             const ArchInfo& arch) {
  std::vector<Candidate> out;
  const int64_t isz = elem_bytes(s.in), osz = elem_bytes(s.out);
  for (const Variant& v : supported_variants(s.in)) {
    const TileParams& t = v.tiles;
    const int64_t nrb = (s.m + t.tile_m - 1) / t.tile_m;
    const int64_t nt = (s.n + t.tile_n - 1) / t.tile_n;
    const int64_t tiles = s.batch * nrb * nt;
    // Exchange path: every tile resident, one per CU.  Split: two per CU.
    const bool exchange = tiles <= arch.num_cu;
    const int64_t resident = exchange ? arch.num_cu : 2 * arch.num_cu;
    const int64_t waves = (tiles + resident - 1) / resident;
    const double clk = arch.clock_ghz * 1e9;
    const double tile_flops = 2.0 * (double)t.tile_m * (double)t.tile_n * (double)s.k;
    // resident tiles share a CU when two are resident per CU
    const double per_tile_s = tile_flops / (mfma_flop_per_clk_cu(s.in) * clk) * (exchange ? 1.0 : 2.0);
    const double t_mfma = (double)waves * per_tile_s;
    Candidate c;
    c.tiles = t;
    c.path = exchange ? "exchange" : "split";
    c.bytes_a = s.batch * s.m * s.k * isz * nt;  // each column tile streams its A rows
    c.bytes_b = s.batch * s.k * s.n * isz * nrb;
    c.bytes_c = s.batch * s.m * s.n * osz * (exchange ? 1 : 3);  // split: write, re-read, re-write
    c.bytes_cut = s.batch * s.m * s.n * 4;  // f32 logits never written to HBM
    // HBM sees A and B once when the XCD L2s and the MALL catch the re-reads.
    const double hbm_bytes = (double)(s.batch * (s.m * s.k + s.k * s.n) * isz) + (double)c.bytes_c;
    const double t_hbm = hbm_bytes / (arch.hbm_gbs * 1e9);
    const double t_softmax = exchange ? 2e-6 : 4e-6;  // row exchange vs second launch
    c.estimated_latency = (std::max(t_mfma, t_hbm) + t_softmax) * 1e6;
    c.score = 1.0 / c.estimated_latency;
    out.push_back(c);
  }
  std::stable_sort(out.begin(), out.end(),
                   [](const Candidate& a, const Candidate& b) { return a.score > b.score; });
  return out;
}

static bool write_best_summary(const ChainSpec& s, const ArchInfo& arch, const Candidate& best,
                               const std::string& path, std::string& err) {
  std::error_code ec;
  const auto parent = std::filesystem::path(path).parent_path();
  if (!parent.empty()) std::filesystem::create_directories(parent, ec);
  std::ostringstream o;
  o << "{\n";
  o << "  \"problem\": {\"m\": " << s.m << ", \"n\": " << s.n << ", \"k\": " << s.k
    << ", \"batch\": " << s.batch << "},\n";
  o << "  \"arch\": {\"smemBytes\": " << arch.lds_bytes << ", \"numSM\": " << arch.num_cu
    << ", \"warpSize\": " << arch.wave_size << ", \"elementBytes\": " << elem_bytes(s.in)
    << ", \"target\": \"gfx950\"},\n";
  o << "  \"best\": {\"tileM\": " << best.tiles.tile_m << ", \"tileN\": " << best.tiles.tile_n
    << ", \"tileK\": " << best.tiles.tile_k << ", \"threadTileM\": " << best.tiles.thread_tile_m
    << ", \"threadTileN\": " << best.tiles.thread_tile_n << ", \"score\": " << best.score
    << ", \"estimatedLatency\": " << best.estimated_latency << ", \"profiledMs\": " << best.profiled_ms
    << ", \"bytesCut\": " << best.bytes_cut << ", \"path\": \"" << best.path << "\"}\n";
  o << "}\n";
  if (!write_file(path, o.str())) {
    err = "failed to open best summary json: " + path;
    return false;
  }
  return true;
}

// 13 columns, as backend/welder/compiler/solver/WelderSolverCAPI.cpp:87-97.
static bool write_candidates(const std::vector<Candidate>& cs, const std::string& path,
                             std::string& err) {
  std::error_code ec;
  const auto parent = std::filesystem::path(path).parent_path();
  if (!parent.empty()) std::filesystem::create_directories(parent, ec);
  std::ostringstream o;
  o << "rank\ttileM\ttileN\ttileK\tthreadTileM\tthreadTileN\tscore\t"
       "estimatedLatency\tprofiledMs\tbytesA\tbytesB\tbytesC\tbytesCut\n";
  for (size_t i = 0; i < cs.size(); ++i) {
    const Candidate& c = cs[i];
    o << i << "\t" << c.tiles.tile_m << "\t" << c.tiles.tile_n << "\t" << c.tiles.tile_k << "\t"
      << c.tiles.thread_tile_m << "\t" << c.tiles.thread_tile_n << "\t" << c.score << "\t"
      << c.estimated_latency << "\t" << c.profiled_ms << "\t" << c.bytes_a << "\t" << c.bytes_b
      << "\t" << c.bytes_c << "\t" << c.bytes_cut << "\n";
  }
  if (!write_file(path, o.str())) {
    err = "failed to open candidates tsv: " + path;
    return false;
  }
  return true;
}

}  // namespace wtc

extern "C" int welder_solver_solve_typical_chain(
    const char* input_mlir_path, const char* best_summary_json_path,
    const char* candidates_tsv_path, int64_t max_connect_level, int verbose,
    int64_t* out_tile_m, int64_t* out_tile_n, int64_t* out_tile_k,
    int64_t* out_thread_tile_m, int64_t* out_thread_tile_n, char* error_buffer,
    size_t error_buffer_size) {
  using namespace wtc;
  set_error(error_buffer, error_buffer_size, "");
  if (!input_mlir_path || !*input_mlir_path) {
    set_error(error_buffer, error_buffer_size, "input_mlir_path is empty");
    return 1;
  }
  if (!best_summary_json_path || !*best_summary_json_path) {
    set_error(error_buffer, error_buffer_size, "best_summary_json_path is empty");
    return 1;
  }
  if (!candidates_tsv_path || !*candidates_tsv_path) {
    set_error(error_buffer, error_buffer_size, "candidates_tsv_path is empty");
    return 1;
  }
  if (!out_tile_m || !out_tile_n || !out_tile_k || !out_thread_tile_m || !out_thread_tile_n) {
    set_error(error_buffer, error_buffer_size, "output tile pointers are null");
    return 1;
  }
  std::string text, diag;
  if (!read_file(input_mlir_path, text)) {
    set_error(error_buffer, error_buffer_size,
              std::string("cannot open input MLIR: ") + input_mlir_path);
    return 2;
  }
  ChainSpec spec;
  if (!recognize_chain(text, spec, diag)) {
    set_error(error_buffer, error_buffer_size,
              std::string("failed to parse MLIR: ") + input_mlir_path + " (" + diag + ")");
    return 2;
  }
  ArchInfo arch;
  const std::vector<Candidate> cs = solve(spec, std::max<int64_t>(0, max_connect_level), arch);
  if (cs.empty()) {
    set_error(error_buffer, error_buffer_size, "solver returned no valid candidates");
    return 3;
  }
  std::string err;
  if (!write_best_summary(spec, arch, cs.front(), best_summary_json_path, err) ||
      !write_candidates(cs, candidates_tsv_path, err)) {
    set_error(error_buffer, error_buffer_size, err);
    return 4;
  }
  if (verbose) {
    std::fprintf(stderr, "[wtc-solver] %zu candidate(s); best %lldx%lldx%lld (%s), est %.2f us\n",
                 cs.size(), (long long)cs.front().tiles.tile_m, (long long)cs.front().tiles.tile_n,
                 (long long)cs.front().tiles.tile_k, cs.front().path.c_str(),
                 cs.front().estimated_latency);
  }
  *out_tile_m = cs.front().tiles.tile_m;
  *out_tile_n = cs.front().tiles.tile_n;
  *out_tile_k = cs.front().tiles.tile_k;
  *out_thread_tile_m = cs.front().tiles.thread_tile_m;
  *out_thread_tile_n = cs.front().tiles.thread_tile_n;
  return 0;
}
