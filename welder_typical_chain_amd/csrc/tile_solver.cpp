// tile_solver.cpp -- the search boundary: gfx950 tile variants, best.json I/O,
// the cost model, and welder_solver_solve_typical_chain.
//
// Replaces the Welder solver behind the same C symbol
// (backend/welder/compiler/solver/WelderSolverCAPI.cpp:104-196).  The
// reference searches a large tile space with an analytic traffic model
// (solveGeneric, solver/WelderSolverSolveEntrypoints.h:157-265) because it
// generates code for any tile; here the kernels are hand-written, so the space
// is the set of built variants and the model is a latency estimate
// calibrated on MI355X (variants.cpp).
#include <algorithm>
#include <cmath>
#include <filesystem>
#include <fstream>
#include <regex>
#include <sstream>

#include "chain_spec.h"
#include "variants.h"
#include "wtc/welder_solver_capi.h"
#include "wtc/wtc_hip.h"

namespace wtc {

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
// ranking
// ---------------------------------------------------------------------------
// One candidate per kernel variant that can run the chain: its tiles, the
// fused path and latency the calibrated cost model gives it (the same
// ranking the launcher's AUTO path uses), and the HBM-side bytes of that
// path in the reference's four columns (compiler/solver/WelderSolverCAPI.cpp:87-97):
// A as streamed by every column tile, B as streamed by every row block, the
// output as written (and, on the split path, re-read and rewritten), and the
// f32 logits a fused path never writes.
std::vector<Candidate> solve(const ChainSpec& s, int64_t /*max_connect_level*/,
                             const ArchInfo& arch) {
  std::vector<Candidate> out;
  const int in_code = elem_to_dtype_code(s.in), out_code = elem_to_dtype_code(s.out);
  if (in_code < 0 || out_code < 0) return out;
  const int64_t isz = elem_bytes(s.in), osz = elem_bytes(s.out);
  const Problem pr{s.batch, s.m, s.n, s.k, in_code, out_code, (int)arch.num_cu, 1};
  const double flop = 2.0 * (double)s.batch * (double)s.m * (double)s.n * (double)s.k;
  for (const VariantDesc& v : variants_for(in_code)) {
    const std::vector<Choice> cs = rank_choices(pr, WTC_PATH_AUTO, v.id);
    if (cs.empty()) continue;
    const Choice& c = cs.front();
    const int64_t nrb = (s.m + v.tile_rows - 1) / v.tile_rows;
    const int64_t nt = (s.n + v.tile_n - 1) / v.tile_n;  // the variant's column tiles
    Candidate cand;
    cand.tiles = TileParams{v.tile_m, v.tile_n, v.tile_k, v.thread_tile_m, v.thread_tile_n};
    cand.variant = v.name;
    cand.path = c.path == WTC_PATH_EXCHANGE ? "exchange" : (c.path == WTC_PATH_SPLIT ? "split" : "rows");
    if (c.path == WTC_PATH_ROWS) {
      // the row block's A stays in LDS; B streams once per pass
      cand.bytes_a = s.batch * s.m * s.k * isz;
      cand.bytes_b = s.batch * s.k * s.n * isz * nrb * 2;
    } else {
      cand.bytes_a = s.batch * s.m * s.k * isz * nt;
      cand.bytes_b = s.batch * s.k * s.n * isz * nrb;
    }
    cand.bytes_c = s.batch * s.m * s.n * osz * (c.path == WTC_PATH_SPLIT ? 3 : 1);
    cand.bytes_cut = s.batch * s.m * s.n * 4;
    cand.estimated_latency = c.est_us;
    cand.score = c.est_us > 0 ? flop / (c.est_us * 1e6) : 0.0;
    out.push_back(cand);
  }
  std::stable_sort(out.begin(), out.end(), [](const Candidate& a, const Candidate& b) {
    return a.estimated_latency < b.estimated_latency;
  });
  return out;
}

bool write_best_summary(const ChainSpec& s, const ArchInfo& arch, const Candidate& best,
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
    << ", \"bytesCut\": " << best.bytes_cut << ", \"path\": \"" << best.path
    << "\", \"variant\": \"" << best.variant << "\"}\n";
  o << "}\n";
  if (!write_file(path, o.str())) {
    err = "failed to open best summary json: " + path;
    return false;
  }
  return true;
}

// 13 columns, as backend/welder/compiler/solver/WelderSolverCAPI.cpp:87-97.
bool write_candidates(const std::vector<Candidate>& cs, const std::string& path,
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
    for (size_t i = 0; i < cs.size(); ++i)
      std::fprintf(stderr, "[wtc-solver] %zu: %s (%lldx%lldx%lld, lane %lldx%lld) on %s, est %.2f us\n",
                   i, cs[i].variant.c_str(), (long long)cs[i].tiles.tile_m,
                   (long long)cs[i].tiles.tile_n, (long long)cs[i].tiles.tile_k,
                   (long long)cs[i].tiles.thread_tile_m, (long long)cs[i].tiles.thread_tile_n,
                   cs[i].path.c_str(), cs[i].estimated_latency);
  }
  *out_tile_m = cs.front().tiles.tile_m;
  *out_tile_n = cs.front().tiles.tile_n;
  *out_tile_k = cs.front().tiles.tile_k;
  *out_thread_tile_m = cs.front().tiles.thread_tile_m;
  *out_thread_tile_n = cs.front().tiles.thread_tile_n;
  return 0;
}
