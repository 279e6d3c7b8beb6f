// wtc_compiler.cpp -- the wtc-compiler command line: the typical-chain
// pipeline driver of the reference (options of compiler/main.cpp:10-90,
// stages of compiler/pipeline/PipelineRunner.cpp:52-219) over this library.
//
// Stages and output layout (<out>/ir, <out>/search, <out>/{fused|baseline})
// follow the reference; what runs in each stage is this build's own:
//   canonicalize  text-level recognition of the chain (no mlir-opt) and the
//                 canonical decomposed form  -> ir/01.canonicalized.mlir, .log
//   tagging       wtc.tag comments + tags JSON -> ir/02.tagged.mlir, 02.tags.json
//   search        welder_solver_solve_typical_chain over the gfx950 kernel
//                 variants -> search/best_summary.json, candidates.tsv, solver.log
//                 (skipped with --best-json or --no-search), then tile overrides
//                 and search/best.json
//   compile       welder_compile_typical_chain_to_nvvm -> <dir>/03..05, kernel_report.txt
//   validate      the artefacts exist and are non-empty -> postbufferize_report.txt
// Modes: full (all stages), --search-only (stop after best.json),
// --compile-only (the reference's semantics: search only when no tiles are given).
// --backend-root / --backend-mode / --pure-api-full are accepted for
// compatibility; there is one in-process backend.
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <filesystem>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "chain_spec.h"
#include "variants.h"
#include "wtc/welder_compile_capi.h"
#include "wtc/welder_solver_capi.h"
#include "wtc/wtc_hip.h"

namespace {

namespace fs = std::filesystem;

enum class Mode { Full, SearchOnly, CompileOnly };

struct Options {
  std::string input;
  std::string output_dir = "/tmp/wtc_out";
  std::string backend_root;
  std::string backend_mode = "process_chain";
  std::string best_json;
  int64_t max_connect_level = 1;
  wtc::TileParams override_tiles;
  bool enable_search = true;
  bool fused = true;
  bool pure_api_full = false;
  Mode mode = Mode::Full;
  bool verbose = false;
  // measure the top-ranked candidates on the GPU and keep the fastest
  bool enable_profiling = false;
  int64_t profile_top_k = 4, profile_warmup = 20, profile_iters = 200;
};

int count_of(const std::string& text, const char* needle) {
  int n = 0;
  const std::string nd(needle);
  for (size_t p = text.find(nd); p != std::string::npos; p = text.find(nd, p + nd.size())) ++n;
  return n;
}

bool contains(const std::string& text, const char* needle) {
  return text.find(needle) != std::string::npos;
}

// Stage 1.  The reference runs mlir-opt --canonicalize (after decomposing a
// named linalg.softmax) and checks that matmul, exp and divf survive
// (compiler/ir/ChainCanonicalize.cpp:77-163); here the chain is recognised
// from the text and re-emitted in canonical decomposed form, then the same
// checks run on the result.
bool canonicalize(const std::string& input, const fs::path& out_mlir, wtc::ChainSpec& spec,
                  std::string& diag) {
  std::string text;
  if (!fs::exists(input)) {
    diag = "input file not found: " + input;
    return false;
  }
  if (!wtc::read_file(input, text) || text.empty()) {
    diag = "failed to read input MLIR: " + input;
    return false;
  }
  std::string why;
  const bool ok = wtc::recognize_chain(text, spec, why);
  std::ostringstream log;
  log << "[wtc canonicalize] input " << input << "\n";
  if (!ok) {
    log << "[wtc canonicalize] not a Matmul -> row-Softmax chain: " << why << "\n";
    wtc::write_file((out_mlir.parent_path() / "01.canonicalize.log").string(), log.str());
    diag = "chain not recognised: " + why + ", see " +
           (out_mlir.parent_path() / "01.canonicalize.log").string();
    return false;
  }
  const std::string canonical = wtc::emit_canonical_mlir(spec);
  log << "[wtc canonicalize] batch=" << spec.batch << " m=" << spec.m << " n=" << spec.n
      << " k=" << spec.k << " in=" << wtc::elem_mlir_name(spec.in)
      << " acc=" << wtc::elem_mlir_name(spec.acc) << " out=" << wtc::elem_mlir_name(spec.out)
      << " softmax=" << (spec.form == wtc::SoftmaxForm::Named ? "named (decomposed)" : "decomposed")
      << " logit_scale=" << spec.logit_scale
      << (spec.runtime_scales ? " runtime_scales" : "") << "\n";
  if (!wtc::write_file(out_mlir.string(), canonical) ||
      !wtc::write_file((out_mlir.parent_path() / "01.canonicalize.log").string(), log.str())) {
    diag = "failed to write " + out_mlir.string();
    return false;
  }
  if (!contains(canonical, "linalg.matmul") && !contains(canonical, "linalg.batch_matmul")) {
    diag = "canonicalize: the chain's matmul is missing from " + out_mlir.string();
    return false;
  }
  if (contains(canonical, "linalg.softmax")) {
    diag = "canonicalize: a named linalg.softmax is still present in " + out_mlir.string() + " (it must be decomposed)";
    return false;
  }
  if (!contains(canonical, "math.exp") || !contains(canonical, "arith.divf")) {
    diag = "canonicalize: " + out_mlir.string() + " lacks the exponential (math.exp) or the division (arith.divf) of a decomposed softmax";
    return false;
  }
  return true;
}

// Stage 2 (compiler/ir/Tagging.cpp:50-159): tags the canonicalized file.
bool tag(const fs::path& canonical_path, const wtc::ChainSpec& spec, const fs::path& tagged_path,
         const fs::path& tags_json_path, std::string& diag) {
  std::string text;
  if (!wtc::read_file(canonical_path.string(), text) || text.empty()) {
    diag = "tag: cannot read " + canonical_path.string() + " (missing or empty)";
    return false;
  }
  if ((count_of(text, "linalg.matmul") + count_of(text, "linalg.batch_matmul")) == 0 ||
      count_of(text, "linalg.generic") == 0) {
    diag = "tag: " + canonical_path.string() + " needs a matmul followed by linalg.generic softmax stages";
    return false;
  }
  std::string tagged, tags_json;
  wtc::tag_chain(text, spec, canonical_path.string(), tagged, tags_json);
  if (!wtc::write_file(tagged_path.string(), tagged)) {
    diag = "tag: cannot write " + tagged_path.string();
    return false;
  }
  if (!wtc::write_file(tags_json_path.string(), tags_json)) {
    diag = "tag: cannot write " + tags_json_path.string();
    return false;
  }
  return true;
}

// The validation stage (compiler/runtime/PostbufferizeFixups.cpp:33-89),
// re-targeted to the HIP artefacts: counts from the canonical IR, the launch
// plan and the kernel report instead of post-bufferize IR, gpu.launch and PTX.
bool validate(const fs::path& dir, std::string& diag) {
  // the files the reference's callers require, then this build's HIP files
  const char* names[] = {"03.after_postbufferize.mlir", "04.after_workgroup_launch.mlir",
                         "05.out.nvvm.runnable.mlir", "03.chain.canonical.mlir",
                         "04.kernel.plan.json", "05.out.hip.launch.json"};
  std::string text[6];
  for (int i = 0; i < 6; ++i)
    if (!wtc::read_file((dir / names[i]).string(), text[i]) || text[i].empty()) {
      diag = std::string(names[i]) + " is missing or empty in " + dir.string();
      return false;
    }
  const std::string& c = text[0];
  const std::string& p = text[4];
  const fs::path kreport = dir / "kernel_report.txt";
  std::string k;
  wtc::read_file(kreport.string(), k);
  auto report_value = [&](const char* key) -> std::string {
    const std::string needle = std::string(key) + "=";
    const size_t at = k.find(needle);
    if (at == std::string::npos) return "0";
    const size_t end = k.find('\n', at);
    return k.substr(at + needle.size(), end == std::string::npos ? std::string::npos
                                                                 : end - at - needle.size());
  };
  std::ostringstream r;
  r << "post_matmul_count=" << count_of(c, "linalg.matmul") + count_of(c, "linalg.batch_matmul")
    << "\n";
  r << "launch_kernel_count=" << count_of(p, "\"name\":") << "\n";
  r << "launch_scratch_bytes=" << report_value("scratch_bytes") << "\n";
  r << "mfma_instruction_count=" << report_value("mfma_instruction_count") << "\n";
  r << "scratch_instruction_count=" << report_value("scratch_instruction_count") << "\n";
  r << "vgpr_spill_count=" << report_value("vgpr_spill_count") << "\n";
  if (!wtc::write_file((dir / "postbufferize_report.txt").string(), r.str())) {
    diag = "could not write " + (dir / "postbufferize_report.txt").string();
    return false;
  }
  return true;
}

// The profile step: time the first `profile_top_k` candidates of the model's
// ranking on the current device (wtc_profile_tiles), put the measured ones
// first, fastest first, and rewrite the search outputs.  A failed
// measurement (no GPU, say) ends the step and keeps the model's ranking, as
// the reference falls back to its heuristic cost for a candidate that fails
// to compile or profile unless told to prune it
// (backend/welder/compiler/driver/WelderCompilerCliOptions.h:333-336).
bool profile_candidates(const Options& o, const wtc::ChainSpec& spec, const fs::path& summary,
                        const fs::path& candidates, const fs::path& search, wtc::TileParams& best) {
  wtc::ArchInfo arch;
  std::vector<wtc::Candidate> cs = wtc::solve(spec, o.max_connect_level, arch);
  const int in = wtc::elem_to_dtype_code(spec.in), out = wtc::elem_to_dtype_code(spec.out);
  std::ostringstream log;
  size_t measured = 0;
  for (size_t i = 0; i < cs.size() && (int64_t)i < o.profile_top_k; ++i) {
    const wtc::TileParams& t = cs[i].tiles;
    const wtc_tiles tiles{t.tile_m, t.tile_n, t.tile_k, t.thread_tile_m, t.thread_tile_n};
    const int path = cs[i].path == "exchange" ? WTC_PATH_EXCHANGE
                     : cs[i].path == "split"  ? WTC_PATH_SPLIT
                                              : WTC_PATH_ROWS;
    double us = 0;
    const int rc = wtc_profile_tiles(spec.batch, spec.m, spec.n, spec.k, in, out, &tiles, path,
                                     (int)o.profile_warmup, (int)o.profile_iters, 0x5EEDull + i, &us);
    log << "[wtc.profile] " << cs[i].variant << " " << cs[i].path << " rc=" << rc;
    if (rc != 0) {
      log << " error=" << wtc_last_error() << " (model ranking kept from here on)\n";
      break;
    }
    log << " us=" << us << " estimated_us=" << cs[i].estimated_latency << "\n";
    cs[i].profiled_ms = us / 1000.0;
    ++measured;
  }
  wtc::write_file((search / "profile.log").string(), log.str());
  if (o.verbose) std::cout << log.str();
  if (measured == 0) return true;
  std::stable_sort(cs.begin(), cs.begin() + measured, [](const wtc::Candidate& a, const wtc::Candidate& b) {
    return a.profiled_ms < b.profiled_ms;
  });
  std::string err;
  if (!wtc::write_best_summary(spec, arch, cs.front(), summary.string(), err) ||
      !wtc::write_candidates(cs, candidates.string(), err)) {
    std::cerr << "wtc-compiler: " << err << "\n";
    return false;
  }
  best = cs.front().tiles;
  return true;
}

bool any_override(const wtc::TileParams& t) {
  return t.tile_m > 0 || t.tile_n > 0 || t.tile_k > 0 || t.thread_tile_m > 0 ||
         t.thread_tile_n > 0;
}

int run_pipeline(const Options& o) {
  std::string diag;
  if (o.output_dir.empty()) {
    std::cerr << "wtc-compiler: no output directory given\n";
    return 1;
  }
  const fs::path root = o.output_dir;
  const fs::path ir = root / "ir", search = root / "search";
  const fs::path compile_dir = root / (o.fused ? "fused" : "baseline");
  std::error_code ec;
  fs::create_directories(ir, ec);
  if (ec) {
    std::cerr << "wtc-compiler: could not create directory " << ir << "\n";
    return 1;
  }

  if (o.verbose) std::cout << "[wtc-compiler] recognising the chain\n";
  wtc::ChainSpec spec;
  const fs::path canonical = ir / "01.canonicalized.mlir";
  if (!canonicalize(o.input, canonical, spec, diag)) {
    std::cerr << "wtc-compiler: the input is not a Matmul -> row-Softmax chain: " << diag << "\n";
    return 1;
  }
  if (o.verbose) std::cout << "[wtc-compiler] writing the tagged chain\n";
  const fs::path tagged = ir / "02.tagged.mlir";
  if (!tag(canonical, spec, tagged, ir / "02.tags.json", diag)) {
    std::cerr << "wtc-compiler: could not write the tagged chain: " << diag << "\n";
    return 1;
  }

  fs::create_directories(search, ec);
  // The backend consumes the canonicalized + tagged input, as in the reference.
  const std::string backend_input = tagged.string();
  wtc::TileParams best;
  bool have_best = false;
  if (!o.best_json.empty()) {
    if (o.verbose) std::cout << "[wtc-compiler] tiles from " << o.best_json << "\n";
    if (!wtc::load_best_json(o.best_json, best, diag)) {
      std::cerr << "wtc-compiler: --best-json unreadable: " << diag << "\n";
      return 1;
    }
    have_best = true;
  }
  if (!have_best && o.enable_search) {
    if (o.verbose) std::cout << "[wtc-compiler] ranking the gfx950 tile variants\n";
    const fs::path summary = search / "best_summary.json", candidates = search / "candidates.tsv";
    const fs::path solver_log = search / "solver.log";
    char err[4096];
    const int rc = welder_solver_solve_typical_chain(
        backend_input.c_str(), summary.c_str(), candidates.c_str(), o.max_connect_level,
        o.verbose ? 1 : 0, &best.tile_m, &best.tile_n, &best.tile_k, &best.thread_tile_m,
        &best.thread_tile_n, err, sizeof err);
    std::ostringstream log;
    log << "[wtc.search] input=" << backend_input << "\n[wtc.search] max_connect_level="
        << o.max_connect_level << "\n[wtc.search] rc=" << rc << (rc ? std::string(" error=") + err : "")
        << "\n";
    wtc::write_file(solver_log.string(), log.str());
    if (rc != 0) {
      std::cerr << "wtc-compiler: the tile solver returned " << rc << " (" << err << "); log in "
                << solver_log.string() << "\n";
      return 1;
    }
    have_best = true;
    if (o.verbose) {
      std::cout << "[wtc-compiler] ranked candidates in " << candidates.string() << "\n";
    }
    if (o.enable_profiling && !profile_candidates(o, spec, summary, candidates, search, best))
      return 1;
  }
  if (any_override(o.override_tiles)) {
    if (o.verbose) std::cout << "[wtc-compiler] tiles overridden on the command line\n";
    const wtc::TileParams& t = o.override_tiles;
    if (t.tile_m > 0) best.tile_m = t.tile_m;
    if (t.tile_n > 0) best.tile_n = t.tile_n;
    if (t.tile_k > 0) best.tile_k = t.tile_k;
    if (t.thread_tile_m > 0) best.thread_tile_m = t.thread_tile_m;
    if (t.thread_tile_n > 0) best.thread_tile_n = t.thread_tile_n;
    have_best = true;
  }
  if (!have_best && o.mode == Mode::SearchOnly) {
    std::cerr << "wtc-compiler: --search-only needs the solver or --best-json to produce tiles\n";
    return 1;
  }
  if (!have_best) {
    // search disabled and no tiles given: the library's default variant for the input type
    const std::vector<wtc::VariantDesc> vs = wtc::variants_for(wtc::elem_to_dtype_code(spec.in));
    if (vs.empty()) {
      std::cerr << "wtc-compiler: no kernel variant for the chain's input type\n";
      return 1;
    }
    best = wtc::TileParams{vs.front().tile_m, vs.front().tile_n, vs.front().tile_k,
                           vs.front().thread_tile_m, vs.front().thread_tile_n};
    if (o.verbose) std::cout << "[wtc-compiler] no search: the default variant of the input type\n";
  }
  const fs::path best_path = search / "best.json";
  if (!wtc::write_best_json(best, best_path.string(), diag)) {
    std::cerr << "wtc-compiler: could not write best.json: " << diag << "\n";
    return 1;
  }
  if (o.verbose)
    std::cout << "[wtc-compiler] tiles " << best.tile_m << "x" << best.tile_n << "x" << best.tile_k
              << ", lane tile " << best.thread_tile_m << "x" << best.thread_tile_n << "\n";
  if (o.mode == Mode::SearchOnly) {
    std::cout << "[wtc-compiler] tiles written to " << best_path.string() << "\n";
    return 0;
  }

  if (o.verbose) std::cout << "[wtc-compiler] planning the gfx950 launch\n";
  fs::create_directories(compile_dir, ec);
  char err[4096];
  const int rc = welder_compile_typical_chain_to_nvvm(
      backend_input.c_str(), compile_dir.c_str(), "", "", best.tile_m, best.tile_n, best.tile_k,
      best.thread_tile_m, best.thread_tile_n, o.fused ? o.max_connect_level : 0, o.fused ? 1 : 0,
      o.verbose ? 1 : 0, err, sizeof err);
  std::ostringstream clog;
  clog << "[wtc.compile] input=" << backend_input << " out=" << compile_dir.string()
       << " fused=" << (o.fused ? 1 : 0) << " tiles=" << best.tile_m << "x" << best.tile_n << "x"
       << best.tile_k << "/" << best.thread_tile_m << "x" << best.thread_tile_n << " rc=" << rc
       << (rc ? std::string(" error=") + err : "") << "\n";
  wtc::write_file((compile_dir / "compile.log").string(), clog.str());
  if (rc != 0) {
    std::cerr << "wtc-compiler: the compile entry point returned " << rc << ": " << err << "\n";
    return 1;
  }
  if (o.verbose) std::cout << "[wtc-compiler] checking the artefacts\n";
  if (!validate(compile_dir, diag)) {
    std::cerr << "wtc-compiler: artefact check failed: " << diag << "\n";
    return 1;
  }
  std::cout << "[wtc-compiler] done: " << (compile_dir / "05.out.nvvm.runnable.mlir").string() << "\n";
  return 0;
}

void usage() {
  std::cout << "wtc-compiler: tile selection and gfx950 launch planning for a Matmul -> row-Softmax\n"
            << "chain given as MLIR text.\n\n"
            << "  wtc-compiler --input FILE [--output-dir DIR] [mode] [tiles] [--repeat N] [--verbose]\n\n"
            << "modes (default: rank the tile variants, then plan and check the launch):\n"
            << "  --search-only             stop after writing search/best.json\n"
            << "  --compile-only            plan with the tiles given (rank only if none are)\n"
            << "  --no-search               take the input type's default variant when no tiles are given\n"
            << "  --fused | --baseline      one fused kernel (default) or the five-kernel unfused chain\n"
            << "tiles:\n"
            << "  --best-json FILE          tileM/tileN/tileK/threadTileM/threadTileN from a JSON file\n"
            << "  --tile-m N  --tile-n N  --tile-k N  --thread-tile-m N  --thread-tile-n N\n"
            << "  --max-connect-level N     recorded in the plan (the fused kernel needs none)\n"
            << "profiling (needs a GPU; the ranking stays the model's where it fails):\n"
            << "  --enable-profiling        time the first candidates on the device, rank them by\n"
            << "                            measured time (candidates.tsv profiledMs), keep the fastest\n"
            << "  --profile-top-k N  --profile-warmup N  --profile-iters N   (4, 20, 200)\n"
            << "accepted and ignored (a single in-process backend):\n"
            << "  --backend-root DIR  --legacy-root DIR  --backend-mode MODE  --pure-api-full\n"
            << "output layout: DIR/ir (01, 02), DIR/search (best.json, best_summary.json,\n"
            << "candidates.tsv), DIR/fused or DIR/baseline (03, 04, 05 and the HIP files);\n"
            << "--repeat N runs the pipeline N times in one process, into DIR/iter_<i>.\n";
}

bool parse_int(const char* s, int64_t& v) {
  try {
    size_t used = 0;
    v = std::stoll(s, &used);
    return used == std::string(s).size();
  } catch (...) {
    return false;
  }
}

}  // namespace

int main(int argc, char** argv) {
  Options o;
  int64_t repeat = 1;
  for (int i = 1; i < argc; ++i) {
    const std::string arg = argv[i];
    const bool has_value = i + 1 < argc;
    auto int_arg = [&](int64_t& dst) {
      if (!parse_int(argv[++i], dst)) {
        std::cerr << "wtc-compiler: " << arg << " takes an integer, not '" << argv[i] << "'\n";
        std::exit(2);
      }
    };
    if (arg == "--input" && has_value) {
      o.input = argv[++i];
    } else if ((arg == "--output-dir" || arg == "--out-dir") && has_value) {
      o.output_dir = argv[++i];
    } else if ((arg == "--backend-root" || arg == "--legacy-root") && has_value) {
      o.backend_root = argv[++i];
    } else if (arg == "--best-json" && has_value) {
      o.best_json = argv[++i];
    } else if (arg == "--backend-mode" && has_value) {
      const std::string m = argv[++i];
      if (m != "shell" && m != "process_chain" && m != "api") {
        std::cerr << "wtc-compiler: --backend-mode is one of shell, process_chain, api (got '" << m << "')\n";
        return 2;
      }
      o.backend_mode = m;
    } else if (arg == "--max-connect-level" && has_value) {
      int_arg(o.max_connect_level);
    } else if (arg == "--tile-m" && has_value) {
      int_arg(o.override_tiles.tile_m);
    } else if (arg == "--tile-n" && has_value) {
      int_arg(o.override_tiles.tile_n);
    } else if (arg == "--tile-k" && has_value) {
      int_arg(o.override_tiles.tile_k);
    } else if (arg == "--thread-tile-m" && has_value) {
      int_arg(o.override_tiles.thread_tile_m);
    } else if (arg == "--thread-tile-n" && has_value) {
      int_arg(o.override_tiles.thread_tile_n);
    } else if (arg == "--no-search") {
      o.enable_search = false;
    } else if (arg == "--pure-api-full") {
      o.pure_api_full = true;
    } else if (arg == "--repeat" && has_value) {
      int_arg(repeat);
    } else if (arg == "--search-only") {
      o.mode = Mode::SearchOnly;
    } else if (arg == "--compile-only") {
      o.mode = Mode::CompileOnly;
    } else if (arg == "--baseline") {
      o.fused = false;
      if (o.max_connect_level > 0) o.max_connect_level = 0;
    } else if (arg == "--fused") {
      o.fused = true;
    } else if (arg == "--enable-profiling") {
      o.enable_profiling = true;
    } else if ((arg == "--profile-top-k" || arg == "--profile-warmup" || arg == "--profile-iters") &&
               has_value) {
      int64_t v = 0;
      if (!parse_int(argv[++i], v) || v < (arg == "--profile-warmup" ? 0 : 1)) {
        std::cerr << "wtc-compiler: " << arg << " needs a positive integer\n";
        return 2;
      }
      (arg == "--profile-top-k" ? o.profile_top_k
                                : (arg == "--profile-warmup" ? o.profile_warmup : o.profile_iters)) = v;
    } else if (arg == "--verbose") {
      o.verbose = true;
    } else if (arg == "--help" || arg == "-h") {
      usage();
      return 0;
    } else {
      std::cerr << "wtc-compiler: unrecognised option " << arg << "\n";
      return 2;
    }
  }
  if (o.input.empty()) {
    std::cerr << "wtc-compiler: give the chain with --input FILE\n";
    return 2;
  }
  if (repeat <= 0) {
    std::cerr << "wtc-compiler: --repeat takes a count of at least 1\n";
    return 2;
  }
  if (repeat == 1) return run_pipeline(o);
  for (int64_t i = 0; i < repeat; ++i) {
    Options it = o;
    it.output_dir = (fs::path(o.output_dir) / ("iter_" + std::to_string(i))).string();
    if (o.verbose)
      std::cout << "[wtc] pipeline run " << (i + 1) << " of " << repeat << " into " << it.output_dir
                << "\n";
    const int rc = run_pipeline(it);
    if (rc != 0) {
      std::cerr << "wtc-compiler: run " << i << " of --repeat ended with status " << rc << "\n";
      return rc;
    }
  }
  return 0;
}
