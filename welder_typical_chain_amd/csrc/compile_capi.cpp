// compile_capi.cpp -- welder_compile_typical_chain_to_nvvm for the gfx950
// kernel library: recognise the chain, check the tiles against the
// instantiated kernel variants, plan the launch and write the stage
// artefacts.  Reference: backend/welder/compiler/driver/WelderCompileCAPI.cpp:20-71
// (argument checks and return codes) and driver/WelderCompileSession.cpp:239-330
// (the session that writes the stage files into out_dir).
#include <dlfcn.h>

#include <cstdio>
#include <filesystem>
#include <sstream>

#include "chain_spec.h"
#include "wtc/welder_compile_capi.h"
#include "wtc/wtc_hip.h"

namespace wtc {

static std::string library_path() {
  Dl_info info{};
  if (dladdr(reinterpret_cast<void*>(&welder_compile_typical_chain_to_nvvm), &info) && info.dli_fname)
    return std::filesystem::absolute(info.dli_fname).string();
  return "libwtc_hip.so";
}

static const char* path_name(int p) {
  switch (p) {
    case WTC_PATH_EXCHANGE: return "exchange";
    case WTC_PATH_SPLIT: return "split";
    case WTC_PATH_UNFUSED: return "unfused";
    default: return "auto";
  }
}

// Resource summary of the kernels, from the kernel_resources.json the build
// writes next to the library (absent: a note says so).
static std::string resources_for(const std::string& lib) {
  std::string text;
  const std::string p = (std::filesystem::path(lib).parent_path() / "kernel_resources.json").string();
  if (!read_file(p, text)) return "kernel resources: not recorded (" + p + " missing)\n";
  return "kernel resources (" + p + "):\n" + text;
}

static int compile_impl(const char* input_mlir_path, const char* out_dir, int64_t tile_m,
                        int64_t tile_n, int64_t tile_k, int64_t thread_tile_m,
                        int64_t thread_tile_n, int64_t max_connect_level, int fused, int verbose,
                        char* error_buffer, size_t error_buffer_size) {
  set_error(error_buffer, error_buffer_size, "");
  if (!input_mlir_path || !*input_mlir_path) {
    set_error(error_buffer, error_buffer_size, "input_mlir_path is empty");
    return 1;
  }
  if (!out_dir || !*out_dir) {
    set_error(error_buffer, error_buffer_size, "out_dir is empty");
    return 1;
  }
  if (tile_m <= 0 || tile_n <= 0 || tile_k <= 0 || thread_tile_m <= 0 || thread_tile_n <= 0) {
    set_error(error_buffer, error_buffer_size, "invalid tile sizes");
    return 1;
  }
  auto session_fail = [&](const std::string& msg) {
    set_error(error_buffer, error_buffer_size, msg);
    return 2;
  };
  std::string text, diag;
  if (!read_file(input_mlir_path, text))
    return session_fail(std::string("cannot read input MLIR: ") + input_mlir_path);
  ChainSpec spec;
  if (!recognize_chain(text, spec, diag)) return session_fail("chain not recognised: " + diag);
  const TileParams tiles{tile_m, tile_n, tile_k, thread_tile_m, thread_tile_n};
  if (!is_supported(tiles, spec.in)) {
    std::ostringstream o;
    o << "no gfx950 kernel variant implements tile " << tile_m << "x" << tile_n << "x" << tile_k
      << " thread tile " << thread_tile_m << "x" << thread_tile_n << " for "
      << elem_mlir_name(spec.in) << "; available:";
    for (const Variant& v : supported_variants(spec.in))
      o << " " << v.tiles.tile_m << "x" << v.tiles.tile_n << "x" << v.tiles.tile_k << "/"
        << v.tiles.thread_tile_m << "x" << v.tiles.thread_tile_n;
    return session_fail(o.str());
  }
  const int in_code = elem_to_dtype_code(spec.in), out_code = elem_to_dtype_code(spec.out);
  // Plan for MI355X: 256 CUs, one exchange workgroup per CU.
  const int path_req = fused ? WTC_PATH_AUTO : WTC_PATH_UNFUSED;
  int64_t grid = 0, ws = 0;
  int path = 0;
  if (wtc_plan(spec.batch, spec.m, spec.n, spec.k, in_code, out_code, path_req, 256, 1, &grid,
               &path, &ws) != WTC_OK)
    return session_fail(std::string("launch plan failed: ") + wtc_last_error());

  std::error_code ec;
  std::filesystem::create_directories(out_dir, ec);
  if (ec) return session_fail(std::string("cannot create out_dir: ") + out_dir);
  const std::filesystem::path od(out_dir);
  const std::string lib = library_path();
  const std::string kin = elem_mlir_name(spec.in), kout = elem_mlir_name(spec.out);

  // kernels of the selected path
  struct K {
    std::string name;
    int64_t grid;
    int lds;
  };
  std::vector<K> ks;
  const int64_t rows = spec.batch * spec.m;
  if (path == WTC_PATH_EXCHANGE) {
    ks.push_back({"chain_tile_kernel<" + kin + "," + kout + ",exchange>", grid, 82944});
  } else if (path == WTC_PATH_SPLIT) {
    ks.push_back({"chain_tile_kernel<" + kin + "," + kout + ",split>", grid, 0});
    ks.push_back({"rescale_rows_kernel<" + kout + ">", (rows + 3) / 4, 8192});
  } else {
    ks.push_back({"chain_tile_kernel<" + kin + ",f32,logits>", grid, 0});
    ks.push_back({"rowmax_kernel", rows, 16});
    ks.push_back({"expsub_kernel", rows, 0});
    ks.push_back({"rowsum_kernel", rows, 16});
    ks.push_back({"rowdiv_kernel<" + kout + ">", rows, 0});
  }

  std::ostringstream plan;
  plan << "{\n  \"target\": \"gfx950\",\n  \"variant\": \"" << supported_variants(spec.in).front().name
       << "\",\n  \"path\": \"" << path_name(path) << "\",\n  \"fused\": " << (fused ? "true" : "false")
       << ",\n  \"max_connect_level\": " << max_connect_level << ",\n  \"tiles\": {\"tileM\": " << tile_m
       << ", \"tileN\": " << tile_n << ", \"tileK\": " << tile_k << ", \"threadTileM\": " << thread_tile_m
       << ", \"threadTileN\": " << thread_tile_n << "},\n  \"kernels\": [\n";
  for (size_t i = 0; i < ks.size(); ++i)
    plan << "    {\"name\": \"" << ks[i].name << "\", \"grid\": [" << ks[i].grid
         << ", 1, 1], \"block\": [256, 1, 1], \"dynamic_lds_bytes\": " << ks[i].lds << "}"
         << (i + 1 < ks.size() ? "," : "") << "\n";
  plan << "  ],\n  \"workspace_bytes\": " << ws << "\n}\n";

  std::ostringstream launch;
  launch << "{\n  \"format\": \"wtc-hip-launch-v1\",\n  \"target\": \"gfx950\",\n  \"library\": \"" << lib
         << "\",\n  \"entry\": \"wtc_matmul_softmax\",\n  \"problem\": {\"batch\": " << spec.batch
         << ", \"m\": " << spec.m << ", \"n\": " << spec.n << ", \"k\": " << spec.k
         << ", \"batched\": " << (spec.batched ? "true" : "false") << "},\n  \"in_dtype\": \"" << kin
         << "\",\n  \"out_dtype\": \"" << kout << "\",\n  \"chain_acc_dtype\": \"" << elem_mlir_name(spec.acc)
         << "\",\n  \"kernel_acc_dtype\": \"f32\",\n  \"dtype_codes\": {\"in\": " << in_code
         << ", \"out\": " << out_code << "},\n  \"logit_scale\": " << spec.logit_scale
         << ",\n  \"runtime_scales\": " << (spec.runtime_scales ? "true" : "false") << ",\n  \"path\": \""
         << path_name(path) << "\",\n  \"path_code\": " << path << ",\n  \"workspace_bytes\": " << ws
         << ",\n  \"softmax_form\": \"" << (spec.form == SoftmaxForm::Named ? "named" : "decomposed")
         << "\"\n}\n";

  std::ostringstream report;
  report << "chain: batch=" << spec.batch << " m=" << spec.m << " n=" << spec.n << " k=" << spec.k
         << " in=" << kin << " out=" << kout << " path=" << path_name(path) << "\n";
  report << "kernels=" << ks.size() << "\n";
  for (const K& k : ks) report << "  " << k.name << " grid=" << k.grid << " block=256\n";
  report << resources_for(lib);

  if (!write_file((od / "03.chain.canonical.mlir").string(), emit_canonical_mlir(spec)) ||
      !write_file((od / "04.kernel.plan.json").string(), plan.str()) ||
      !write_file((od / "05.out.hip.launch.json").string(), launch.str()) ||
      !write_file((od / "kernel_report.txt").string(), report.str()))
    return session_fail(std::string("failed to write artefacts into ") + out_dir);
  if (verbose)
    std::fprintf(stderr, "[wtc-compile] %s -> %s (%s, %zu kernel(s))\n", input_mlir_path, out_dir,
                 path_name(path), ks.size());
  return 0;
}

}  // namespace wtc

extern "C" int welder_compile_typical_chain_to_nvvm(
    const char* input_mlir_path, const char* out_dir, const char* /*workgroup_pass_plugin_path*/,
    const char* /*welder_compiler_bin_path*/, int64_t tile_m, int64_t tile_n, int64_t tile_k,
    int64_t thread_tile_m, int64_t thread_tile_n, int64_t max_connect_level, int fused, int verbose,
    char* error_buffer, size_t error_buffer_size) {
  return wtc::compile_impl(input_mlir_path, out_dir, tile_m, tile_n, tile_k, thread_tile_m,
                           thread_tile_n, max_connect_level, fused, verbose, error_buffer,
                           error_buffer_size);
}

extern "C" int welder_compile_typical_chain_to_hip(
    const char* input_mlir_path, const char* out_dir, const char* workgroup_pass_plugin_path,
    const char* welder_compiler_bin_path, int64_t tile_m, int64_t tile_n, int64_t tile_k,
    int64_t thread_tile_m, int64_t thread_tile_n, int64_t max_connect_level, int fused, int verbose,
    char* error_buffer, size_t error_buffer_size) {
  return welder_compile_typical_chain_to_nvvm(input_mlir_path, out_dir, workgroup_pass_plugin_path,
                                              welder_compiler_bin_path, tile_m, tile_n, tile_k,
                                              thread_tile_m, thread_tile_n, max_connect_level, fused,
                                              verbose, error_buffer, error_buffer_size);
}
