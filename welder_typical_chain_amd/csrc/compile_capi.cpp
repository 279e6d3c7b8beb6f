// compile_capi.cpp -- welder_compile_typical_chain_to_nvvm for the gfx950
// kernel library: recognise the chain, check the tiles against the
// instantiated kernel variants, plan the launch and write the stage
// artefacts.  Reference: backend/welder/compiler/driver/WelderCompileCAPI.cpp:20-71
// (argument checks and return codes) and driver/WelderCompileSession.cpp:239-330
// (the session that writes the stage files into out_dir).
#include <dlfcn.h>

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <map>
#include <sstream>
#include <utility>
#include <vector>

#include "chain_spec.h"
#include "variants.h"
#include "wtc/welder_compile_capi.h"
#include "wtc/wtc_hip.h"

namespace wtc {

// Workgroup sizes of the kernels (defined with the kernels and the launcher
// in the library).
int chain_kernel_threads(int in_dt);
int wide_kernel_threads();
int rows_kernel_threads();
int rescale_waves_per_row(int64_t rows_total, int cu_count);
// Compute units of the current device, or `fallback` when no GPU is visible.
int device_cu_count(int fallback);
// Dynamic LDS bytes the launcher adds to the exchange kernel of wave layout ks.
int exchange_lds_pad(int in_dt, int out_dt, int loaders);

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
    case WTC_PATH_ROWS: return "rows";
    default: return "auto";
  }
}

// Per-kernel resources of the library's own code objects, from the
// kernel_resources.tsv the build writes next to the library: mangled name ->
// column -> value.
using ResourceTable = std::map<std::string, std::map<std::string, std::string>>;

static bool load_resources(const std::string& lib, ResourceTable& table, std::string& where) {
  where = (std::filesystem::path(lib).parent_path() / "kernel_resources.tsv").string();
  std::string text;
  if (!read_file(where, text)) return false;
  std::istringstream in(text);
  std::string line;
  std::vector<std::string> cols;
  auto split = [](const std::string& l) {
    std::vector<std::string> v;
    std::string cell;
    std::istringstream ls(l);
    while (std::getline(ls, cell, '\t')) v.push_back(cell);
    return v;
  };
  if (!std::getline(in, line)) return false;
  cols = split(line);
  while (std::getline(in, line)) {
    const std::vector<std::string> v = split(line);
    if (v.empty()) continue;
    auto& row = table[v[0]];
    for (size_t i = 1; i < v.size() && i < cols.size(); ++i) row[cols[i]] = v[i];
  }
  return true;
}

static const std::map<std::string, std::string>* find_kernel(const ResourceTable& t,
                                                             const std::string& prefix) {
  auto it = t.lower_bound(prefix);
  if (it != t.end() && it->first.compare(0, prefix.size(), prefix) == 0) return &it->second;
  return nullptr;
}

static int64_t cell(const std::map<std::string, std::string>* row, const char* col) {
  if (!row) return 0;
  auto it = row->find(col);
  return it == row->end() ? 0 : std::strtoll(it->second.c_str(), nullptr, 10);
}

// memref type of a chain operand (rank 3 when batched).
static std::string memref_of(const ChainSpec& spec, int64_t d1, int64_t d2, Elem e) {
  std::ostringstream o;
  o << "memref<";
  if (spec.batched) o << spec.batch << "x";
  o << d1 << "x" << d2 << "x" << elem_mlir_name(e) << ">";
  return o.str();
}

// One kernel of a path as the stage files describe it.
struct StageKernel {
  std::string name;   // display name (template arguments spelled out)
  std::string kind;   // tile_exchange / tile_split / tile_logits / rows / rescale / rowmax / ...
  int64_t grid;
  int block;
  int64_t lds;        // static + dynamic LDS bytes
};

// 04c.after_linalg_to_loops.mlir: the loop nests of the path's kernels as
// this build runs them, with this problem's bounds (the reference's file at
// this stage is its chain lowered to loops; here the loops are those of the
// hand-written gfx950 kernels, the bodies named by the instructions they issue).
static std::string emit_loop_structure(const ChainSpec& spec, const VariantDesc& var, int in_code,
                                       const char* path, const std::vector<StageKernel>& ks) {
  const int64_t eb = in_code == WTC_DTYPE_FP8_E4M3 ? 1 : in_code == WTC_DTYPE_F32 ? 4 : 2;
  const int64_t tk = 128 / eb;                                  // elements of one 128-byte k-tile
  const int64_t nk = (spec.k * eb + 127) / 128;                 // k-tiles
  const int64_t tm = var.tile_rows, tn = var.id == kVarTile256x256 ? 256 : 128;
  const int64_t rows = spec.batch * spec.m, nT = (spec.n + tn - 1) / tn;
  const char* mfma = in_code == WTC_DTYPE_FP8_E4M3 ? "v_mfma_scale_f32_32x32x64_f8f6f4"
                     : in_code == WTC_DTYPE_BF16 ? "v_mfma_f32_32x32x16_bf16"
                     : in_code == WTC_DTYPE_F32 ? "v_mfma_f32_32x32x2f32" : "v_mfma_f32_32x32x16_f16";
  const int64_t ksteps = in_code == WTC_DTYPE_FP8_E4M3 ? 2 : in_code == WTC_DTYPE_F32 ? 16 : 4;
  std::ostringstream o;
  o << "// Loop structure of the " << path << " path's kernels on gfx950 (variant " << var.name
    << "),\n// with this problem's bounds: batch " << spec.batch << ", M " << spec.m << ", N " << spec.n
    << ", K " << spec.k << ".  Each func is one HIP kernel; scf.parallel is its grid.\n"
    << "module attributes {wtc.target = \"gfx950\", wtc.path = \"" << path << "\"} {\n";
  int ind = 4;  // constants are declared at the depth of the loop that uses them
  auto c = [&](const char* nm, int64_t v) {
    o << std::string(ind, ' ') << "%" << nm << " = arith.constant " << v << " : index\n";
  };
  for (size_t i = 0; i < ks.size(); ++i) {
    const StageKernel& k = ks[i];
    o << "  // " << k.name << ": grid " << k.grid << " x " << k.block << " threads, " << k.lds
      << " bytes of LDS\n  func.func @kernel" << i << "() {\n";
    c("c0", 0);
    c("c1", 1);
    c("grid", k.grid);
    c("c2", 2);
    o << "    scf.parallel (%wg) = (%c0) to (%grid) step (%c1) {\n";
    ind = 6;
    if (k.kind.rfind("tile_", 0) == 0) {
      c("nk", nk);
      c("ks", ksteps);
      c("tm", tm);
      c("tn", tn);
      o << "      // workgroup -> (row block, column tile) of " << tm << "x" << tn
        << ", XCD-aware order\n"
        << "      scf.for %kt = %c0 to %nk step %c1 {  // k-tiles of " << tk
        << " elements: direct-to-LDS buffer loads of k-tile kt+3 into the LDS ring\n"
        << "        scf.for %s = %c0 to %ks step %c1 {  // LDS fragment reads (B: ds_read_b64_tr), "
        << mfma << ", f32 accumulators\n        }\n      }\n";
      if (k.kind == "tile_logits") {
        o << "      scf.for %r = %c0 to %tm step %c1 {  // logits scale*acc in f32: 16-byte stores\n"
          << "        scf.for %n = %c0 to %tn step %c1 {\n        }\n      }\n";
      } else {
        o << "      scf.for %r = %c0 to %tm step %c1 {  // row statistics over the tile's columns: "
             "max, exp2(fma(acc, c2, -max)), sum\n"
          << "        scf.for %n = %c0 to %tn step %c1 {\n        }\n      }\n";
        if (k.kind == "tile_exchange") {
          c("nT", nT);
          o << "      scf.for %q = %c0 to %nT step %c1 {  // row exchange: tagged log-sum-exp entries "
               "of the row block's tiles, polled\n      }\n"
            << "      scf.for %r = %c0 to %tm step %c1 {  // out = exp2(y - max) * exp2(max - lse): "
               "16-byte non-temporal stores\n"
            << "        scf.for %n = %c0 to %tn step %c1 {\n        }\n      }\n";
        } else {
          o << "      scf.for %r = %c0 to %tm step %c1 {  // exp2(y - tile max) stored; per-row "
               "(max, sum) of the tile to the workspace\n"
            << "        scf.for %n = %c0 to %tn step %c1 {\n        }\n      }\n";
        }
      }
    } else if (k.kind == "rows") {
      c("nT", (spec.n + 127) / 128);
      c("ks", (spec.k + 15) / 16);
      o << "      // one 128-row block over all of N; A staged in LDS once\n"
        << "      scf.for %pass = %c0 to %c2 step %c1 {  // pass 0: online row max/sum; pass 1: "
           "exp2(y - max - log2 sum) stored\n"
        << "        scf.for %t = %c0 to %nT step %c1 {  // 128-column B tiles through a 3-stage "
           "direct-to-LDS ring\n"
        << "          scf.for %s = %c0 to %ks step %c1 {  // " << mfma << "\n          }\n"
        << "        }\n      }\n";
    } else if (k.kind == "rescale") {
      c("n", spec.n);
      c("nT", nT);
      o << "      // waves of one row: merge the row's " << nT << " tile statistics, then rescale\n"
        << "      scf.for %q = %c0 to %nT step %c1 {\n      }\n"
        << "      scf.for %j = %c0 to %n step %c1 {  // out *= exp2(m_t - M) / S, 16-byte loads and "
           "stores in place\n      }\n";
    } else {
      c("n", spec.n);
      o << "      scf.for %j = %c0 to %n step %c1 {  // " << k.kind << " over row wg of " << rows
        << " rows\n      }\n";
    }
    o << "      scf.reduce\n    }\n    return\n  }\n";
    ind = 4;
  }
  o << "}\n";
  return o.str();
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
  const int in_code = elem_to_dtype_code(spec.in), out_code = elem_to_dtype_code(spec.out);
  VariantDesc var{};
  if (!find_variant(in_code, tile_m, tile_n, tile_k, thread_tile_m, thread_tile_n, &var)) {
    std::ostringstream o;
    o << "no gfx950 kernel variant implements tile " << tile_m << "x" << tile_n << "x" << tile_k
      << " thread tile " << thread_tile_m << "x" << thread_tile_n << " for "
      << elem_mlir_name(spec.in) << "; available:";
    for (const VariantDesc& v : variants_for(in_code))
      o << " " << v.tile_m << "x" << v.tile_n << "x" << v.tile_k << "/" << v.thread_tile_m << "x"
        << v.thread_tile_n << " (" << v.name << ")";
    return session_fail(o.str());
  }
  // Plan for the current device (MI355X's 256 CUs without one); the
  // exchange kernel's LDS footprint holds one of its workgroups per CU.  The
  // fused chain runs the variant of the given tiles on the path the cost
  // model ranks first for it.  The unfused baseline runs the same variant
  // when it has a logits epilogue; the rows variant has none (it only runs
  // fused), and then the baseline takes the variant ranked first for the
  // unfused path.
  const int cu_count = device_cu_count(256);
  const int path_req = fused ? WTC_PATH_AUTO : WTC_PATH_UNFUSED;
  const VariantDesc requested = var;
  wtc_tiles want{tile_m, tile_n, tile_k, thread_tile_m, thread_tile_n};
  if (!fused && !(var.paths & (1u << WTC_PATH_UNFUSED))) {
    wtc_tiles best{};
    if (wtc_plan_tiles(spec.batch, spec.m, spec.n, spec.k, in_code, out_code, WTC_PATH_UNFUSED,
                       nullptr, cu_count, 1, &best, nullptr, nullptr, nullptr, nullptr) != WTC_OK)
      return session_fail(std::string("launch plan failed: ") + wtc_last_error());
    want = best;
    find_variant(in_code, want.tile_m, want.tile_n, want.tile_k, want.thread_tile_m,
                 want.thread_tile_n, &var);
  }
  int64_t grid = 0, ws = 0;
  int path = 0;
  double est_us = 0;
  if (wtc_plan_tiles(spec.batch, spec.m, spec.n, spec.k, in_code, out_code, path_req, &want,
                     cu_count, 1, nullptr, &path, &grid, &ws, &est_us) != WTC_OK)
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
    std::string symbol_prefix;  // of the mangled name in the code object
    int64_t grid;
    int lds;
    int block = 256;
    std::string kind = "rowwise";  // loop structure in 04c (StageKernel::kind)
  };
  // chain_tile_kernel<in, out, epi, PF = 3, tile rows, ks>
  auto chain_sym = [](int in, int out, int epi, int tm = 128, int lw = 0) {
    return "_ZN3wtc17chain_tile_kernelILi" + std::to_string(in) + "ELi" + std::to_string(out) +
           "ELi" + std::to_string(epi) + "ELi3ELi" + std::to_string(tm) + "ELi" + std::to_string(lw) + "E";
  };
  // chain_wide_kernel<in, out, epi>: the 256x256 tiles
  auto wide_sym = [](int in, int out, int epi) {
    return "_ZN3wtc17chain_wide_kernelILi" + std::to_string(in) + "ELi" + std::to_string(out) +
           "ELi" + std::to_string(epi) + "E";
  };
  const bool wide = var.id == kVarTile256x256;
  // the split / unfused tile kernel of the variant: display name and symbol
  auto tile_kern = [&](int out, const std::string& out_name, int epi, const std::string& epi_name) {
    if (wide) return std::make_pair("chain_wide_kernel<" + kin + "," + out_name + "," + epi_name + ",256x256>",
                                    wide_sym(in_code, out, epi));
    const std::string layout = std::to_string(var.tile_rows) + "x128" + (var.loaders ? ",loaders" : "");
    return std::make_pair("chain_tile_kernel<" + kin + "," + out_name + "," + epi_name + "," + layout + ">",
                          chain_sym(in_code, out, epi, var.tile_rows, var.loaders));
  };
  const std::string out_t = "ILi" + std::to_string(out_code) + "E";
  std::vector<K> ks;
  const int64_t rows = spec.batch * spec.m;
  const int tile_threads = wide ? wide_kernel_threads() : chain_kernel_threads(in_code);
  if (path == WTC_PATH_ROWS) {
    ks.push_back({"chain_rows_kernel<" + kin + "," + kout + ">",
                  "_ZN3wtc17chain_rows_kernelILi" + std::to_string(in_code) + "ELi" +
                      std::to_string(out_code) + "E",
                  grid, 0, rows_kernel_threads(), "rows"});
  } else if (path == WTC_PATH_EXCHANGE) {
    ks.push_back({"chain_tile_kernel<" + kin + "," + kout + ",exchange,128x128" +
                      (var.loaders ? ",loaders" : "") + ">",
                  chain_sym(in_code, out_code, 0, 128, var.loaders), grid,
                  exchange_lds_pad(in_code, out_code, var.loaders), tile_threads, "tile_exchange"});
  } else if (path == WTC_PATH_SPLIT) {
    const auto tk = tile_kern(out_code, kout, 1, "split");
    ks.push_back({tk.first, tk.second, grid, 0, tile_threads, "tile_split"});
    ks.push_back({"rescale_rows_kernel<" + kout + ">", "_ZN3wtc19rescale_rows_kernel" + out_t,
                  (rows * rescale_waves_per_row(rows, cu_count) + 3) / 4, 0, 256, "rescale"});
  } else {
    const auto tk = tile_kern(0, "f32", 2, "logits");
    ks.push_back({tk.first, tk.second, grid, 0, tile_threads, "tile_logits"});
    ks.push_back({"rowmax_kernel", "_ZN3wtc13rowmax_kernel", rows, 0, 256, "row max"});
    ks.push_back({"expsub_kernel", "_ZN3wtc13expsub_kernel", rows, 0, 256, "exp(x - max)"});
    ks.push_back({"rowsum_kernel", "_ZN3wtc13rowsum_kernel", rows, 0, 256, "row sum"});
    ks.push_back({"rowdiv_kernel<" + kout + ">", "_ZN3wtc13rowdiv_kernel" + out_t, rows, 0, 256, "divide"});
  }

  std::ostringstream plan;
  auto tiles_json = [](const wtc_tiles& t) {
    return "{\"tileM\": " + std::to_string(t.tile_m) + ", \"tileN\": " + std::to_string(t.tile_n) +
           ", \"tileK\": " + std::to_string(t.tile_k) + ", \"threadTileM\": " +
           std::to_string(t.thread_tile_m) + ", \"threadTileN\": " + std::to_string(t.thread_tile_n) + "}";
  };
  const wtc_tiles asked{tile_m, tile_n, tile_k, thread_tile_m, thread_tile_n};
  plan << "{\n  \"target\": \"gfx950\",\n  \"variant\": \"" << var.name << "\",\n  \"requested_variant\": \""
       << requested.name << "\",\n  \"path\": \"" << path_name(path) << "\",\n  \"fused\": "
       << (fused ? "true" : "false") << ",\n  \"max_connect_level\": " << max_connect_level
       << ",\n  \"tiles\": " << tiles_json(want) << ",\n  \"requested_tiles\": " << tiles_json(asked)
       << ",\n  \"estimated_us\": " << est_us << ",\n  \"kernels\": [\n";
  for (size_t i = 0; i < ks.size(); ++i)
    plan << "    {\"name\": \"" << ks[i].name << "\", \"grid\": [" << ks[i].grid
         << ", 1, 1], \"block\": [" << ks[i].block << ", 1, 1], \"dynamic_lds_bytes\": " << ks[i].lds
         << "}"
         << (i + 1 < ks.size() ? "," : "") << "\n";
  plan << "  ],\n  \"workspace_bytes\": " << ws << "\n}\n";

  std::ostringstream launch;
  launch << "{\n  \"format\": \"wtc-hip-launch-v1\",\n  \"target\": \"gfx950\",\n  \"library\": \"" << lib
         << "\",\n  \"entry\": \"wtc_matmul_softmax_tiles\",\n  \"variant\": \"" << var.name
         << "\",\n  \"tiles\": " << tiles_json(want) << ",\n  \"problem\": {\"batch\": " << spec.batch
         << ", \"m\": " << spec.m << ", \"n\": " << spec.n << ", \"k\": " << spec.k
         << ", \"batched\": " << (spec.batched ? "true" : "false") << "},\n  \"in_dtype\": \"" << kin
         << "\",\n  \"out_dtype\": \"" << kout << "\",\n  \"chain_acc_dtype\": \"" << elem_mlir_name(spec.acc)
         << "\",\n  \"kernel_acc_dtype\": \"f32\",\n  \"dtype_codes\": {\"in\": " << in_code
         << ", \"out\": " << out_code << "},\n  \"logit_scale\": " << spec.logit_scale
         << ",\n  \"runtime_scales\": " << (spec.runtime_scales ? "true" : "false") << ",\n  \"path\": \""
         << path_name(path) << "\",\n  \"path_code\": " << path << ",\n  \"workspace_bytes\": " << ws
         << ",\n  \"softmax_form\": \"" << (spec.form == SoftmaxForm::Named ? "named" : "decomposed")
         << "\"\n}\n";

  // Artifact report: the counterpart of the reference's post-bufferize
  // report (compiler/runtime/PostbufferizeFixups.cpp:60-82), re-targeted to
  // the gfx950 code object: MFMA instructions instead of nvvm.mma.sync,
  // scratch instructions / spills instead of PTX ld.local / st.local.
  ResourceTable table;
  std::string res_path;
  const bool have_res = load_resources(lib, table, res_path);
  int64_t mfma = 0, scratch_ops = 0, scratch_bytes = 0, vspill = 0, sspill = 0, dma = 0, tr = 0;
  int missing = 0;
  std::ostringstream per_kernel;
  std::vector<StageKernel> stage_ks;
  for (const K& k : ks) {
    const auto* row = have_res ? find_kernel(table, k.symbol_prefix) : nullptr;
    if (!row) ++missing;
    stage_ks.push_back({k.name, k.kind, k.grid, k.block, cell(row, "lds_bytes") + k.lds});
    mfma += cell(row, "mfma");
    scratch_ops += cell(row, "scratch_ops");
    scratch_bytes += cell(row, "scratch_bytes");
    vspill += cell(row, "vgpr_spill_count");
    sspill += cell(row, "sgpr_spill_count");
    dma += cell(row, "lds_dma_loads");
    tr += cell(row, "ds_read_tr");
    per_kernel << "kernel " << k.name << " grid=" << k.grid << " block=" << k.block;
    if (row)
      per_kernel << " vgpr=" << cell(row, "vgpr_count") << " agpr=" << cell(row, "agpr_count")
                 << " sgpr=" << cell(row, "sgpr_count") << " lds_static=" << cell(row, "lds_bytes")
                 << " lds_dynamic=" << k.lds << " mfma=" << cell(row, "mfma")
                 << " scratch_bytes=" << cell(row, "scratch_bytes");
    else
      per_kernel << " (no resource record)";
    per_kernel << "\n";
  }
  const std::string canonical = emit_canonical_mlir(spec);
  std::ostringstream report;
  report << "chain_matmul_count=" << (canonical.find("linalg.") != std::string::npos ? 1 : 0) << "\n";
  report << "launch_kernel_count=" << ks.size() << "\n";
  report << "mfma_instruction_count=" << mfma << "\n";
  report << "lds_dma_load_count=" << dma << "\n";
  report << "lds_transpose_read_count=" << tr << "\n";
  report << "scratch_instruction_count=" << scratch_ops << "\n";
  report << "scratch_bytes=" << scratch_bytes << "\n";
  report << "vgpr_spill_count=" << vspill << "\n";
  report << "sgpr_spill_count=" << sspill << "\n";
  report << "kernels_without_resource_record=" << missing << "\n";
  report << "resources=" << (have_res ? res_path : "missing") << "\n";
  report << "chain: batch=" << spec.batch << " m=" << spec.m << " n=" << spec.n << " k=" << spec.k
         << " in=" << kin << " out=" << kout << " path=" << path_name(path) << "\n";
  report << per_kernel.str();

  // The stage files under the reference's names (its callers check that they
  // exist and are not empty, count operations in them, and its regression
  // script looks for "workgroup(" in 04 and "gpu.launch_func" in 05): the
  // canonical chain (03), each kernel's launch with its LDS as the workgroup
  // attribution (04), the kernels' loop structure (04c), and the runnable
  // module: one gpu.launch_func per kernel of the gfx950 code object, with
  // the entry point and its arguments as attributes (05).
  const std::string a_t = memref_of(spec, spec.m, spec.k, spec.in);
  const std::string b_t = memref_of(spec, spec.k, spec.n, spec.in);
  const std::string o_t = memref_of(spec, spec.m, spec.n, spec.out);
  const std::string w_t = "memref<" + std::to_string(ws) + "xi8>";
  const std::string sig = "(%a: " + a_t + ", %b: " + b_t + ", %out: " + o_t + ", %ws: " + w_t + ")";
  auto sym_of = [](std::string kname) {
    for (char& c : kname)
      if (!std::isalnum(static_cast<unsigned char>(c))) c = '_';
    return kname;
  };
  std::ostringstream wg;
  wg << "// Launches of the fused Matmul -> row-Softmax chain on gfx950, " << path_name(path)
     << " path: one launch region per HIP kernel\n// with its grid, block and LDS (static + dynamic "
        "bytes, the workgroup attribution).  The bodies are the\n// kernels of the code object "
        "05.out.gfx950.hsaco (library "
     << lib << "), variant " << var.name << ".\n"
     << "module attributes {gpu.container_module, wtc.target = \"gfx950\", wtc.path = \""
     << path_name(path) << "\", wtc.compute_units = " << cu_count << " : i32} {\n"
     << "  func.func @chain" << sig << " {\n    %c1 = arith.constant 1 : index\n";
  for (size_t i = 0; i < ks.size(); ++i) {
    wg << "    %g" << i << " = arith.constant " << ks[i].grid << " : index\n"
       << "    %t" << i << " = arith.constant " << ks[i].block << " : index\n"
       << "    gpu.launch blocks(%bx" << i << ", %by" << i << ", %bz" << i << ") in (%gx" << i << " = %g" << i
       << ", %gy" << i << " = %c1, %gz" << i << " = %c1) threads(%tx" << i << ", %ty" << i << ", %tz" << i
       << ") in (%sx" << i << " = %t" << i << ", %sy" << i << " = %c1, %sz" << i
       << " = %c1) workgroup(%lds" << i << " : memref<" << stage_ks[i].lds << "xi8, 3>) {\n"
       << "      // body: " << ks[i].name << "\n      gpu.terminator\n    }\n";
  }
  wg << "    return\n  }\n}\n";
  std::ostringstream run;
  run << "// Runnable artefact of the chain for gfx950 (no NVVM is involved): the kernels of\n"
      << "// the HIP code object 05.out.gfx950.hsaco, launched by wtc_matmul_softmax_tiles with\n"
      << "// the arguments in the module attributes.  Per-kernel resources are in kernel_report.txt.\n"
      << "module attributes {gpu.container_module, wtc.target = \"gfx950\", wtc.code_object = "
         "\"05.out.gfx950.hsaco\", "
      << "wtc.library = \"" << lib << "\", wtc.entry = \"wtc_matmul_softmax_tiles\", wtc.variant = \""
      << var.name << "\", wtc.tiles = [" << want.tile_m << ", " << want.tile_n << ", " << want.tile_k
      << ", " << want.thread_tile_m << ", " << want.thread_tile_n << "], wtc.path = \""
      << path_name(path) << "\", wtc.path_code = " << path << " : i32, wtc.in_dtype = " << in_code
      << " : i32, wtc.out_dtype = " << out_code << " : i32, wtc.batch = " << spec.batch
      << " : i64, wtc.m = " << spec.m << " : i64, wtc.n = " << spec.n << " : i64, wtc.k = " << spec.k
      << " : i64, wtc.workspace_bytes = " << ws << " : i64, wtc.mfma_instructions = " << mfma
      << " : i64, wtc.scratch_bytes = " << scratch_bytes << " : i64} {\n"
      << "  gpu.module @wtc_kernels [#rocdl.target<chip = \"gfx950\">] {\n  }\n"
      << "  func.func @chain" << sig << " {\n    %c1 = arith.constant 1 : index\n";
  for (size_t i = 0; i < ks.size(); ++i) {
    run << "    %g" << i << " = arith.constant " << ks[i].grid << " : index\n"
        << "    %t" << i << " = arith.constant " << ks[i].block << " : index\n"
        << "    %l" << i << " = arith.constant " << ks[i].lds << " : i32\n"
        << "    gpu.launch_func @wtc_kernels::@" << sym_of(ks[i].name) << " blocks in (%g" << i
        << ", %c1, %c1) threads in (%t" << i << ", %c1, %c1) dynamic_shared_memory_size %l" << i
        << " args(%a : " << a_t << ", %b : " << b_t << ", %out : " << o_t << ", %ws : " << w_t
        << ")\n";
  }
  run << "    return\n  }\n}\n";
  const std::string loops = emit_loop_structure(spec, var, in_code, path_name(path), stage_ks);
  if (!write_file((od / "03.after_postbufferize.mlir").string(), canonical) ||
      !write_file((od / "04.after_workgroup_launch.mlir").string(), wg.str()) ||
      !write_file((od / "04c.after_linalg_to_loops.mlir").string(), loops) ||
      !write_file((od / "05.out.nvvm.runnable.mlir").string(), run.str()) ||
      !write_file((od / "03.chain.canonical.mlir").string(), canonical) ||
      !write_file((od / "04.kernel.plan.json").string(), plan.str()) ||
      !write_file((od / "05.out.hip.launch.json").string(), launch.str()) ||
      !write_file((od / "kernel_report.txt").string(), report.str()))
    return session_fail(std::string("failed to write artefacts into ") + out_dir);
  // The device code objects holding the path's kernels, when the build left
  // them next to the library.
  const std::filesystem::path libdir = std::filesystem::path(lib).parent_path();
  std::vector<std::pair<std::string, std::string>> cos = {
      {"fused_matmul_softmax.gfx950.co", "05.out.gfx950.hsaco"}};
  if (path == WTC_PATH_UNFUSED) cos.push_back({"unfused_chain.gfx950.co", "05.out.rows.gfx950.hsaco"});
  for (const auto& c : cos) {
    if (!std::filesystem::exists(libdir / c.first)) continue;
    std::filesystem::copy_file(libdir / c.first, od / c.second,
                               std::filesystem::copy_options::overwrite_existing, ec);
    if (ec) return session_fail("failed to copy the code object into " + std::string(out_dir));
  }
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
