// chain_spec.h -- the recognised Matmul -> row-Softmax chain and the host
// helpers shared by the reference-compatible C entry points
// (welder_compile_typical_chain_to_nvvm, welder_solver_solve_typical_chain)
// and the wtc-compiler CLI.  Host-only C++17, no HIP.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace wtc {

// Element types as spelled in MLIR.
enum class Elem { F32, F16, BF16, F8E4M3FN, Unknown };

const char* elem_mlir_name(Elem e);
int elem_bytes(Elem e);
int elem_to_dtype_code(Elem e);  // WTC_DTYPE_* of include/wtc/wtc_hip.h, -1 if none

enum class SoftmaxForm { Decomposed, Named };

struct ChainSpec {
  int64_t batch = 1;  // 1 and !batched for linalg.matmul
  bool batched = false;
  int64_t m = 0, n = 0, k = 0;
  Elem in = Elem::Unknown;   // A and B
  Elem acc = Elem::Unknown;  // matmul result element type (the outs tensor)
  Elem out = Elem::Unknown;  // softmax output element type
  SoftmaxForm form = SoftmaxForm::Decomposed;
  double logit_scale = 1.0;      // constant multiplier of the logits, if any
  bool runtime_scales = false;   // f32 scalar arguments multiply the logits (fp8 dequant)
  int matmul_ops = 0, generic_ops = 0, reduction_hints = 0, exp_ops = 0, div_ops = 0;
};

// Parses the chain out of MLIR text.  Accepts the reference's chain files
// (mlir/matmul_softmax_chain*.mlir: matmul from a zero fill, decomposed
// max/exp/sum/div generics or a named linalg.softmax) and their batched /
// scaled / fp8 variants (linalg.batch_matmul, a mulf generic by a constant
// or by f32 scalar arguments).  Returns false with a diagnostic otherwise.
bool recognize_chain(const std::string& text, ChainSpec& spec, std::string& diag);

// The chain in canonical decomposed form (the shape the reference's
// canonicalize stage produces with linalg.softmax decomposed).
std::string emit_canonical_mlir(const ChainSpec& spec);

// Stage-2 artefacts: the input with wtc.tag comments and the tags JSON,
// in the reference's format (compiler/ir/Tagging.cpp:94-150).
void tag_chain(const std::string& text, const ChainSpec& spec, const std::string& source,
               std::string& tagged_mlir, std::string& tags_json);

// ---- tile parameters (best.json) ------------------------------------------
struct TileParams {
  int64_t tile_m = 0, tile_n = 0, tile_k = 0, thread_tile_m = 0, thread_tile_n = 0;
};

// best.json read/write with the reference's keys and regex reader
// (compiler/scheduler/Search.cpp:12-20,35-86).
bool load_best_json(const std::string& path, TileParams& t, std::string& diag);
bool write_best_json(const TileParams& t, const std::string& path, std::string& diag);

// ---- solver ---------------------------------------------------------------
// One kernel variant (variants.h) with the fused path the cost model ranks
// first for it on this problem.
struct Candidate {
  TileParams tiles;
  std::string variant;           // variant name
  double score = 0;              // higher is better: estimated TFLOP/s
  double estimated_latency = 0;  // microseconds per call
  double profiled_ms = -1;
  int64_t bytes_a = 0, bytes_b = 0, bytes_c = 0, bytes_cut = 0;
  std::string path;              // exchange | split | rows
};
struct ArchInfo {
  int64_t lds_bytes = 160 * 1024;
  int64_t num_cu = 256;
  int64_t wave_size = 64;
  double clock_ghz = 2.4;  // peak engine clock (the cost model uses the clock under load)
  double hbm_gbs = 8000.0;
};
std::vector<Candidate> solve(const ChainSpec& spec, int64_t max_connect_level,
                             const ArchInfo& arch);
// best_summary.json and candidates.tsv in the reference's formats
// (backend/welder/compiler/solver/WelderSolverCAPI.cpp:40-97).
bool write_best_summary(const ChainSpec& s, const ArchInfo& arch, const Candidate& best,
                        const std::string& path, std::string& err);
bool write_candidates(const std::vector<Candidate>& cs, const std::string& path, std::string& err);

// ---- misc ---------------------------------------------------------------------
bool read_file(const std::string& path, std::string& out);
bool write_file(const std::string& path, const std::string& text);
void set_error(char* buf, size_t size, const std::string& msg);

}  // namespace wtc
