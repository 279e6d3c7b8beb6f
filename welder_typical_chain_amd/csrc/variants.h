// variants.h -- the kernel variants of the gfx950 library (the tile space
// behind the solver) and the cost model that ranks them for a problem.
//
// Host-only, plain C++: linked into the launcher (AUTO selection), the solver
// C-ABI (candidates.tsv / best.json) and the compile C-ABI (plan of a given
// best.json), so that all three rank with the same numbers.
//
// In the reference the tile space is whatever tile sizes the code generator
// accepts, enumerated and scored by an analytic traffic model
// (backend/welder/compiler/solver/WelderSolverSolveEntrypoints.h:157-265).
// Here the kernels are hand-written, so the space is the set of instantiated
// kernel variants, and the score is a latency estimate calibrated on MI355X
// (welder_typical_chain_amd/calibrate.py measures it).
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace wtc {

enum VariantId : int {
  kVarTile128 = 0,        // 128x128 tile; 16-bit/fp8: 8 waves of 64x32, f32: 4 waves of 64x64
  kVarTile128Loaders = 1,  // 128x128 tile, 4 MFMA waves of 64x64 + 4 loader waves (16-bit/fp8)
  kVarTile256 = 2,        // 256x128 tile, 8 waves of 64x64 (16-bit/fp8)
  kVarRows = 3,           // one 128-row block over all of n, two passes (16-bit, k <= 128)
  kVarTile256x256 = 4,    // 256x256 tile, 4 waves of 128x128, 64-byte k-slabs (16-bit/fp8)
  kNumVariants = 5,
};

// One variant in the reference's tile vocabulary (best.json): tile_k counts
// elements of the input type in one pipeline stage of K, the thread tile is
// the accumulator footprint of one lane (rows x columns).
struct VariantDesc {
  int id;
  const char* name;
  int64_t tile_m, tile_n, tile_k, thread_tile_m, thread_tile_n;
  int tile_rows;   // rows of one workgroup's tile (its columns: tile_n)
  int loaders;     // 1: the 128-row layout whose loads are issued by loader waves
  unsigned paths;  // bit (1 << WTC_PATH_x) for each path the variant runs
};

// The variants implemented for an input type (WTC_DTYPE_*), in id order
// (a static table: empty for an unknown type).
const std::vector<VariantDesc>& variants_for(int in_dt);
// The variant with exactly these five tile parameters, if any.
bool find_variant(int in_dt, int64_t tile_m, int64_t tile_n, int64_t tile_k, int64_t thread_tile_m,
                  int64_t thread_tile_n, VariantDesc* out);
bool variant_by_id(int in_dt, int id, VariantDesc* out);

// Limits of the kernels behind the paths (the launcher checks that its
// kernels agree).
constexpr int64_t kExchangeMaxTiles = 1024;   // slot generation words of a workspace
constexpr int64_t kExchangeMaxColTiles = 64;  // one lane per column tile of a row block
constexpr int64_t kSplitMaxColTiles = 512;    // row statistics the rescale kernel merges
constexpr int64_t kRowsMaxK = 128;            // the rows kernel keeps all of K in one stage

// Problem geometry the model and the launcher share.
struct Problem {
  int64_t batch, m, n, k;
  int in_dt, out_dt;
  int cu_count;   // compute units of the device
  int xch_per_cu; // exchange-kernel workgroups one CU holds (1 with its LDS pad)
};

// Whether a (variant, path) pair can run a problem, and why not (empty when
// it can; builds the message, so only for error reports).
bool feasible(const VariantDesc& v, int path, const Problem& p);
std::string infeasible_reason(const VariantDesc& v, int path, const Problem& p);

// Estimated microseconds per back-to-back call of `path` on variant `v`.
double estimate_us(const VariantDesc& v, int path, const Problem& p);

struct Choice {
  VariantDesc v;
  int path;
  double est_us;
};
// Every feasible (variant, path) pair, fastest first.  `path` = WTC_PATH_AUTO
// ranks the fused paths (exchange, split, rows); another path ranks only that
// one; `variant` >= 0 keeps only that variant.
std::vector<Choice> rank_choices(const Problem& p, int path, int variant = -1);
// The first of rank_choices without building the list; false when nothing
// is feasible.
bool best_choice(const Problem& p, int path, int variant, Choice* out);

// Grid of the path's first kernel.
int64_t variant_grid(const VariantDesc& v, int path, const Problem& p);

}  // namespace wtc
