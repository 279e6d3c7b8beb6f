// wtc_kernels.h -- kernel parameter block and symbol table shared by the
// HIP kernels (fused_matmul_softmax.hip, wide_tile.hip, unfused_chain.hip) and the host
// launcher (launch.hip).  Internal to the library; the public C-ABI is
// include/wtc/wtc_hip.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wtc {

enum : int { kEpiExchange = 0, kEpiSplit = 1, kEpiLogits = 2 };

// The exchange path keeps one generation word per tile slot (slot = row
// block * column tiles + column tile) and 128 tagged 64-bit entries per slot;
// a launch uses at most this many slots.
constexpr int kMaxExchangeTiles = 1024;

struct ChainParams {
  const uint8_t* a;
  const uint8_t* b;
  uint8_t* out;
  int64_t M, N, K;                       // per batch
  int64_t a_bstride, b_bstride, o_bstride;  // bytes between batches
  int64_t lda_bytes, ldb_bytes, ldo_bytes;  // row pitches in bytes
  float c2;         // scale * log2(e): softmax runs as exp2(c2*x - max)
  float lin_scale;  // scale for kEpiLogits
  int nRB;          // row blocks (of 128 rows) per batch
  int nT;           // column tiles (of 128 columns) per row block
  float2* partial;  // split path: [batch][nRB * tile rows][nT] per-tile row (max, sumexp), log2
  uint64_t* ent;    // exchange path: [slot][128] tagged per-row log-sum-exp entries
  uint32_t* gen;    // exchange path: [kMaxExchangeTiles] slot generation words
  uint32_t* err;    // [0] bit 0: an exchange wait timed out; [1] longest wait
                    // (100 MHz ticks); [2] number of timed-out waits
  uint32_t* mailbox;    // host-visible word set on a timed-out wait (may be NULL)
  uint64_t spin_ticks;  // exchange wait limit, 100 MHz ticks
};

// tile_rows: 128, or 256 (split epilogue, and f32 logits, with 16-bit or fp8
// inputs); loaders: 1 for the 128-row layout with 4 MFMA and 4 loader waves
// (exchange and split epilogues, and f32 logits, with 16-bit or fp8 inputs).
// NULL for a combination not built.
const void* chain_kernel_symbol(int in_dt, int out_dt, int epi, int tile_rows = 128, int loaders = 0);
const void* rescale_kernel_symbol(int out_dt);
// Waves that share one row in rescale_rows_kernel (its grid is rows * wpr / 4).
int rescale_waves_per_row(int64_t rows_total, int cu_count);
const void* zero_kernel_symbol();
// Static LDS of the exchange-epilogue kernel of this wave layout.
int chain_kernel_lds_bytes(int in_dt, int out_dt, int loaders = 0);
int chain_kernel_threads(int in_dt);  // workgroup size of chain_tile_kernel (every layout)

// 256x256 tiles (wide_tile.hip): split epilogue (any output type) or f32
// logits, 16-bit or fp8 inputs; NULL otherwise.  Same arguments as
// chain_tile_kernel; the split path's statistics are [rows][nT] with nT the
// 256-column tiles.
const void* wide_kernel_symbol(int in_dt, int out_dt, int epi);
int wide_kernel_threads();

// One workgroup per 128-row block, two passes over N (K <= rows_kernel_max_k()).
const void* rows_kernel_symbol(int in_dt, int out_dt);
int rows_kernel_threads();
int rows_kernel_max_k();

// Unfused five-kernel baseline (matmul, row max, exp, row sum, divide).
const void* rowmax_kernel_symbol();
const void* expsub_kernel_symbol();
const void* rowsum_kernel_symbol();
const void* rowdiv_kernel_symbol(int out_dt);

}  // namespace wtc
