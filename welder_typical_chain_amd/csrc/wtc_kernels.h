// wtc_kernels.h -- kernel parameter block and symbol table shared by the
// HIP kernels (fused_matmul_softmax.hip, unfused_chain.hip) and the host
// launcher (launch.hip).  Internal to the library; the public C-ABI is
// include/wtc/wtc_hip.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wtc {

enum : int { kEpiExchange = 0, kEpiSplit = 1, kEpiLogits = 2 };

// 32-bit words of workspace per row block for the exchange: the arrival
// counter at word kSyncCnt and the generation word at kSyncGen, each in a
// 128-byte line of its own.
constexpr int kSyncWords = 64;
constexpr int kSyncCnt = 0;
constexpr int kSyncGen = 32;

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
  float2* partial;  // [batch*nRB*128][nT] per-tile row (max, sumexp), log2 domain
  uint32_t* sync;   // [batch*nRB][kSyncWords] row-block counter and generation
  uint32_t* err;    // [0] bit 0: a row-block wait timed out; [1] longest wait
                    // (100 MHz ticks); [2] number of timed-out waits
  uint64_t spin_ticks;  // row-block wait limit, 100 MHz ticks
};

// tile_rows: 128, or 256 for the split path with 16-bit or fp8 inputs (else NULL).
const void* chain_kernel_symbol(int in_dt, int out_dt, int epi, int tile_rows = 128);
const void* rescale_kernel_symbol(int out_dt);
// Waves that share one row in rescale_rows_kernel (its grid is rows * wpr / 4).
int rescale_waves_per_row(int64_t rows_total, int cu_count);
const void* zero_kernel_symbol();
int chain_kernel_lds_bytes(int in_dt, int out_dt);
// Tile height (128 or 256) the split path uses for this problem on a device
// with cu_count compute units.
int split_tile_rows(int in_dt, int64_t batch, int64_t m, int64_t n, int cu_count);
int chain_kernel_threads(int in_dt);  // workgroup size of chain_tile_kernel

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
