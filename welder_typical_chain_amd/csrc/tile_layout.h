// tile_layout.h -- index maps of the fused Matmul->row-Softmax kernels for
// gfx950.  Everything here is plain integer arithmetic usable on host and
// device, so the CPU test (tests/layout_check.cpp) can replay one workgroup's
// data movement and check it against a plain matmul.
//
// Vocabulary.
//   chunk   16 contiguous bytes along K (8 f16/bf16, 16 fp8, 4 f32).  One
//           chunk is what a lane hands one MFMA-operand register quad.
//   k-tile  128 bytes of K (8 chunks) staged per pipeline step.
//   tile    BM x BN block of the output owned by one workgroup.
//   row block  BM rows of one batch: the tiles that share a softmax row.
//
// LDS layout of one pipeline stage (both operands k-contiguous so every
// MFMA operand fetch is a single ds_read_b128):
//   A: [BM rows][8 chunks], chunk c of row m stored at slot c ^ ((m>>1)&7).
//      16 lanes reading 16 consecutive rows at one chunk hit 16 distinct
//      4-bank groups; the 16 lanes of a store (2 rows x 8 chunks) do too.
//   B: [8 chunks][BN cols], column n of chunk row kc stored at
//      n ^ ((n>>4)&3).  The B tile arrives N-contiguous from HBM and is
//      transposed in registers before this store (B is [K,N] row-major).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define WTC_HD __host__ __device__ inline
#else
#define WTC_HD inline
#endif

namespace wtc {

enum : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_FP8 = 3 };

WTC_HD constexpr int dtype_bytes(int dt) {
  return dt == DT_F32 ? 4 : (dt == DT_FP8 ? 1 : 2);
}

constexpr int kChunkBytes = 16;
constexpr int kKTileBytes = 128;
constexpr int kChunksPerKTile = kKTileBytes / kChunkBytes; // 8

// ---- A operand (row-major [M,K]) ----------------------------------------
// Byte offset of (row m, chunk c) inside the A stage buffer.
WTC_HD constexpr int a_lds_offset(int m, int c) {
  return m * kKTileBytes + ((c ^ ((m >> 1) & 7)) * kChunkBytes);
}
// Every thread fetches part of both operands (straight-line code, so the
// compiler can count outstanding loads exactly).  A: thread t, pass j (0..3)
// fetches chunk t%8 of row t/8 + 32j with one 128-bit load; the 8 lanes of a
// row cover its 128 contiguous bytes.
WTC_HD constexpr int a_load_row(int t, int j) { return (t >> 3) + 32 * j; }
WTC_HD constexpr int a_load_chunk(int t) { return t & 7; }

// ---- B operand (row-major [K,N]) ----------------------------------------
// Column n of chunk row kc is stored at slot n ^ ((n>>4)&7): 16 consecutive
// columns (a fragment read) and the 16 columns 4g+c, g = 0..15 (one store
// instruction of 16 loader lanes) both land in 16 distinct slots mod 16.
WTC_HD constexpr int b_swz(int n) { return n ^ ((n >> 4) & 7); }
// Byte offset of (chunk row kc, column n) inside the B stage buffer of width BN.
WTC_HD constexpr int b_lds_offset(int kc, int n, int BN) {
  return (kc * BN + b_swz(n)) * kChunkBytes;
}
// B: thread t owns columns 4*(t%32)+0..3 of the k-rows of chunk row
// kc = t/32: an (elements-per-chunk) x 4 block that it transposes into 4
// chunks, one per column.  32 lanes cover 128 contiguous columns.
WTC_HD constexpr int b_load_colgroup(int t) { return t & 31; }
WTC_HD constexpr int b_load_chunkrow(int t) { return t >> 5; }

// ---- MFMA fragments (32x32xK, wave64) -------------------------------------
// Lane l supplies row/col (l % 32) and chunk (2*s + l/32) of k-substep s.
WTC_HD constexpr int frag_row(int lane) { return lane & 31; }
WTC_HD constexpr int frag_chunk(int lane, int s) { return 2 * s + (lane >> 5); }
// 32x32 accumulator: register v of lane l holds D[i][j] with
// j = l % 32 and i = 8*(v/4) + 4*(l/32) + v%4.
WTC_HD constexpr int acc_i(int lane, int v) {
  return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}
WTC_HD constexpr int acc_j(int lane) { return lane & 31; }

// ---- register transpose of B (N-contiguous rows -> K-contiguous chunks) ---
// 16-bit elements: `lo`/`hi` hold columns (2*(c/2), 2*(c/2)+1) of k-rows 2w
// and 2w+1; returns word w of the chunk of column c (two consecutive k).
WTC_HD constexpr uint32_t transpose16_word(uint32_t lo, uint32_t hi, int c) {
  return (c & 1) ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
}
// 8-bit elements: r0..r3 hold columns 0..3 of k-rows 4w..4w+3; returns word w
// of the chunk of column c (four consecutive k).
WTC_HD constexpr uint32_t transpose8_word(uint32_t r0, uint32_t r1, uint32_t r2,
                                          uint32_t r3, int c) {
  return ((r0 >> (8 * c)) & 0xFFu) | (((r1 >> (8 * c)) & 0xFFu) << 8) |
         (((r2 >> (8 * c)) & 0xFFu) << 16) | (((r3 >> (8 * c)) & 0xFFu) << 24);
}

// A B loader holds its k-rows as 16 row-major 32-bit words (4 columns per
// row: 2 words of f16/bf16, 1 of fp8, 4 of f32).  Index of the word holding
// column c of k-row r:
WTC_HD constexpr int b_src_word(int sz, int r, int c) {
  return sz == 2 ? r * 2 + (c >> 1) : (sz == 1 ? r : r * 4 + c);
}
// Word w of the K-contiguous chunk of column c, from the loader's words.
template <typename Words>
WTC_HD uint32_t b_unit_word(const Words& rw, int sz, int c, int w) {
  if (sz == 2) return transpose16_word(rw(b_src_word(2, 2 * w, c)), rw(b_src_word(2, 2 * w + 1, c)), c);
  if (sz == 1)
    return transpose8_word(rw(b_src_word(1, 4 * w, c)), rw(b_src_word(1, 4 * w + 1, c)),
                           rw(b_src_word(1, 4 * w + 2, c)), rw(b_src_word(1, 4 * w + 3, c)), c);
  return rw(b_src_word(4, w, c));
}

// ---- direct-to-LDS (DMA) staging of 16-bit k-tiles --------------------------
// A buffer_load ... lds instruction writes lane i's 16 bytes at
// LDS base + 16*i: each wave instruction fills one contiguous 1 KiB block, so
// the swizzles are realised by choosing which global chunk each lane fetches.
// With nb blocks per wave (16 / waves), wave w issues instructions
// j = 0..nb-1 for A and for B: block b = nb*w + j.
WTC_HD constexpr int dma_block(int wave, int j, int nb) { return nb * wave + j; }
// A block b = rows 8b..8b+7 of the A stage; lane i lands in row 8b + i/8,
// slot i%8, which a_lds_offset assigns to chunk slot ^ ((row>>1)&7).
WTC_HD constexpr int dma_a_row(int b, int lane) { return 8 * b + (lane >> 3); }
WTC_HD constexpr int dma_a_chunk(int b, int lane) {
  return (lane & 7) ^ ((dma_a_row(b, lane) >> 1) & 7);
}
// B stays K-major ([k][n], 256 bytes per k-row for BN = 128 16-bit columns)
// with 16-byte chunks XOR-swizzled by k%4: element (k, n) lives at
// btr_offset(k, n).  B block b = k-rows 4b..4b+3; lane i lands in row
// 4b + i/16, slot i%16, which holds chunk slot ^ 4*(row%4).
WTC_HD constexpr int btr_offset(int k, int n) {
  return k * 256 + ((((n >> 3) ^ ((k & 3) << 2)) & 15) << 4) + (n & 7) * 2;
}
WTC_HD constexpr int dma_b_row(int b, int lane) { return 4 * b + (lane >> 4); }
WTC_HD constexpr int dma_b_chunk(int b, int lane) {
  return (lane & 15) ^ ((dma_b_row(b, lane) & 3) << 2);
}
// The B operand is read with ds_read_b64_tr_b16: within each group of 16
// lanes the 4 x 16 matrix formed by lanes 4r..4r+3 (row r, 4 elements each)
// is transposed, so lane i receives column i: element r of its result is
// element i%4 of lane 4r + i/4.  For MFMA k-step s, n-subtile base nb and
// half h (k-quad), lane l supplies the address of (btr_k, btr_n) and gets
// B[16s + 8(l/32) + 4h + r][nb + l%32] for r = 0..3: with h = 0, 1 that is
// the same 8 consecutive k the A fragment of lane l holds (frag_chunk).
WTC_HD constexpr int btr_k(int s, int h, int lane) {
  return 16 * s + 8 * (lane >> 5) + 4 * h + ((lane & 15) >> 2);
}
WTC_HD constexpr int btr_n(int nb, int lane) { return nb + 16 * ((lane >> 4) & 1) + 4 * (lane & 3); }

// ---- direct-to-LDS staging of 8-bit (fp8) k-tiles ---------------------------
// A uses the 16-bit layout above unchanged (a chunk is 16 fp8 instead of 8
// f16).  B stays K-major ([k][n], 128 bytes per k-row for BN = 128 columns,
// 128 k-rows per k-tile) with 16-byte chunks XOR-swizzled by 2*((k/2)%4):
// element (k, n) lives at btr8_offset(k, n).  B block b = k-rows 8b..8b+7;
// lane i lands in row 8b + i/8, slot i%8, which holds chunk slot ^ 2*((row/2)%4).
WTC_HD constexpr int btr8_offset(int k, int n) {
  return k * 128 + ((((n >> 4) ^ (((k >> 1) & 3) << 1)) & 7) << 4) + (n & 15);
}
WTC_HD constexpr int dma8_b_row(int b, int lane) { return 8 * b + (lane >> 3); }
WTC_HD constexpr int dma8_b_chunk(int b, int lane) {
  return (lane & 7) ^ (((dma8_b_row(b, lane) >> 1) & 3) << 1);
}
// The fp8 MFMA (32x32x64) takes 32 bytes per lane: lane l supplies row /
// column l%32 and, for k-step s, k = 64s + 32(l/32) + 0..31.  A arrives as
// two ds_read_b128 of chunks 4s + 2(l/32) and 4s + 2(l/32) + 1.  B arrives
// as four ds_read_b64_tr_b8 (q = 0..3); within each group of 16 lanes that
// read returns to lane i, byte r, byte i%8 of the 8 bytes read by lane
// 2r + i/8.  So source lane j of a group reads k-row 64s + 32h + 8q + j/2,
// columns nb + 16*(group%2) + 8*(j%2) .. +7, and lane i of the group then
// holds column nb + 16*(group%2) + i, k = 64s + 32h + 8q + r.
WTC_HD constexpr int btr8_k(int s, int q, int lane) {
  return 64 * s + 32 * (lane >> 5) + 8 * q + ((lane & 15) >> 1);
}
WTC_HD constexpr int btr8_n(int nb, int lane) { return nb + 16 * ((lane >> 4) & 1) + 8 * (lane & 1); }

// ---- 64-byte k-slabs of the 256x256 tiles -----------------------------------
// A 256x256 tile stages 64 bytes of K per ring stage (a k-slab: 32 f16/bf16
// or 64 fp8 values): A [256 rows][4 chunks], chunk c of row m at slot
// c ^ ((m >> 2) & 3).  The 16 lanes of a fragment read (16 consecutive rows,
// one chunk) then hit 16 distinct 16-byte bank groups: row m sits at group
// 4 * (m % 4) of its 256-byte line plus the slot, and the slot differs for
// m, m + 4, m + 8, m + 12.  B keeps the K-major layouts above (btr_offset,
// btr8_offset): each 128-column half of the tile is one such B buffer of
// 32 (16-bit) or 64 (fp8) k-rows.
WTC_HD constexpr int a64_lds_offset(int m, int c) { return m * 64 + ((c ^ ((m >> 2) & 3)) << 4); }
// Direct-to-LDS block b of A (1 KiB) = rows 16b .. 16b+15; lane i lands in
// row 16b + i/4, slot i%4, so it fetches chunk slot ^ ((row >> 2) & 3), which
// does not depend on b.
WTC_HD constexpr int dma64_a_row(int b, int lane) { return 16 * b + (lane >> 2); }
WTC_HD constexpr int dma64_a_chunk(int b, int lane) {
  return (lane & 3) ^ ((dma64_a_row(b, lane) >> 2) & 3);
}
// MFMA A fragments from a k-slab: 16-bit k-step s (0, 1) takes chunk
// 2s + lane/32 of row lane%32; fp8 (one k-step of 64) takes chunks
// 2*(lane/32) + hh, hh = 0, 1.
WTC_HD constexpr int frag64_chunk16(int lane, int s) { return 2 * s + (lane >> 5); }
WTC_HD constexpr int frag64_chunk8(int lane, int hh) { return 2 * (lane >> 5) + hh; }

// ---- workgroup -> tile ------------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8).
// tile_of_block() first gives XCD x the contiguous range of logical ids
// [x*G/8, (x+1)*G/8), then maps logical ids to (row block, column tile) in
// groups of kGroupRows row blocks walked column-major, so the tiles one XCD
// holds at a time form a compact 2-D block: with 16x16 tiles and 32 per XCD,
// 4 row blocks x 8 column tiles (3 MiB of operands for a K=1024 f16 chain
// instead of 4.5 MiB for 2 full row blocks), which is what its L2 has to
// fetch over the fabric.
constexpr int kGroupRows = 4;

WTC_HD constexpr uint32_t xcd_remap(uint32_t b, uint32_t G) {
  return (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
}

// rows = row blocks (over all batches), cols = column tiles per row block.
// 32-bit arithmetic: the launcher keeps grids below 2^31 workgroups.
WTC_HD void tile_of_block(uint32_t b, uint32_t G, uint32_t rows, uint32_t cols, uint32_t* row,
                          uint32_t* col) {
  const uint32_t t = xcd_remap(b, G);
  const uint32_t per_group = (uint32_t)kGroupRows * cols;
  const uint32_t group = t / per_group;
  const uint32_t first = group * kGroupRows;
  const uint32_t in_group = (rows - first) < (uint32_t)kGroupRows ? (rows - first) : kGroupRows;
  const uint32_t r = t - group * per_group;
  *row = first + r % in_group;
  *col = r / in_group;
}

// ---- the row-block kernel's output stage (16-bit outputs) ----------------
// Byte offset of 16-byte chunk c (columns 8c .. 8c+7) of row r in an out
// stage of 128-column tiles: 256 bytes per row, chunks XOR-swizzled by
// r % 16, so that the 16 rows of a compute wave's 16-byte write and the 16
// chunks of an I/O wave's row read both fall in 16 distinct bank groups.
WTC_HD constexpr int rows_out_offset(int r, int c) { return r * 256 + ((c ^ (r & 15)) << 4); }

} // namespace wtc
