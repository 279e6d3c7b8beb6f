// fused_matmul_softmax.hip -- the Welder typical chain's hot path on gfx950:
//   out[b, M, N] = softmax_row(scale * (A[b, M, K] . B[b, K, N]))
// hand-written for CDNA4 (wave64, 32x32 MFMA, 160 KB LDS, 8 XCDs).
//
// Replaces the fused kernel that welder-compiler's GPU codegen emits
// (reference: bench/baselines/default/fused/04c.after_linalg_to_loops.mlir:41-313,
// chain spec mlir/matmul_softmax_chain_f16_native.mlir:7-95).
//
// One workgroup owns a TM x 128 output tile (TM = 128; 256 on the split
// path of large problems).  16-bit and fp8 inputs: 512 threads = 8 waves, 2
// per SIMD (the wave layouts are described at Cfg); k-tiles of 128 bytes of
// K stream through an LDS ring filled by direct-to-LDS buffer loads, B stays
// K-major in LDS and its MFMA operands are read with LDS transpose reads.  f32 inputs:
// 256 threads = 4 waves in a 2x2 grid; k-tiles are loaded `PF` ahead into
// registers (out-of-range lanes read zero, so the outstanding-load count
// stays exact), B is transposed in registers, and a two-stage LDS ring feeds
// the MFMAs.  Accumulation is f32.  The MFMA is issued as D = B^T . A^T so
// that each lane's accumulators belong to ONE output row: row max / sum are
// then in-register, one cross-half swap, and one LDS exchange between the
// waves sharing the row.
//
// Epilogues (template parameter EPI):
//   kEpiExchange  single pass.  Every tile publishes its per-row (max, sumexp)
//                 to HBM, the tiles of one row block (all co-resident, the
//                 launcher checks occupancy) meet at a counter, each merges the
//                 row statistics and writes normalised outputs once.
//   kEpiSplit     first pass of the two-pass online softmax for rows wider
//                 than what can be co-resident: stores exp2(y - tile_max) and
//                 the per-tile (max, sumexp); `rescale_rows_kernel` merges the
//                 statistics and rescales in place.
//   kEpiLogits    stores scale*(A.B) in the output type (first kernel of the
//                 unfused five-kernel baseline).
//
// Note on bit casts: `__builtin_bit_cast(float, vec[e])` applied directly to
// an element of an ext_vector miscompiles with this toolchain (element 0 is
// read for every e); elements are always copied to a scalar first.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "device_common.h"
#include "exchange_entries.h"
#include "tile_layout.h"
#include "wtc_kernels.h"

namespace wtc {

// Phase stamps, built only into the profiling library libwtc_hip_stamps.so
// (WTC_PHASE_STAMPS): lane 0 of every wave of an exchange-path tile reads
// the 100 MHz real-time counter at its phase boundaries, and at the end wave
// 0 and the first loader wave write them to g_phase_stamps[tile][16]:
//   0 start            1 k-tile 0 landed     2 K loop done
//   3 wave statistics  4 entries published and acknowledged
//   5 after the barrier that follows       6 tile staged (before the next)
//   7 after it: the row block's table complete
//   8 factors written  9 after the barrier that follows (generation stored)
//   10 stores acknowledged
//   11, 12 the shader-clock counter (s_memtime) at 1 and 2
//   13, 14 the first loader wave's poll: start, end
//   15 (row block << 8) | XCD
// The stamps add no work to the kernel's phases (counter reads only).
#if defined(WTC_PHASE_STAMPS)
constexpr bool kPhaseStamps = true;
#else
constexpr bool kPhaseStamps = false;
#endif
constexpr int kStampWords = 16;
constexpr int kStampTiles = 4096;
#if defined(WTC_PHASE_STAMPS)
__device__ int64_t g_phase_stamps[kStampTiles * kStampWords];
#endif


constexpr int BM = 128;
constexpr int BN = 128;
constexpr int A_STAGE_BYTES = BM * kKTileBytes;                  // 16 KiB
constexpr int STAGE_BYTES = A_STAGE_BYTES + BN * kKTileBytes;    // 32 KiB

// Per input type, tile height TM and wave layout LW.  16-bit and fp8 inputs
// stream through a ring of direct-to-LDS loads with 8 waves, 2 per SIMD:
//   LW = 0, TM = 128: a 2x4 grid of 64x32 blocks; every wave issues its
//     share of each k-tile's loads between its MFMAs (while one wave of a
//     SIMD waits to issue a load, the other issues MFMAs); 4 stages of 32 KiB.
//   LW = 0, TM = 256: a 4x2 grid of 64x64 blocks, 3 stages of 48 KiB (the
//     split path of large problems: a quarter less L2 and a third less LDS
//     traffic per MFMA).
//   LW = 1, TM = 128 (loader waves): 4 MFMA waves, one per SIMD, in a 2x2
//     grid of 64x64 blocks (a third less LDS read traffic per MFMA than
//     64x32 blocks), and 4 loader waves that issue every direct-to-LDS load,
//     so an MFMA wave never waits for the memory pipeline to take a load.
//     All 8 waves share the epilogue's polling, merging and stores.
// f32 goes through a 2-stage ring filled from registers with 4 waves of
// 64x64 (TM = 128, LW = 0 only).  Every ring keeps k-tiles kt+1 .. kt+3 in
// flight or landed while k-tile kt's fragments are in registers, so 3 stages
// suffice when a stage may be refilled as soon as its fragments have been read.
template <int IN_DT, int TM = 128, int LW = 0> struct Cfg {
  static constexpr bool kDma = IN_DT == DT_F16 || IN_DT == DT_BF16 || IN_DT == DT_FP8;
  static_assert(TM == 128 || (TM == 256 && kDma), "tile height");
  static_assert(LW == 0 || (LW == 1 && kDma && TM == 128), "loader-wave layout");
  static constexpr bool kLoaders = LW == 1;
  static constexpr int kBM = TM;
  static constexpr int kWavesM = kDma ? TM / 64 : 2;                         // MFMA waves along M
  static constexpr int kWavesN = kLoaders ? 2 : (kDma ? 8 / kWavesM : 2);   // ... along N
  static constexpr int kMfmaWaves = kWavesM * kWavesN;
  static constexpr int kWaves = kLoaders ? 2 * kMfmaWaves : kMfmaWaves;
  static constexpr int kLoadWaves = kLoaders ? kWaves - kMfmaWaves : kWaves;  // issue the loads
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kNT = BN / kWavesN / 32;  // 32-column subtiles per MFMA wave
  // MFMA k-steps of one k-tile (16-bit: 4 of 16; fp8: 2 of 64)
  static constexpr int kKSteps = IN_DT == DT_FP8 ? 2 : 4;
  static constexpr int kABlocksPerWave = TM / 8 / kLoadWaves;  // 1 KiB load blocks of A
  static constexpr int kBBlocksPerWave = 16 / kLoadWaves;      // ... and of B
  static constexpr int kAStageBytes = TM * kKTileBytes;
  static constexpr int kStageBytes = kAStageBytes + BN * kKTileBytes;
  static constexpr int kStages = kDma ? (TM == 256 ? 3 : 4) : 2;
  static constexpr int kRingBytes = kStages * kStageBytes;
};


// The epilogue stages the tile in LDS as f32 rows of kStagePitch floats (the
// 4-float pad spreads the 32 rows one wave writes at a time over all banks).
constexpr int kStagePitch = BN + 4;

// The exchange path's table of the row block's tile log-sum-exps, [slot][row]
// with a row pitch of 129 floats (the 4 threads of a row read 4 slots from 4
// different banks), for up to 64 column tiles.
constexpr int kLsePitch = 129;

template <int IN_DT, int OUT_DT, int TM = 128, int LW = 0, bool XCH = false> struct EpiLayout {
  static constexpr int STAGING = TM * kStagePitch * 4;
  // exchange path: the log-sum-exp table follows the staged tile
  static constexpr int LSE_OFF = (STAGING + 255) / 256 * 256;
  static constexpr int LSE_END = XCH ? LSE_OFF + 64 * kLsePitch * 4 : STAGING;
  static constexpr int RING = Cfg<IN_DT, TM, LW>::kRingBytes;
  static constexpr int UNION = LSE_END > RING ? LSE_END : RING;
  static constexpr int RED_OFF = (UNION + 255) / 256 * 256;
  // wstat[kWavesN][TM] (float2), factor[kWavesN][TM] (float), then the
  // exchange path's tile log-sum-exps [TM] (float) and slot generations [64]
  static constexpr int TOTAL = RED_OFF + 3 * Cfg<IN_DT, TM, LW>::kWavesN * TM * 4 + TM * 4 + 64 * 4;
  static_assert(TOTAL <= 160 * 1024, "LDS");
};

// -------------------------------------------------------------------------
// HBM -> registers -> LDS staging of one k-tile.  Every thread issues the same
// straight-line sequence: 4 x 128-bit loads of A and one B block (8 x 64-bit
// for 16-bit types, 16 x 32-bit for fp8, 4 x 128-bit for f32).
// -------------------------------------------------------------------------
struct Tile {
  __amdgpu_buffer_rsrc_t ra, rb;
  int64_t row0, n0, M, N, K, lda, ldb;
};

__device__ inline uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

template <int IN_DT> struct StageRegs {
  u32x4 a[4];
  uint32_t b[16];  // the thread's B k-rows, row-major, 4 columns per row

  __device__ inline void load(const Tile& tl, int kt, int t) {
    constexpr int SZ = dtype_bytes(IN_DT);
    constexpr int EPC = kChunkBytes / SZ;
    const int64_t kb = (int64_t)kt * kKTileBytes + a_load_chunk(t) * kChunkBytes;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t row = tl.row0 + a_load_row(t, j);
      const bool ok = row < tl.M && kb < tl.K * SZ;
      a[j] = bload16(tl.ra, ok ? (uint32_t)(row * tl.lda + kb) : kOutOfRange);
    }
    const int64_t n = tl.n0 + 4 * b_load_colgroup(t);
    const int64_t k0 = (int64_t)kt * (kKTileBytes / SZ) + b_load_chunkrow(t) * EPC;
#pragma unroll
    for (int r = 0; r < EPC; ++r) {
      const int64_t k = k0 + r;
      const bool ok = n < tl.N && k < tl.K;
      const uint32_t off = ok ? (uint32_t)(k * tl.ldb + n * SZ) : kOutOfRange;
      if constexpr (SZ == 2) {
        const u32x2 x = bload8(tl.rb, off);
        b[2 * r] = x[0];
        b[2 * r + 1] = x[1];
      } else if constexpr (SZ == 1) {
        b[r] = bload4(tl.rb, off);
      } else {
        const u32x4 x = bload16(tl.rb, off);
#pragma unroll
        for (int e = 0; e < 4; ++e) b[4 * r + e] = x[e];
      }
    }
  }

  __device__ inline void store(uint8_t* stage, int t) const {
    constexpr int SZ = dtype_bytes(IN_DT);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4*>(stage + a_lds_offset(a_load_row(t, j), a_load_chunk(t))) = a[j];
    const int g = b_load_colgroup(t), kc = b_load_chunkrow(t);
    uint8_t* sB = stage + A_STAGE_BYTES;
    auto rw = [this](int i) { return b[i]; };
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u32x4 v;
#pragma unroll
      for (int w = 0; w < 4; ++w) v[w] = b_unit_word(rw, SZ, c, w);
      *reinterpret_cast<u32x4*>(sB + b_lds_offset(kc, 4 * g + c, BN)) = v;
    }
  }
};

// -------------------------------------------------------------------------
// Direct-to-LDS staging (16-bit inputs).  The loads are issued from inline
// asm with their outstanding count tracked by hand: the compiler would
// otherwise wait for every load in flight before any LDS read, since it
// cannot tell the ring stages apart.  Extra loads in flight can only make
// the compiler's own s_waitcnt more conservative, never unsafe.
// -------------------------------------------------------------------------
// Per-lane byte offsets of one wave's direct-to-LDS loads, computed once:
// k-tile kt of A block j is at a_base[j] + kt*128 (masked to the zero range
// when its chunk lies past K), of B block j at b_base[j] + kt*b_step.  Rows
// past M and k-rows past K fall outside the descriptors' ranges by
// themselves; columns past N are parked at kOutOfRange, which stays out of
// range for every k-tile (kt*b_step < 2^31).
// NBA / NBB: 1 KiB blocks of A / B per wave per k-tile; ASTAGE: bytes of the
// A part of a stage (B follows it).  The wave's blocks are consecutive
// (dma_block), so per lane only the first block's offsets are kept: A block
// j is 8 rows further down (its chunk swizzle recomputed from the row), B
// block j KR k-rows further (its column and chunk do not depend on the
// block).  Few registers: the 256-row tile needs every one it can get.
template <int IN_DT, int NBA, int NBB, int ASTAGE>
struct DmaPlan {
  static constexpr int SZ = dtype_bytes(IN_DT);
  static constexpr int KE = kKTileBytes / SZ;  // k-rows of B per k-tile
  static constexpr int KR = SZ == 1 ? 8 : 4;   // k-rows of B per 1 KiB block
  static constexpr int LPT = NBA + NBB;        // loads per wave per k-tile
  i32x4 ra, rb;
  uint32_t a_off;        // byte offset of the lane's A row in block 0 (chunk added per block)
  uint32_t b_off;        // B byte offset of the lane in block 0, kOutOfRange past N
  uint32_t k_bytes;      // K * element bytes
  uint32_t lda8, b_blk;  // 8 * lda: A bytes per block; KR * ldb: B bytes per block
  uint32_t b_step;       // KE * ldb: bytes of B per k-tile
  uint32_t lds_a0, lds_b0;  // LDS byte offsets of the wave's first A / B block in a stage
  uint32_t a_chunk0;        // A chunk byte offset of the lane in its even blocks
  static_assert(NBA % 2 == 0, "the wave's first A block is even");

  // All extents and pitches fit in 31 bits (the launcher checks that one
  // batch slice of A and of B is below 2 GiB), so everything here is 32-bit.
  __device__ inline void init(const void* a, const void* b, uint32_t a_bytes, uint32_t b_bytes,
                              uint32_t row0, uint32_t n0, uint32_t M_, uint32_t N, uint32_t K,
                              uint32_t lda, uint32_t ldb, int wave_u, int lane) {
    const i32x4 ra_v = raw_rsrc(a, a_bytes), rb_v = raw_rsrc(b, b_bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // wave-uniform: keep them in scalar registers
      ra[i] = __builtin_amdgcn_readfirstlane(ra_v[i]);
      rb[i] = __builtin_amdgcn_readfirstlane(rb_v[i]);
    }
    (void)M_;
    k_bytes = K * SZ;
    b_step = KE * ldb;
    lda8 = 8 * lda;
    b_blk = KR * ldb;
    const int blk_a0 = dma_block(wave_u, 0, NBA);
    const int blk_b0 = dma_block(wave_u, 0, NBB);
    a_off = (row0 + (uint32_t)dma_a_row(blk_a0, lane)) * lda;
    a_chunk0 = (uint32_t)dma_a_chunk(blk_a0, lane) * kChunkBytes;
    // a B chunk is 16 bytes: 8 columns of 16-bit data, 16 of fp8
    const uint32_t krow = SZ == 1 ? (uint32_t)dma8_b_row(blk_b0, lane) : (uint32_t)dma_b_row(blk_b0, lane);
    const uint32_t n = n0 + (SZ == 1 ? 16u * (uint32_t)dma8_b_chunk(blk_b0, lane)
                                     : 8u * (uint32_t)dma_b_chunk(blk_b0, lane));
    b_off = n < N ? krow * ldb + n * SZ : kOutOfRange;
    lds_a0 = blk_a0 * 1024;
    lds_b0 = ASTAGE + blk_b0 * 1024;
  }

  __device__ inline void issue_a(uint32_t stage, int kt, int q) const {
    // block blk_a0 + q: row a_row + 8q, chunk slot (lane % 8) ^ ((row >> 1) % 8)
    // = (lane % 8) ^ ((4 * blk + lane / 16) % 8) (dma_a_chunk); lane / 16 < 4,
    // so for an even first block this is the first block's slot ^ 4 (q odd)
    const uint32_t chunk = a_chunk0 ^ ((q & 1) ? 4u * kChunkBytes : 0u);
    // Rows past M need no test: their offsets lie beyond the batch slice the
    // buffer descriptor covers, so they read zero (and a row's values only
    // ever reach that row's own outputs, which are not stored past M).
    const uint32_t ka = (uint32_t)kt * kKTileBytes;
    dma16(ra, ka + chunk < k_bytes ? a_off + q * lda8 + chunk + ka : kOutOfRange,
          stage + lds_a0 + q * 1024);
  }
  __device__ inline void issue_b(uint32_t stage, int kt, int q) const {
    dma16(rb, b_off != kOutOfRange ? b_off + q * b_blk + (uint32_t)kt * b_step : kOutOfRange,
          stage + lds_b0 + q * 1024);
  }

  // Load j (0 .. LPT-1) of k-tile kt: A and B blocks alternate while both
  // last, the rest of the larger operand follows.
  __device__ inline void issue_one(uint32_t stage, int kt, int j) const {
    constexpr int PAIRS = NBA < NBB ? NBA : NBB;
    if (j < 2 * PAIRS) {
      if (j & 1)
        issue_b(stage, kt, j >> 1);
      else
        issue_a(stage, kt, j >> 1);
    } else if (NBB > NBA) {
      issue_b(stage, kt, j - PAIRS);
    } else {
      issue_a(stage, kt, j - PAIRS);
    }
  }

  // One k-tile (A and B over all waves) into the stage at LDS byte address
  // `stage`.
  __device__ inline void issue(uint32_t stage, int kt) const {
#pragma unroll
    for (int j = 0; j < LPT; ++j) issue_one(stage, kt, j);
  }
};

struct Frags;
__device__ inline void read_frags_tr(const uint8_t* stage, int lane, int wm, int wn, int s, Frags& f);

// -------------------------------------------------------------------------
// MFMA over one LDS stage: wave (wm, wn) accumulates its 64x64 block.
// acc[mt][nt] holds D = B^T A^T for m-subtile mt, n-subtile nt.
// Fragments of step s+1 are read while the MFMAs of step s issue.
// -------------------------------------------------------------------------
struct Frags {
  u32x4 a[2], b[2];
};

__device__ inline void read_frags(const uint8_t* stage, int lane, int wm, int wn, int s, Frags& f) {
  const uint8_t* sA = stage;
  const uint8_t* sB = stage + A_STAGE_BYTES;
  const int r = frag_row(lane);
  const int kch = frag_chunk(lane, s);
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
    f.a[mt] = *reinterpret_cast<const u32x4*>(sA + a_lds_offset(wm * 64 + mt * 32 + r, kch));
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
    f.b[nt] = *reinterpret_cast<const u32x4*>(sB + b_lds_offset(kch, wn * 64 + nt * 32 + r, BN));
}

// 16-bit fragments with B read K-major through the transpose read.
__device__ inline void read_frags_tr(const uint8_t* stage, int lane, int wm, int wn, int s, Frags& f) {
  const uint8_t* sA = stage;
  const uint8_t* sB = stage + A_STAGE_BYTES;
  const int r = frag_row(lane);
  const int kch = frag_chunk(lane, s);
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
    f.a[mt] = *reinterpret_cast<const u32x4*>(sA + a_lds_offset(wm * 64 + mt * 32 + r, kch));
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int nb = wn * 64 + nt * 32;
    const u32x2 lo = tr_read(sB + btr_offset(btr_k(s, 0, lane), btr_n(nb, lane)));
    const u32x2 hi = tr_read(sB + btr_offset(btr_k(s, 1, lane), btr_n(nb, lane)));
    f.b[nt] = u32x4{lo[0], lo[1], hi[0], hi[1]};
  }
}

template <int IN_DT>
__device__ inline void mma_step(const Frags& f, f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      if constexpr (IN_DT == DT_F16) {
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(f16x8, f.b[nt]), __builtin_bit_cast(f16x8, f.a[mt]), acc[mt][nt], 0, 0, 0);
      } else if constexpr (IN_DT == DT_BF16) {
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8, f.b[nt]), __builtin_bit_cast(bf16x8, f.a[mt]), acc[mt][nt], 0, 0, 0);
      } else {
        const u32x4 bv = f.b[nt], av = f.a[mt];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t bw = bv[e], aw = av[e];
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
              __builtin_bit_cast(float, bw), __builtin_bit_cast(float, aw), acc[mt][nt], 0, 0, 0);
        }
      }
    }
}

__device__ inline void mma_step_fp8(const Frags& f0, const Frags& f1, f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const u32x4 a0 = f0.a[mt], a1 = f1.a[mt], b0 = f0.b[nt], b1 = f1.b[nt];
      const i32x8 av = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                        (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
      const i32x8 bv = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3],
                        (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
      acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv, av, acc[mt][nt], 0, 0, 0, 0, 0, 0);
    }
}

template <int IN_DT>
__device__ inline void mma_stage(const uint8_t* stage, int lane, int wm, int wn,
                                 f32x16 (&acc)[2][2]) {
  constexpr int S = kChunksPerKTile / 2;  // chunk-pair steps per k-tile
  Frags f[2];
  read_frags(stage, lane, wm, wn, 0, f[0]);
  if constexpr (IN_DT == DT_FP8) {
#pragma unroll
    for (int s = 0; s < S; s += 2) {
      read_frags(stage, lane, wm, wn, s + 1, f[1]);
      const Frags cur = f[0];
      if (s + 2 < S) read_frags(stage, lane, wm, wn, s + 2, f[0]);
      mma_step_fp8(cur, f[1], acc);
    }
  } else {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (s + 1 < S) read_frags(stage, lane, wm, wn, s + 1, f[(s + 1) & 1]);
      mma_step<IN_DT>(f[s & 1], acc);
    }
  }
}

// All MFMA operands of one k-tile for one wave: A fragments [step][m-subtile],
// B fragments [step][n-subtile], for the wave's KSW k-steps.
template <int NTN, int KSW>
struct KTileFrags {
  u32x4 a[KSW][2], b[KSW][NTN];
};

// Per-lane LDS offsets of a wave's fragment reads inside a stage.  Every read
// of a k-tile is one of these plus a compile-time offset -- the m-subtile adds
// 32 rows (4096 bytes: the A swizzle depends on row/2 mod 8 only), the
// k-step and half (quad) of B add whole k-rows (its swizzle depends on k mod
// 4, fp8: k/2 mod 4 only) -- so a step's reads need these few address
// registers instead of one per read.  A: per k-step s the chunk 2s + lane/32
// (16-bit) or, for fp8, entry 2s + hh for chunk 4s + 2(lane/32) + hh.  B: per
// n-subtile nt (first column nw + nt * 32), k-step 0, half / quad 0.
template <bool F8, int NTN, int KSW, int ASTAGE>
struct FragBase {
  static constexpr int NA = F8 ? 2 * KSW : KSW;
  uint32_t a[NA], b[NTN];
  __device__ inline void init(int lane, int wm, int nw) {
    const int r = frag_row(lane);
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int c = F8 ? 4 * (i >> 1) + 2 * (lane >> 5) + (i & 1) : frag_chunk(lane, i);
      a[i] = (uint32_t)a_lds_offset(wm * 64 + r, c);
    }
#pragma unroll
    for (int nt = 0; nt < NTN; ++nt) {
      const int nb = nw + nt * 32;
      b[nt] = (uint32_t)(ASTAGE + (F8 ? btr8_offset(btr8_k(0, 0, lane), btr8_n(nb, lane))
                                      : btr_offset(btr_k(0, 0, lane), btr_n(nb, lane))));
    }
  }
};

// LDS read i of a k-tile's fragments (2 + 2*NTN reads per k-step s): the two
// A fragments (ds_read_b128), then the halves of the NTN B fragments
// (ds_read_b64_tr_b16).
template <int NTN, int KSW, int ASTAGE>
__device__ inline void read_frag_piece(const uint8_t* stage,
                                       const FragBase<false, NTN, KSW, ASTAGE>& fb, int i,
                                       KTileFrags<NTN, KSW>& f) {
  constexpr int RPS = 2 + 2 * NTN;
  const int s = i / RPS, u = i % RPS;
  if (u < 2) {
    f.a[s][u] = *reinterpret_cast<const u32x4*>(stage + fb.a[s] + u * 4096);
  } else {
    const int nt = (u - 2) >> 1, h = (u - 2) & 1;
    const u32x2 v = tr_read(stage + fb.b[nt] + (16 * s + 4 * h) * 256);
    f.b[s][nt][2 * h] = v[0];
    f.b[s][nt][2 * h + 1] = v[1];
  }
}

// MFMA i of a k-tile (2*NTN per k-step): k-step i / (2*NTN), subtile
// (mt, nt) = ((i / NTN) % 2, i % NTN).
template <int IN_DT, int NTN, int KSW>
__device__ inline void mma_piece(const KTileFrags<NTN, KSW>& f, int i, f32x16 (&acc)[2][NTN]) {
  const int s = i / (2 * NTN), mt = (i / NTN) & 1, nt = i % NTN;
  if constexpr (IN_DT == DT_F16) {
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, f.b[s][nt]), __builtin_bit_cast(f16x8, f.a[s][mt]), acc[mt][nt], 0, 0, 0);
  } else {
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, f.b[s][nt]), __builtin_bit_cast(bf16x8, f.a[s][mt]), acc[mt][nt], 0, 0, 0);
  }
}

// fp8 (e4m3) operands of one k-tile (128 k = 2 MFMA k-steps of 64; KSW of
// them for this wave) for one wave of 64 rows x 32*NTN columns: A
// [step][m-subtile][16-byte half], B [step][n-subtile][8-byte transpose read].
template <int NTN, int KSW>
struct KTileFrags8 {
  u32x4 a[KSW][2][2];
  u32x2 b[KSW][NTN][4];
};

// LDS read i (0 .. KSW*(4+4*NTN)-1) of an fp8 k-tile's fragments: per k-step
// s, reads 0-3 are the A halves (ds_read_b128: chunks 4s + 2(lane/32) + 0/1
// of m-subtiles 0, 1), then four ds_read_b64_tr_b8 of B per n-subtile.
template <int NTN, int KSW, int ASTAGE>
__device__ inline void read_frag_piece8(const uint8_t* stage,
                                        const FragBase<true, NTN, KSW, ASTAGE>& fb, int i,
                                        KTileFrags8<NTN, KSW>& f) {
  constexpr int RPS = 4 + 4 * NTN;
  const int s = i / RPS, u = i % RPS;
  if (u < 4) {
    const int mt = u >> 1, hh = u & 1;
    f.a[s][mt][hh] = *reinterpret_cast<const u32x4*>(stage + fb.a[2 * s + hh] + mt * 4096);
  } else {
    const int nt = (u - 4) >> 2, q = (u - 4) & 3;
    f.b[s][nt][q] = tr8_read(stage + fb.b[nt] + (64 * s + 8 * q) * 128);
  }
}

// MFMA i (0 .. KSW*2*NTN-1) of an fp8 k-tile: k-step i / (2*NTN), m-subtile
// (i / NTN) % 2, n-subtile i % NTN (v_mfma_f32_32x32x64_f8f6f4, both
// operands e4m3, no block scales).
template <int NTN, int KSW>
__device__ inline void mma_piece8(const KTileFrags8<NTN, KSW>& f, int i, f32x16 (&acc)[2][NTN]) {
  const int s = i / (2 * NTN), mt = (i / NTN) & 1, nt = i % NTN;
  const u32x4 a0 = f.a[s][mt][0], a1 = f.a[s][mt][1];
  const u32x2 b0 = f.b[s][nt][0], b1 = f.b[s][nt][1], b2 = f.b[s][nt][2], b3 = f.b[s][nt][3];
  const i32x8 av = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                    (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
  const i32x8 bv = {(int)b0[0], (int)b0[1], (int)b1[0], (int)b1[1],
                    (int)b2[0], (int)b2[1], (int)b3[0], (int)b3[1]};
  acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv, av, acc[mt][nt], 0, 0, 0, 0, 0, 0);
}

// The row exchange's tagged entries, generation words and bounded waits:
// exchange_entries.h.

// Groups of one main-loop step: the smallest g >= loads that divides both
// the fragment reads and the MFMAs of a k-tile (0 if none does).
constexpr int step_groups(int loads, int reads, int mfmas) {
  for (int g = loads; g <= reads && g <= mfmas; ++g)
    if (reads % g == 0 && mfmas % g == 0) return g;
  return 0;
}

// -------------------------------------------------------------------------
// The kernel
// -------------------------------------------------------------------------
// The leading scalar arguments are what a tile needs before its first load
// is issued.  As separate kernel arguments they are preloaded into SGPRs on
// gfx950 (this file is compiled with -amdgpu-kernarg-preload-count), so the
// first k-tiles are requested without waiting for a kernarg fetch; the
// ChainParams fields are only read after that.  grid32 is the launch's
// workgroup count (gridDim.x would be read from the hidden kernel arguments
// in memory).  Sizes and per-batch strides are 32-bit: the launcher keeps one
// batch slice of A, B and out below 2 GiB.
template <int IN_DT, int OUT_DT, int EPI, int PF, int TM, int LW>
__global__ void __launch_bounds__((Cfg<IN_DT, TM, LW>::kThreads), 1)
chain_tile_kernel(const uint8_t* a_in, const uint8_t* b_in, uint32_t M32, uint32_t N32,
                  uint32_t K32, uint32_t lda32, uint32_t ldb32, uint32_t nT32, uint32_t nRB32,
                  uint32_t a_bs32, uint32_t b_bs32, uint32_t grid32, const ChainParams p) {
  using C = Cfg<IN_DT, TM, LW>;
  using L = EpiLayout<IN_DT, OUT_DT, TM, LW, EPI == kEpiExchange>;
  static_assert(EPI != kEpiExchange || TM == 128, "the exchange path runs 128-row tiles");
  constexpr int BM = TM;  // tile rows
  constexpr int NT = C::kThreads;
  constexpr int WN = C::kWavesN;  // MFMA waves along N
  constexpr int NTN = C::kNT;     // 32-column subtiles per MFMA wave
  constexpr bool LDW = C::kLoaders;
  __shared__ __attribute__((aligned(16))) uint8_t smem[L::TOTAL];
  float2* wstat = reinterpret_cast<float2*>(smem + L::RED_OFF);  // [WN][BM] wave (max, sum)
  float* factor = reinterpret_cast<float*>(wstat + WN * BM);     // [WN][BM]

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  // MFMA wave = wm * WN + wn owns rows wm*64 .. +63 and columns nw .. nw +
  // 32*NTN - 1 of the tile; with loader waves (LW = 1) waves kMfmaWaves ..
  // issue the loads and own no block (their wm, wn are not used).
  const int wm = wave / WN, wn = wave % WN;
  const int nw = wn * 32 * NTN;  // first column of the wave's block
  const bool loader = LDW && __builtin_amdgcn_readfirstlane(wave) >= C::kMfmaWaves;

  uint32_t rbg, nt;  // row block across batches, column tile
  tile_of_block(blockIdx.x, grid32, grid32 / nT32, nT32, &rbg, &nt);
  const uint32_t bt = rbg / nRB32;
  const uint32_t rb = rbg - bt * nRB32;
  const int64_t row0 = rb * BM;
  const int64_t n0 = nt * BN;
  [[maybe_unused]] uint64_t tlv[kStampWords] = {};
  auto stamp = [&](int i) {
    if constexpr (kPhaseStamps && EPI == kEpiExchange)
      if (lane == 0) tlv[i] = __builtin_amdgcn_s_memrealtime();
  };
  stamp(0);

  constexpr int SZ = dtype_bytes(IN_DT);
  const int nk = (int)(((uint64_t)K32 * SZ + kKTileBytes - 1) / kKTileBytes);
  // Exchange path: lane j of every wave reads the generation word of slot
  // slot0 + j of the row block (lanes past nT re-read the last one), once the
  // first k-tiles are requested: the load then stays in flight through the
  // main loop.  Unconditional on purpose: under `if (t == 0)`, or ahead of the
  // 32-bit multiply-adds of the load setup -- which the compiler emits as
  // 64-bit multiply-adds with an undefined high addend that may land on the
  // load's destination register -- the compiler waits for it right there.
  const uint32_t slot0 = rbg * nT32;
  uint32_t gen_lane = 0;
  auto load_gen0 = [&]() {
    if constexpr (EPI == kEpiExchange)
      gen_lane = __hip_atomic_load(p.gen + slot0 + ((uint32_t)lane < nT32 ? (uint32_t)lane : nT32 - 1),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };

  f32x16 acc[2][NTN];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NTN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  if constexpr (C::kDma) {
    // ---- main loop, 16-bit / fp8: ring of direct-to-LDS loads -------------
    // k-tile j goes to stage j % S.  Iteration kt: wait until k-tile kt+1 has
    // landed (its fragments are read during this iteration) and every wave
    // has read k-tile kt's fragments (last iteration), refill stage
    // (kt+3) % S -- free by then for S = 3 and S = 4 -- with k-tile kt+3,
    // read k-tile kt+1's fragments into registers and run k-tile kt's MFMAs
    // from the fragments read one iteration earlier: the MFMAs never wait
    // for LDS, and k-tiles kt+2, kt+3 stay in flight.  Each loading wave (all
    // waves, or the loader waves of LW = 1) issues LPT loads per k-tile.
    // Loads past the last k-tile read zeros into stages that are never used.
    constexpr int S = C::kStages;
    constexpr int D = 3;  // k-tiles requested ahead of the one whose MFMAs run
    static_assert(S >= D, "ring depth");
    constexpr int ASTAGE = C::kAStageBytes;
    constexpr int STAGE = C::kStageBytes;
    constexpr bool F8 = IN_DT == DT_FP8;
    using Plan = DmaPlan<IN_DT, C::kABlocksPerWave, C::kBBlocksPerWave, ASTAGE>;
    constexpr int LPT = Plan::LPT;                            // loads per wave per k-tile
    constexpr int KSW = C::kKSteps;  // MFMA k-steps of a k-tile
    constexpr int RPT = F8 ? KSW * (4 + 4 * NTN) : KSW * (2 + 2 * NTN);  // fragment reads
    constexpr int MPT = KSW * 2 * NTN;                                  // MFMAs
    // G groups per k-tile step: the fewest (>= LPT) that divide the reads and
    // the MFMAs evenly (with loader waves the MFMA waves' groups hold no load,
    // and the same interleave of reads and MFMAs keeps the matrix core fed)
    constexpr int G = step_groups(LPT, RPT, MPT);
    static_assert(G > 0, "k-tile step groups");
    using Frags = std::conditional_t<F8, KTileFrags8<NTN, KSW>, KTileFrags<NTN, KSW>>;
    FragBase<F8, NTN, KSW, ASTAGE> fb;
    fb.init(lane, wm, nw);
    auto read_piece = [&](const uint8_t* st, int i, Frags& f) {
      if constexpr (F8)
        read_frag_piece8<NTN, KSW, ASTAGE>(st, fb, i, f);
      else
        read_frag_piece<NTN, KSW, ASTAGE>(st, fb, i, f);
    };
    auto mma = [&](const Frags& f, int i) {
      if constexpr (F8)
        mma_piece8<NTN, KSW>(f, i, acc);
      else
        mma_piece<IN_DT, NTN, KSW>(f, i, acc);
    };
    // the wave's index among the loading waves
    const int wave_u = __builtin_amdgcn_readfirstlane(wave) - (loader ? C::kMfmaWaves : 0);
    Plan d;
    d.init(a_in + (uint64_t)bt * a_bs32, b_in + (uint64_t)bt * b_bs32, a_bs32, b_bs32,
           (uint32_t)row0, (uint32_t)n0, M32, N32, K32, lda32, ldb32, wave_u, lane);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(WTC_LDS uint8_t*)smem;
    if (nk == 0) load_gen0();
    if (nk > 0) {
      if (!LDW || loader) {
#pragma unroll
        for (int q = 0; q < D; ++q) d.issue(lds0 + q * STAGE, q);
      }
      load_gen0();  // newer than the k-tile loads: only makes the waits below stricter
      wait_loads_barrier<LPT * (D - 1)>();  // k-tile 0 landed
      stamp(1);
      if constexpr (kPhaseStamps && EPI == kEpiExchange)
        if (lane == 0) tlv[11] = __builtin_amdgcn_s_memtime();
      if (loader) {
        // Loader waves: the same waits and barriers as the MFMA waves, one
        // per k-tile; after each, k-tile kt+3 into the stage kt+3 % S.
        for (int kt = 0; kt < nk; ++kt) {
          wait_loads_barrier<LPT * (D - 2)>();
          const uint32_t fill = lds0 + ((kt + D) % S) * STAGE;
#pragma unroll
          for (int j = 0; j < LPT; ++j) d.issue_one(fill, kt + D, j);
        }
        wait_loads_barrier<0>();
      } else {
      Frags f0, f1;
#pragma unroll
      for (int i = 0; i < RPT; ++i) read_piece(smem, i, f0);
      // One k-tile step, in G groups of (LW = 0: a load of k-tile kt+3 in
      // the first LPT groups; RPT/G fragment reads of k-tile kt+1, MPT/G
      // MFMAs of k-tile kt).  A wave that issues a direct-to-LDS load stalls
      // until the memory pipeline accepts it; spreading the MFMAs between the
      // loads keeps the matrix core busy through those stalls (with loader
      // waves the MFMA waves never wait there).  sched_barrier pins the
      // groups (MFMAs touch no memory, so the compiler would otherwise move
      // them freely, also across s_barrier).
      auto step = [&](int kt, const Frags& cur, Frags& next) {
        __builtin_amdgcn_sched_barrier(0);
        wait_loads_barrier<LPT * (D - 2)>();  // k-tile kt+1 landed; kt's fragments read
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t fill = lds0 + ((kt + D) % S) * STAGE;
        const uint8_t* rd = smem + ((kt + 1) % S) * STAGE;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          if (!LDW && g < LPT) d.issue_one(fill, kt + D, g);
#pragma unroll
          for (int i = 0; i < RPT / G; ++i) read_piece(rd, (RPT / G) * g + i, next);
#pragma unroll
          for (int i = 0; i < MPT / G; ++i) mma(cur, (MPT / G) * g + i);
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      for (int kt = 0; kt < nk; kt += 2) {
        step(kt, f0, f1);
        if (kt + 1 < nk) step(kt + 1, f1, f0);
      }
      wait_loads_barrier<0>();
      }
      stamp(2);
      if constexpr (kPhaseStamps && EPI == kEpiExchange)
        if (lane == 0) tlv[12] = __builtin_amdgcn_s_memtime();
    }
  } else if (nk == 0) {
    load_gen0();
  } else {
    load_gen0();
    // ---- main loop, fp8 / f32: PF k-tiles in registers, 2-stage LDS ring --
    // k-tile j lives in R[j % PF] and is loaded PF-1 iterations before the
    // iteration that moves it to LDS.  Loads past the last k-tile read zeros
    // (buffer range check), so the steady-state loop issues every load and
    // store unconditionally and the compiler's count of outstanding loads
    // stays exact; the last nk % PF k-tiles run in a guarded tail.
    static_assert(NT == 256 && NTN == 2, "register path layout");
    Tile tl;
    tl.ra = make_rsrc(a_in + (uint64_t)bt * a_bs32, a_bs32);
    tl.rb = make_rsrc(b_in + (uint64_t)bt * b_bs32, b_bs32);
    tl.row0 = row0;
    tl.n0 = n0;
    tl.M = M32;
    tl.N = N32;
    tl.K = K32;
    tl.lda = lda32;
    tl.ldb = ldb32;
    StageRegs<IN_DT> R[PF];
#pragma unroll
    for (int q = 0; q < PF; ++q) R[q].load(tl, q, t);
    R[0].store(smem, t);
    R[0].load(tl, PF, t);
    __syncthreads();
    const int nfull = nk - nk % PF;
    for (int t0 = 0; t0 < nfull; t0 += PF) {
#pragma unroll
      for (int q = 0; q < PF; ++q) {
        const int kt = t0 + q;
        mma_stage<IN_DT>(smem + (kt & 1) * STAGE_BYTES, lane, wm, wn, acc);
        R[(q + 1) % PF].store(smem + ((kt + 1) & 1) * STAGE_BYTES, t);
        R[(q + 1) % PF].load(tl, kt + 1 + PF, t);
        __syncthreads();
      }
    }
#pragma unroll
    for (int q = 0; q + 1 < PF; ++q) {
      const int kt = nfull + q;
      if (kt < nk) {
        mma_stage<IN_DT>(smem + (kt & 1) * STAGE_BYTES, lane, wm, wn, acc);
        R[(q + 1) % PF].store(smem + ((kt + 1) & 1) * STAGE_BYTES, t);
        __syncthreads();
      }
    }
  }

  // ---- epilogue --------------------------------------------------------------
  // Lane owns output rows m_loc(mt) = wm*64 + mt*32 + lane%32 and, for each
  // n-subtile j, the 16 columns n_loc = nw + j*32 + acc_i(lane, v).  Each
  // wave normalises its exponentials against the max of its own columns
  // (wave max m_w, sum s_w per row, kept in LDS); the tile's statistics and
  // the final scale factors are combined from those, so one LDS exchange
  // serves both.  Loader waves (LW = 1) hold no block: they skip the
  // per-wave statistics and the staging and take part in the rest.
  //
  // The statistics run on the raw accumulators: y = c2 * acc (log2 domain)
  // is monotone in acc, so a row's max of y is c2 times its max of acc (its
  // min when c2 < 0; rounding is monotone, so this is exactly the max of the
  // rounded products), and each exponential is exp2(fma(acc, c2, -max)),
  // one instruction before the exponent and one rounding of its argument.
  const int jr = acc_j(lane);
  const int nvalid = p.N - n0 < BN ? (int)(p.N - n0) : BN;  // columns of this tile inside N
  if constexpr (EPI == kEpiLogits) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int j = 0; j < NTN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[mt][j][v] *= p.lin_scale;
  } else {
    float c2 = p.c2;
    if (nvalid < BN) {
      // Ragged last column tile: columns past N get the accumulator value
      // that no max (min) selects and whose exponential is 0: -inf, or +inf
      // when c2 < 0.  A zero scale makes every logit 0: the columns inside N
      // get 0 and the scale 1, so the padding still works.
      if (c2 == 0.0f) c2 = 1.0f;
      const float pad = c2 < 0.0f ? INFINITY : -INFINITY;
      const bool zero = p.c2 == 0.0f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < NTN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int n_loc = nw + j * 32 + acc_i(lane, v);
            acc[mt][j][v] = n_loc < nvalid ? (zero ? 0.0f : acc[mt][j][v]) : pad;
          }
    }
    // Both m-subtiles in one block of straight-line code, with the sign of
    // the scale resolved by one uniform branch around it, so that the
    // scheduler interleaves the two subtiles' reductions and exponentials;
    // each extreme is taken over four independent partial extremes (a max
    // does not depend on the order, so the result is the same).
    auto stats = [&](auto neg_c) {
      constexpr bool NEG = decltype(neg_c)::value;
      auto pick = [](float a, float b) { return NEG ? fminf(a, b) : fmaxf(a, b); };
      // partial extremes per subtile (one on the 256-row layout, whose
      // waves have no registers to spare)
      constexpr int PX = TM == 256 ? 1 : 4;
      float ext[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        // the row's extreme accumulator over the wave's columns (lane l and
        // l ^ 32 hold the two halves of the row)
        float ex[PX];
#pragma unroll
        for (int i = 0; i < PX; ++i) ex[i] = acc[mt][0][i];
#pragma unroll
        for (int j = 0; j < NTN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if (j > 0 || v >= PX) ex[v % PX] = pick(ex[v % PX], acc[mt][j][v]);
        ext[mt] = ex[0];
#pragma unroll
        for (int i = 1; i < PX; ++i) ext[mt] = pick(ext[mt], ex[i]);
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) ext[mt] = NEG ? xor32_min(ext[mt]) : xor32_max(ext[mt]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        // max of y; -inf when every column of the wave lies past N (pad * c2)
        const float mx = ext[mt] * c2;
        const float nbase = mx == -INFINITY ? 0.0f : -mx;
        float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // independent partial sums
#pragma unroll
        for (int j = 0; j < NTN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[mt][j][v], c2, nbase));
            acc[mt][j][v] = e;
            s4[v & 3] += e;
          }
        const float sm = xor32_sum((s4[0] + s4[1]) + (s4[2] + s4[3]));
        if (lane < 32) wstat[wn * BM + wm * 64 + mt * 32 + jr] = make_float2(mx, sm);
      }
    };
    if (!loader) {
      if (c2 < 0.0f)
        stats(std::true_type{});
      else
        stats(std::false_type{});
    }
  }
  stamp(3);

  // The tile's statistics of row r from the WN wave entries.
  auto tile_stat = [&](int r) {
    float tm = wstat[r].x;
#pragma unroll
    for (int w = 1; w < WN; ++w) tm = fmaxf(tm, wstat[w * BM + r].x);
    // tm is finite (every tile has a column inside N); a wave whose columns
    // all lie past N has max -inf and sum 0, and exp2(-inf) = 0
    float ts = 0.0f;
#pragma unroll
    for (int w = 0; w < WN; ++w) {
      const float2 e = wstat[w * BM + r];
      ts += e.y * __builtin_amdgcn_exp2f(e.x - tm);
    }
    return make_float2(tm, ts);
  };
  // A row block of a single column tile (N <= 128) needs no exchange: the
  // tile's own statistics are the row's.
  const bool solo = EPI == kEpiExchange && nT32 == 1u;
  // Exchange path: the generation words of the row block's slots in LDS, and
  // the table of the row block's per-tile log-sum-exps [slot][kLsePitch]
  // (log2 domain; this tile's own slot is filled from its statistics).
  uint32_t* sgen = reinterpret_cast<uint32_t*>(factor + WN * BM + BM);  // [64]
  float* lse_all = reinterpret_cast<float*>(smem + L::LSE_OFF);
  const uint32_t own_slot = slot0 + nt;
  if constexpr (EPI == kEpiExchange)
    if (t < 64 && (uint32_t)t < nT32) sgen[t] = gen_lane;
  if constexpr (EPI != kEpiLogits) {
    __syncthreads();  // the wave statistics (and slot generations) are in place
    if (t < BM) {
      const float2 st = tile_stat(t);
      if constexpr (EPI == kEpiExchange) {
        // publish the row's log-sum-exp over this tile with this launch's tag
        const float lse = st.x + __builtin_amdgcn_logf(st.y);
        lse_all[nt * kLsePitch + t] = lse;
        if (!solo) store_entry(p.ent + (uint64_t)own_slot * BM + t, lse, sgen[nt] + 1u);
        // Wait until the entry stores are acknowledged.  Not for ordering --
        // the tags make every entry self-describing -- but measured: without
        // the wait, entries became visible to the other XCDs late on some
        // MI355X boxes (the exchange took 2-4 us longer), with it never.
        __builtin_amdgcn_s_waitcnt(0);
        stamp(4);
      } else {
        // split: per-tile (max, sumexp) for the rescale kernel
        store_stat(p.partial + ((int64_t)rbg * BM + t) * p.nT + nt, st.x, st.y);
      }
    }
  }

  // Stage the tile in LDS as f32 (the ring is free: every load has landed
  // and every wave is past the last k-tile), for the stores' 16-byte rows.
  float* stg = reinterpret_cast<float*>(smem);
  auto stage_tile = [&]() {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int j = 0; j < NTN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m_loc = wm * 64 + mt * 32 + jr;
          const int n_loc = nw + j * 32 + acc_i(lane, 4 * g);
          *reinterpret_cast<f32x4*>(stg + m_loc * kStagePitch + n_loc) =
              f32x4{acc[mt][j][4 * g], acc[mt][j][4 * g + 1], acc[mt][j][4 * g + 2],
                    acc[mt][j][4 * g + 3]};
        }
  };

  // Exchange path: poll the other tiles' half-slots of the row block into
  // the table.  Polling wave pw of NWP takes half-slots hs = pw, pw + NWP,
  // ... (slot hs / 2, rows (hs % 2) * 64 + lane), U at a time: one wave load
  // is 64 consecutive rows of one slot (512 contiguous bytes), and a
  // half-slot is done when every lane's entry carries the expected tag;
  // otherwise the wave sleeps briefly and reloads only what is not done.
  auto poll_table = [&](int pw_any, int NWP) {
    constexpr int U = 8;
    const int pw = __builtin_amdgcn_readfirstlane(pw_any);  // wave-uniform: scalar branches
    const int nT = (int)nT32;
    bool in_time = true;
    uint64_t waited = 0;
    for (int hb = pw; hb < 2 * nT; hb += U * NWP) {
      bool done[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int hs = hb + NWP * u;
        done[u] = !(hs < 2 * nT && (hs >> 1) != (int)nt);  // wave-uniform
      }
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      for (;;) {
        uint64_t e[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int hs = hb + NWP * u;
          if (!done[u])
            e[u] = load_entry(p.ent + (uint64_t)(slot0 + (hs >> 1)) * BM + (hs & 1) * 64 + lane);
        }
        bool all = true;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int hs = hb + NWP * u, q = hs >> 1;
          if (!done[u]) {
            if (__all(entry_tag(e[u]) == sgen[q] + 1u) || !in_time) {
              done[u] = true;
              lse_all[q * kLsePitch + (hs & 1) * 64 + lane] = entry_lse(e[u]);
            } else {
              all = false;
            }
          }
        }
        if (all) break;
        __builtin_amdgcn_s_sleep(1);
        const uint64_t w = __builtin_amdgcn_s_memrealtime() - t0;
        waited = w > waited ? w : waited;
        if (w > p.spin_ticks) in_time = false;  // one more pass takes what is there
      }
    }
    if (lane == 0 && waited > 0) {
      record_wait(p.err, waited);
      if (!in_time) report_timeout(p.err, p.mailbox);
    }
  };

  if constexpr (EPI == kEpiExchange && LDW) {
    // Loader waves poll as soon as this tile's entries are acknowledged,
    // while the MFMA waves stage the tile.
    __syncthreads();  // this tile's entry stores are acknowledged
    stamp(5);
    if (!loader) {
      stage_tile();
    } else if (!solo) {
      stamp(13);
      poll_table(wave - C::kMfmaWaves, C::kWaves - C::kMfmaWaves);
      stamp(14);
    }
    stamp(6);
    __syncthreads();  // the table and the staged tile are complete
    stamp(7);
  } else {
    if (!loader) stage_tile();
    stamp(6);
    if constexpr (EPI == kEpiExchange) {
      __syncthreads();  // the entries are acknowledged, the own log-sum-exps in the table
      stamp(5);
      if (!solo) {
        stamp(13);
        poll_table(wave, NT / 64);
        stamp(14);
        __syncthreads();  // the table is complete
      }
      stamp(7);
    }
  }

  if constexpr (EPI != kEpiLogits) {
    constexpr int P = NT / BM;  // threads per row (WN, or 2 WN with loader waves)
    static_assert(P % WN == 0 && (P & (P - 1)) == 0 && P <= 4, "threads per row");
    const int r = t / P, h = t % P;
    if constexpr (EPI == kEpiExchange) {
      float gm = -INFINITY, gs = 0.0f;  // running max and sum of exp2(L - gm)
      if (solo) {
        if (h == 0) {  // the row's statistics from this tile's wave entries in LDS
          const float2 ts = tile_stat(r);
          gm = ts.x;
          gs = ts.y;
        }
      } else {
        // Thread h of the row's P merges the tile log-sum-exps q = h, h + P,
        // h + 2P, ... in groups of four: every read is unconditional (an index
        // past nT reads slot 0 and is replaced by -inf), so the four reads
        // issue together.
        const int nT = (int)nT32;
        const int ng = (nT + 4 * P - 1) / (4 * P);
        for (int g = 0; g < ng; ++g) {
          float l[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int q = g * 4 * P + u * P + h;
            const float v = lse_all[(q < nT ? q : 0) * kLsePitch + r];
            l[u] = q < nT ? v : -INFINITY;
          }
          const float nm = fmaxf(gm, fmaxf(fmaxf(l[0], l[1]), fmaxf(l[2], l[3])));
          const float ref = nm == -INFINITY ? 0.0f : nm;  // no entry at all in this share
          float cs = gm == -INFINITY ? 0.0f : gs * __builtin_amdgcn_exp2f(gm - ref);
#pragma unroll
          for (int u = 0; u < 4; ++u) cs += __builtin_amdgcn_exp2f(l[u] - ref);
          gm = nm;
          gs = cs;
        }
      }
      // The P threads of row r are P consecutive lanes of one quad: the row
      // max over the quad (DPP quad permutes xor 1, xor 2), each share
      // rescaled to it, then the sum over the quad.  Some share holds a
      // finite log-sum-exp (every tile has a column inside N), so M is finite;
      // a share without entries has gm = -inf and contributes 0.
      float M = gm;
#pragma unroll
      for (int off = 1; off < P; off <<= 1) M = fmaxf(M, off == 1 ? dpp_quad<0xB1>(M) : dpp_quad<0x4E>(M));
      float S = gm == -INFINITY ? 0.0f : gs * __builtin_amdgcn_exp2f(gm - M);
#pragma unroll
      for (int off = 1; off < P; off <<= 1) S += off == 1 ? dpp_quad<0xB1>(S) : dpp_quad<0x4E>(S);
      // thread (r, h < WN) owns the factor of row r, column slice of wave h:
      // exp2(m_w - L) with L = max + log2(sum) the row's log-sum-exp
      const float row_lse = M + __builtin_amdgcn_logf(S);
      if (h < WN) {
        const float mw = wstat[h * BM + r].x;
        factor[h * BM + r] = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - row_lse);
      }
    } else {
      // split: exponentials relative to the tile max, as the statistics say
      if (h < WN) {
        const float mw = wstat[h * BM + r].x;
        factor[h * BM + r] = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - tile_stat(r).x);
      }
    }
  }
  stamp(8);
  __syncthreads();
  // Every thread has its entries of the other slots: the next launch's
  // entries of this tile's slot may carry the next tag.
  if constexpr (EPI == kEpiExchange)
    if (t == 0 && !solo)
      __hip_atomic_store(p.gen + own_slot, sgen[nt] + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  stamp(9);

  // ---- scale, convert and store: 16 output bytes per thread per step -------
  // The exchange path writes final outputs that this launch never reads
  // again: non-temporal stores keep them from lingering dirty in L2 (C2:
  // 18.2 -> 17.5 us per call).  The split path's outputs are re-read by the
  // rescale kernel and stay ordinary stores (non-temporal ones cost 6 % there).
  uint8_t* o_base = p.out + bt * p.o_bstride;
  constexpr int OSZ = OutTraits<OUT_DT>::SZ;
  // The type the tile's outputs are stored in: the split path keeps its
  // intermediate exponentials (rescaled in place afterwards) in f16 when the
  // output is bf16, so that a bf16 output is rounded to bf16 once.
  constexpr int kStoreDt = EPI == kEpiSplit ? split_store_dt(OUT_DT) : OUT_DT;
  constexpr int EPC = 16 / OSZ;       // elements per 16-byte chunk
  constexpr int CPR = BN / EPC;       // chunks per tile row
  auto store16 = [](uint8_t* dst, const u32x4& v) {
    if constexpr (EPI == kEpiExchange)
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));
    else
      *reinterpret_cast<u32x4*>(dst) = v;
  };
#pragma unroll 4
  for (int idx = t; idx < BM * CPR; idx += NT) {
    const int row = idx / CPR, ch = idx % CPR;
    const int64_t m = row0 + row;
    const int64_t n = n0 + ch * EPC;
    if (m < p.M && n < p.N) {
      const float f = EPI == kEpiLogits ? 1.0f
                      : factor[(ch * EPC / (32 * NTN)) * BM + row] *
                            (EPI == kEpiSplit ? split_store_scale(OUT_DT) : 1.0f);
      const float* src = stg + row * kStagePitch + ch * EPC;
      if constexpr (OSZ == 4) {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(src) * f;
        store16(o_base + m * p.ldo_bytes + n * OSZ, __builtin_bit_cast(u32x4, x0));
      } else {
        uint32_t w0, w1, w2, w3;
        pack4_product<kStoreDt>(*reinterpret_cast<const f32x4*>(src), f, &w0, &w1);
        pack4_product<kStoreDt>(*reinterpret_cast<const f32x4*>(src + 4), f, &w2, &w3);
        store16(o_base + m * p.ldo_bytes + n * OSZ, u32x4{w0, w1, w2, w3});
      }
    }
  }
#if defined(WTC_PHASE_STAMPS)
  if constexpr (EPI == kEpiExchange) {
    __builtin_amdgcn_s_waitcnt(0);
    stamp(10);
    const int first_loader = LDW ? C::kMfmaWaves * 64 : 64;
    if (blockIdx.x < (unsigned)kStampTiles && (t == 0 || t == first_loader)) {
      int64_t* st = g_phase_stamps + (int64_t)blockIdx.x * kStampWords;
      if (t == 0) {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        for (int i = 0; i <= 12; ++i) st[i] = (int64_t)tlv[i];
        st[15] = ((int64_t)rbg << 8) | (xcc & 0xF);
      } else {
        st[13] = (int64_t)tlv[13];
        st[14] = (int64_t)tlv[14];
      }
    }
  }
#endif
}

// -------------------------------------------------------------------------
// Second pass of the split (online two-pass) softmax over tiles of
// 2^tshift columns (128 or 256).  `wpr` waves share a
// row (the launcher picks it so that few, wide rows still give every CU
// enough waves); wave `part` of a row takes its 16-byte chunks part, part +
// wpr, ... in steps of 64 lanes.  Every wave merges the row's nT tile
// statistics into (max, sum) itself, then rescales its chunks of the
// tile-relative exponentials in place: out *= exp2(m_t - M) / S.  Eight
// chunks per lane are loaded before any is stored, so each lane keeps eight
// loads in flight (C5: 36.3 -> 35.1 us against four; C4 unchanged).
// -------------------------------------------------------------------------
template <int OUT_DT>
__global__ void __launch_bounds__(256)
rescale_rows_kernel(uint8_t* __restrict__ out, const float2* __restrict__ partial,
                    int64_t rows_total, int64_t M, int64_t rows_pad, int64_t N,
                    int64_t ldo_bytes, int64_t o_bstride, int nT, int tshift, int wpr) {
  constexpr int MAX_NT = 512;
  constexpr int U = 8;  // chunks in flight per lane
  __shared__ float fac[4][MAX_NT];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + w;  // global wave
  const int64_t grow = gw / wpr;                   // row over batch*M
  const int part = (int)(gw - grow * wpr);
  const bool live = grow < rows_total;
  int64_t bt = 0, m = 0;
  if (live) {
    bt = grow / M;
    m = grow % M;
    // [batch][row, padded to the tile height: rows_pad per batch][column tile]
    const float2* st = partial + (bt * rows_pad + m) * nT;
    float gm = -INFINITY;
    for (int q = lane; q < nT; q += 64) gm = fmaxf(gm, st[q].x);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off));
    float gs = 0.0f;
    for (int q = lane; q < nT; q += 64) gs += st[q].y * __builtin_amdgcn_exp2f(st[q].x - gm);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) gs += __shfl_xor(gs, off);
    const float inv = 1.0f / gs / split_store_scale(OUT_DT);  // the stored values' scale removed
    for (int q = lane; q < nT; q += 64) fac[w][q] = __builtin_amdgcn_exp2f(st[q].x - gm) * inv;
  }
  __syncthreads();
  if (!live) return;
  constexpr int OSZ = OutTraits<OUT_DT>::SZ;
  constexpr int EPC = 16 / OSZ;
  uint8_t* rowp = out + bt * o_bstride + m * ldo_bytes;
  const int64_t nch = N / EPC;                 // 16-byte chunks in the row
  const int64_t step = (int64_t)64 * wpr;      // chunks between a lane's consecutive chunks
  auto scale = [&](u32x4 u, float f) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t x = u[e];
      uint32_t y;
      if constexpr (OUT_DT == DT_F32) {
        y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, x) * f);
      } else if constexpr (OUT_DT == DT_F16) {
        const uint16_t lo = (uint16_t)(x & 0xFFFFu), hi = (uint16_t)(x >> 16);
        const float x0 = (float)__builtin_bit_cast(_Float16, lo) * f;
        const float x1 = (float)__builtin_bit_cast(_Float16, hi) * f;
        y = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x0) |
            ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x1) << 16);
      } else {
        // bf16 output: the tile kernel left its exponentials in f16
        // (split_store_dt), rounded to bf16 once here
        static_assert(split_store_dt(DT_BF16) == DT_F16, "bf16 outputs stage f16 exponentials");
        const uint16_t lo = (uint16_t)(x & 0xFFFFu), hi = (uint16_t)(x >> 16);
        const float x0 = (float)__builtin_bit_cast(_Float16, lo) * f;
        const float x1 = (float)__builtin_bit_cast(_Float16, hi) * f;
        y = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x0) |
            ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x1) << 16);
      }
      u[e] = y;
    }
    return u;
  };
  int64_t c = (int64_t)part * 64 + lane;
  for (; c + (U - 1) * step < nch; c += U * step) {
    u32x4 v[U];
#pragma unroll
    for (int i = 0; i < U; ++i) v[i] = *reinterpret_cast<const u32x4*>(rowp + (c + i * step) * 16);
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int64_t n = (c + i * step) * EPC;
      *reinterpret_cast<u32x4*>(rowp + (c + i * step) * 16) = scale(v[i], fac[w][n >> tshift]);
    }
  }
  for (; c < nch; c += step) {
    const int64_t n = c * EPC;
    *reinterpret_cast<u32x4*>(rowp + c * 16) = scale(*reinterpret_cast<const u32x4*>(rowp + c * 16), fac[w][n >> tshift]);
  }
}

// Zero fill with a kernel (no hipMemset, so it may sit inside a captured graph).
__global__ void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// -------------------------------------------------------------------------
// Instantiation table
// -------------------------------------------------------------------------
constexpr int kPF = 3;

template <int IN_DT, int OUT_DT, int EPI, int TM, int LW>
static const void* tile_kernel_ptr() {
  return reinterpret_cast<const void*>(&chain_tile_kernel<IN_DT, OUT_DT, EPI, kPF, TM, LW>);
}

template <int IN_DT, int EPI, int TM, int LW>
static const void* by_out(int out_dt) {
  switch (out_dt) {
    case DT_F32: return tile_kernel_ptr<IN_DT, DT_F32, EPI, TM, LW>();
    case DT_F16: return tile_kernel_ptr<IN_DT, DT_F16, EPI, TM, LW>();
    case DT_BF16: return tile_kernel_ptr<IN_DT, DT_BF16, EPI, TM, LW>();
  }
  return nullptr;
}

template <int EPI>
static const void* by_in(int in_dt, int out_dt) {
  switch (in_dt) {
    case DT_F32: return by_out<DT_F32, EPI, 128, 0>(out_dt);
    case DT_F16: return by_out<DT_F16, EPI, 128, 0>(out_dt);
    case DT_BF16: return by_out<DT_BF16, EPI, 128, 0>(out_dt);
    case DT_FP8: return by_out<DT_FP8, EPI, 128, 0>(out_dt);
  }
  return nullptr;
}

// 128-row tiles with loader waves (16-bit and fp8 inputs).
template <int EPI>
static const void* loaders_by_in(int in_dt, int out_dt) {
  switch (in_dt) {
    case DT_F16: return by_out<DT_F16, EPI, 128, 1>(out_dt);
    case DT_BF16: return by_out<DT_BF16, EPI, 128, 1>(out_dt);
    case DT_FP8: return by_out<DT_FP8, EPI, 128, 1>(out_dt);
  }
  return nullptr;
}

// 256-row tiles: the split path with 16-bit or fp8 inputs.
static const void* split256_by_in(int in_dt, int out_dt) {
  switch (in_dt) {
    case DT_F16: return by_out<DT_F16, kEpiSplit, 256, 0>(out_dt);
    case DT_BF16: return by_out<DT_BF16, kEpiSplit, 256, 0>(out_dt);
    case DT_FP8: return by_out<DT_FP8, kEpiSplit, 256, 0>(out_dt);
  }
  return nullptr;
}

// f32 logits (the unfused path's first kernel) on the 256-row and loader-wave
// layouts, so that every tile variant also runs the unfused chain.
template <int TM, int LW>
static const void* logits_by_in(int in_dt) {
  switch (in_dt) {
    case DT_F16: return tile_kernel_ptr<DT_F16, DT_F32, kEpiLogits, TM, LW>();
    case DT_BF16: return tile_kernel_ptr<DT_BF16, DT_F32, kEpiLogits, TM, LW>();
    case DT_FP8: return tile_kernel_ptr<DT_FP8, DT_F32, kEpiLogits, TM, LW>();
  }
  return nullptr;
}

const void* chain_kernel_symbol(int in_dt, int out_dt, int epi, int tile_rows, int loaders) {
  if (tile_rows == 256) {
    if (loaders) return nullptr;
    if (epi == kEpiSplit) return split256_by_in(in_dt, out_dt);
    if (epi == kEpiLogits) return out_dt == DT_F32 ? logits_by_in<256, 0>(in_dt) : nullptr;
    return nullptr;
  }
  if (tile_rows != 128) return nullptr;
  if (loaders) {
    if (epi == kEpiExchange) return loaders_by_in<kEpiExchange>(in_dt, out_dt);
    if (epi == kEpiSplit) return loaders_by_in<kEpiSplit>(in_dt, out_dt);
    if (epi == kEpiLogits) return out_dt == DT_F32 ? logits_by_in<128, 1>(in_dt) : nullptr;
    return nullptr;
  }
  if (epi == kEpiExchange) return by_in<kEpiExchange>(in_dt, out_dt);
  if (epi == kEpiSplit) return by_in<kEpiSplit>(in_dt, out_dt);
  if (epi == kEpiLogits) return by_in<kEpiLogits>(in_dt, out_dt);
  return nullptr;
}

const void* rescale_kernel_symbol(int out_dt) {
  switch (out_dt) {
    case DT_F32: return reinterpret_cast<const void*>(&rescale_rows_kernel<DT_F32>);
    case DT_F16: return reinterpret_cast<const void*>(&rescale_rows_kernel<DT_F16>);
    case DT_BF16: return reinterpret_cast<const void*>(&rescale_rows_kernel<DT_BF16>);
  }
  return nullptr;
}

const void* zero_kernel_symbol() { return reinterpret_cast<const void*>(&zero_words_kernel); }

template <int IN_DT, int LW>
static int lds_bytes_for(int out_dt) {
  switch (out_dt) {
    case DT_F32: return EpiLayout<IN_DT, DT_F32, 128, LW, true>::TOTAL;
    case DT_F16: return EpiLayout<IN_DT, DT_F16, 128, LW, true>::TOTAL;
    case DT_BF16: return EpiLayout<IN_DT, DT_BF16, 128, LW, true>::TOTAL;
  }
  return 0;
}

int chain_kernel_threads(int in_dt) {
  switch (in_dt) {
    case DT_F32: return Cfg<DT_F32>::kThreads;
    case DT_F16: return Cfg<DT_F16>::kThreads;
    case DT_BF16: return Cfg<DT_BF16>::kThreads;
    case DT_FP8: return Cfg<DT_FP8>::kThreads;
  }
  return 0;
}

int chain_kernel_lds_bytes(int in_dt, int out_dt, int loaders) {
  if (loaders) {
    switch (in_dt) {
      case DT_F16: return lds_bytes_for<DT_F16, 1>(out_dt);
      case DT_BF16: return lds_bytes_for<DT_BF16, 1>(out_dt);
      case DT_FP8: return lds_bytes_for<DT_FP8, 1>(out_dt);
    }
    return 0;
  }
  switch (in_dt) {
    case DT_F32: return lds_bytes_for<DT_F32, 0>(out_dt);
    case DT_F16: return lds_bytes_for<DT_F16, 0>(out_dt);
    case DT_BF16: return lds_bytes_for<DT_BF16, 0>(out_dt);
    case DT_FP8: return lds_bytes_for<DT_FP8, 0>(out_dt);
  }
  return 0;
}

}  // namespace wtc

#if defined(WTC_PHASE_STAMPS)
// Copies the phase stamps of tiles [0, tiles) of the last exchange launch
// (int64 [tiles][16], layout above) to host memory; synchronous.
extern "C" int wtc_phase_stamps_read(int64_t* host, int64_t tiles) {
  if (!host || tiles <= 0 || tiles > wtc::kStampTiles) return 1;
  const size_t bytes = (size_t)tiles * wtc::kStampWords * sizeof(int64_t);
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(wtc::g_phase_stamps), bytes, 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : 3;
}
#endif
