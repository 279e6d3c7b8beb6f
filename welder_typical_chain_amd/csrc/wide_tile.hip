// wide_tile.hip -- 256x256 output tiles of the chain
//   out[b, M, N] = softmax_row(scale * (A[b, M, K] . B[b, K, N]))
// for the split (online two-pass) path of large problems and for the f32
// logits of the unfused path, on gfx950.
//
// Replaces, like chain_tile_kernel, the fused kernel welder-compiler emits
// (reference: bench/baselines/default/fused/04c.after_linalg_to_loops.mlir:41-313);
// the split epilogue is the first pass of the two-pass softmax whose second
// pass is rescale_rows_kernel (fused_matmul_softmax.hip).
//
// Why a second tile kernel: at large M and N the K loops of the 128-row
// tiles are bound by how fast k-tiles reach LDS (about 30 bytes per clock
// per CU under full load), not by the matrix cores.  A 256x256 tile needs
// 32 bytes of operands per clock of MFMA work at the dense rate, against 48
// for 256x128 and 64 for 128x128.
//
// Shape of a workgroup: 256 threads = 4 waves, one per SIMD, in a 2x2 grid;
// each wave owns a 128x128 block of the tile (4x4 MFMA subtiles of 32x32,
// 256 f32 accumulators per lane).  K streams in k-slabs of 64 bytes (32
// f16/bf16 or 64 fp8 values) through a 4-stage LDS ring of 32 KiB stages,
// filled by direct-to-LDS buffer loads; three slabs are requested ahead of
// the one whose MFMAs run, and the fragments of the next slab are read into
// registers while the MFMAs of the current one issue (the same pipeline as
// chain_tile_kernel's, at half the k-tile and twice the tile).  The MFMA is
// issued as D = B^T . A^T, so each lane's accumulators belong to one output
// row.  Layouts: tile_layout.h (a64_lds_offset for A; B keeps the K-major
// layouts of the 128-column tiles, one per half of the tile's columns).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "device_common.h"
#include "tile_layout.h"
#include "wtc_kernels.h"

namespace wtc {
namespace {

constexpr int kTM = 256;                       // tile rows
constexpr int kTN = 256;                       // tile columns
constexpr int kSlab = 64;                      // bytes of K per ring stage
constexpr int kAStage = kTM * kSlab;           // 16 KiB of A per stage
constexpr int kBHalf = 8192;                   // one 128-column half of B per stage
constexpr int kStage = kAStage + 2 * kBHalf;   // 32 KiB
constexpr int kStages = 4;                     // ring stages (three slabs in flight)
constexpr int kThreads = 256;
constexpr int kLoads = 8;                      // direct-to-LDS loads per wave per slab

// LDS: the ring, reused after the K loop to stage the output tile in the
// output type (f32: two rounds of 128 rows), then the row statistics.
template <int OUT_DT> struct WideLds {
  static constexpr int OSZ = OutTraits<OUT_DT>::SZ;
  static constexpr int ROUNDS = OSZ == 4 ? 2 : 1;
  static constexpr int ROWS = kTM / ROUNDS;     // tile rows staged per round
  static constexpr int PITCH = kTN * OSZ + 16;  // bytes per staged row (16-byte aligned)
  static constexpr int STAGING = ROWS * PITCH;
  static constexpr int RING = kStages * kStage;
  static constexpr int UNION = STAGING > RING ? STAGING : RING;
  static constexpr int RED_OFF = (UNION + 255) / 256 * 256;
  // wred[2][kTM] (per wave column half: the row's max, then its sumexp) and
  // tmax[kTM] (the row's max over the tile), floats
  static constexpr int TOTAL = RED_OFF + 3 * kTM * 4;
  static_assert(TOTAL <= 160 * 1024, "LDS");
};

// Per-lane byte offsets of one wave's direct-to-LDS loads.  Wave w loads A
// blocks 4w .. 4w+3 (rows 64w .. 64w+63) and B blocks 4(w%2) .. 4(w%2)+3 of
// column half w/2; per lane only the first block's offsets are kept (an A
// block is 16 rows further, a B block KR k-rows further; the chunk a lane
// fetches is the same in every block).  Rows past M and k-rows past K lie
// beyond the descriptors' ranges and read zero; columns past N are parked
// at kOutOfRange.
template <int IN_DT> struct WidePlan {
  static constexpr int SZ = dtype_bytes(IN_DT);
  static constexpr int KE = kSlab / SZ;        // k-rows of B per slab
  static constexpr int KR = SZ == 1 ? 8 : 4;   // k-rows of B per 1 KiB block
  i32x4 ra, rb;
  uint32_t a_off, a_chunk, k_bytes, lda16;
  uint32_t b_off, b_blk, b_step;
  uint32_t lds_a, lds_b;

  __device__ inline void init(const void* a, const void* b, uint32_t a_bytes, uint32_t b_bytes,
                              uint32_t row0, uint32_t n0, uint32_t N, uint32_t K, uint32_t lda,
                              uint32_t ldb, int wave, int lane) {
    const i32x4 ra_v = raw_rsrc(a, a_bytes), rb_v = raw_rsrc(b, b_bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = __builtin_amdgcn_readfirstlane(ra_v[i]);
      rb[i] = __builtin_amdgcn_readfirstlane(rb_v[i]);
    }
    k_bytes = K * SZ;
    lda16 = 16 * lda;
    b_blk = KR * ldb;
    b_step = KE * ldb;
    a_off = (row0 + (uint32_t)dma64_a_row(4 * wave, lane)) * lda;
    a_chunk = (uint32_t)dma64_a_chunk(0, lane) * kChunkBytes;
    const int half = wave >> 1, blk = 4 * (wave & 1);
    const uint32_t krow = SZ == 1 ? (uint32_t)dma8_b_row(blk, lane) : (uint32_t)dma_b_row(blk, lane);
    const uint32_t n = n0 + 128u * half +
                       (SZ == 1 ? 16u * (uint32_t)dma8_b_chunk(blk, lane) : 8u * (uint32_t)dma_b_chunk(blk, lane));
    b_off = n < N ? krow * ldb + n * SZ : kOutOfRange;
    lds_a = (uint32_t)wave * 4096u;
    lds_b = (uint32_t)(kAStage + half * kBHalf + blk * 1024);
  }
  __device__ inline void issue_a(uint32_t stage, int kt, int q) const {
    const uint32_t ka = (uint32_t)kt * kSlab;
    dma16(ra, ka + a_chunk < k_bytes ? a_off + q * lda16 + a_chunk + ka : kOutOfRange,
          stage + lds_a + q * 1024);
  }
  __device__ inline void issue_b(uint32_t stage, int kt, int q) const {
    dma16(rb, b_off != kOutOfRange ? b_off + q * b_blk + (uint32_t)kt * b_step : kOutOfRange,
          stage + lds_b + q * 1024);
  }
  // load j (0 .. kLoads-1) of slab kt: A and B blocks alternate
  __device__ inline void issue_one(uint32_t stage, int kt, int j) const {
    if (j & 1)
      issue_b(stage, kt, j >> 1);
    else
      issue_a(stage, kt, j >> 1);
  }
  __device__ inline void issue(uint32_t stage, int kt) const {
#pragma unroll
    for (int j = 0; j < kLoads; ++j) issue_one(stage, kt, j);
  }
};

// Per-lane LDS offsets of a wave's fragment reads inside a stage: two A
// bases (16-bit: k-steps 0 and 1; fp8: the two chunks of the one k-step; an
// m-subtile adds 32 rows = 2048 bytes, the swizzle depends on (row/4) % 4
// only) and one B base per n-subtile (a k-step or k-quad adds whole k-rows;
// the B swizzles depend on k % 4, fp8 (k/2) % 4, only).
template <bool F8> struct WideFragBase {
  uint32_t a[2], b[4];
  __device__ inline void init(int lane, int wm, int wn) {
    const int row = wm * 128 + frag_row(lane);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      a[i] = (uint32_t)a64_lds_offset(row, F8 ? frag64_chunk8(lane, i) : frag64_chunk16(lane, i));
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int nb = nt * 32;
      b[nt] = (uint32_t)(kAStage + wn * kBHalf +
                         (F8 ? btr8_offset(btr8_k(0, 0, lane), btr8_n(nb, lane))
                             : btr_offset(btr_k(0, 0, lane), btr_n(nb, lane))));
    }
  }
};

// A slab's MFMA operands come in two parts, read and consumed in turn, so
// that a wave never holds more than one slab's worth of fragments plus one
// part (the K loop below).
//   16-bit: part s = k-step s (2 per slab): 4 A fragments (ds_read_b128) and
//     4 B fragments of two ds_read_b64_tr_b16 halves each; 12 reads and 16
//     MFMAs per part.
//   fp8 (one k-step of 64 per slab): part 0 = the 4 A fragments (two
//     ds_read_b128 each) and B n-subtiles 0, 1 (four ds_read_b64_tr_b8
//     each), 16 reads; part 1 = B n-subtiles 2, 3, 8 reads.  MFMAs of
//     n-subtiles 0, 1 use part 0; those of 2, 3 use A from part 0 and part 1.
struct Part16 {
  u32x4 a[4];
  u32x4 b[4];  // halves h = 0, 1 in words 2h, 2h+1
};
struct Part8A {
  u32x4 a[4][2];
  u32x2 b[2][4];  // n-subtiles 0, 1
};
struct Part8B {
  u32x2 b[2][4];  // n-subtiles 2, 3
};

// 16-bit: read u (0..11) of k-step s.
__device__ inline void read16(const uint8_t* st, const WideFragBase<false>& fb, int s, int u,
                              Part16& f) {
  if (u < 4) {
    f.a[u] = *reinterpret_cast<const u32x4*>(st + fb.a[s] + u * 2048);
  } else {
    const int nt = (u - 4) >> 1, h = (u - 4) & 1;
    const u32x2 v = tr_read(st + fb.b[nt] + (16 * s + 4 * h) * 256);
    f.b[nt][2 * h] = v[0];
    f.b[nt][2 * h + 1] = v[1];
  }
}
// fp8: A fragment halves of m-subtile mt; B quad q of n-subtile nt.
__device__ inline void read8_a(const uint8_t* st, const WideFragBase<true>& fb, int mt, Part8A& f) {
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
    f.a[mt][hh] = *reinterpret_cast<const u32x4*>(st + fb.a[hh] + mt * 2048);
}
__device__ inline u32x2 read8_b(const uint8_t* st, const WideFragBase<true>& fb, int nt, int q) {
  return tr8_read(st + fb.b[nt] + 8 * q * 128);
}

template <int IN_DT>
__device__ inline void mma16(const Part16& f, int mt, int nt, f32x16 (&acc)[4][4]) {
  if constexpr (IN_DT == DT_F16)
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, f.b[nt]), __builtin_bit_cast(f16x8, f.a[mt]), acc[mt][nt], 0, 0, 0);
  else
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, f.b[nt]), __builtin_bit_cast(bf16x8, f.a[mt]), acc[mt][nt], 0, 0, 0);
}
// v_mfma_f32_32x32x64_f8f6f4, both operands e4m3, no block scales
__device__ inline void mma8(const u32x4 (&a)[2], const u32x2 (&b)[4], f32x16& acc) {
  const u32x4 a0 = a[0], a1 = a[1];
  const u32x2 b0 = b[0], b1 = b[1], b2 = b[2], b3 = b[3];
  const i32x8 av = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                    (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
  const i32x8 bv = {(int)b0[0], (int)b0[1], (int)b1[0], (int)b1[1],
                    (int)b2[0], (int)b2[1], (int)b3[0], (int)b3[1]};
  acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv, av, acc, 0, 0, 0, 0, 0, 0);
}

}  // namespace

// -------------------------------------------------------------------------
// The kernel.  Arguments as chain_tile_kernel's (the leading scalars are
// preloaded into SGPRs; grid32 is the launch's workgroup count).  EPI:
// kEpiSplit (first pass of the two-pass softmax: exp2(y - tile max) in the
// output type and the tile's per-row (max, sumexp)) or kEpiLogits (f32
// scale * A.B).
// -------------------------------------------------------------------------
template <int IN_DT, int OUT_DT, int EPI>
__global__ void __launch_bounds__(kThreads, 1)
chain_wide_kernel(const uint8_t* a_in, const uint8_t* b_in, uint32_t M32, uint32_t N32,
                  uint32_t K32, uint32_t lda32, uint32_t ldb32, uint32_t nT32, uint32_t nRB32,
                  uint32_t a_bs32, uint32_t b_bs32, uint32_t grid32, const ChainParams p) {
  static_assert(IN_DT == DT_F16 || IN_DT == DT_BF16 || IN_DT == DT_FP8, "16-bit or fp8 inputs");
  static_assert(EPI == kEpiSplit || EPI == kEpiLogits, "split or logits epilogue");
  using L = WideLds<OUT_DT>;
  constexpr bool F8 = IN_DT == DT_FP8;
  constexpr int SZ = dtype_bytes(IN_DT);
  __shared__ __attribute__((aligned(16))) uint8_t smem[L::TOTAL];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  uint32_t rbg, nt;  // row block across batches, column tile
  tile_of_block(blockIdx.x, grid32, grid32 / nT32, nT32, &rbg, &nt);
  const uint32_t bt = rbg / nRB32;
  const uint32_t rb = rbg - bt * nRB32;
  const uint32_t row0 = rb * kTM;
  const uint32_t n0 = nt * kTN;
  const int nk = (int)(((uint64_t)K32 * SZ + kSlab - 1) / kSlab);

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // ---- main loop: ring of direct-to-LDS loads ------------------------------
  // Slab j goes to stage j % kStages; slabs 0 .. kStages-1 are requested up
  // front.  Iteration kt (slab kt), with part 0 of slab kt in registers:
  //   phase 0: MFMAs of part 0, reads of part 1 of slab kt;
  //   wait until slab kt+1 has landed and every wave has read slab kt (its
  //   last reads were in phase 0), then refill stage kt % kStages with slab
  //   kt + kStages;
  //   phase 1: MFMAs of part 1 (and, fp8, A of part 0), reads of part 0 of
  //   slab kt+1, and the refill's loads.
  // Three slabs stay in flight while one is computed.  sched_barrier pins
  // the groups of each phase (MFMAs touch no memory, so the compiler would
  // otherwise move them freely, also across s_barrier).  Loads past the last
  // slab read zeros into stages that are never read.
  WideFragBase<F8> fb;
  fb.init(lane, wm, wn);
  WidePlan<IN_DT> d;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  d.init(a_in + (uint64_t)bt * a_bs32, b_in + (uint64_t)bt * b_bs32, a_bs32, b_bs32, row0, n0,
         N32, K32, lda32, ldb32, wave_u, lane);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(WTC_LDS uint8_t*)smem;
  if (nk > 0) {
#pragma unroll
    for (int q = 0; q < kStages; ++q) d.issue(lds0 + q * kStage, q);
    wait_loads_barrier<kLoads * (kStages - 1)>();  // slab 0 landed
    if constexpr (!F8) {
      Part16 p0, p1;
#pragma unroll
      for (int u = 0; u < 12; ++u) read16(smem, fb, 0, u, p0);
      for (int kt = 0; kt < nk; ++kt) {
        const uint8_t* cur = smem + (kt % kStages) * kStage;
        const uint8_t* nxt = smem + ((kt + 1) % kStages) * kStage;
        const uint32_t fill = lds0 + (kt % kStages) * kStage;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
          for (int u = 0; u < 3; ++u) read16(cur, fb, 1, 3 * g + u, p1);
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) mma16<IN_DT>(p0, g, nt, acc);
          __builtin_amdgcn_sched_barrier(0);
        }
        wait_loads_barrier<kLoads * (kStages - 2)>();  // slab kt+1 landed; slab kt read
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          // each load right behind an MFMA, so that the matrix core has work
          // while the wave waits for the memory pipeline to take the load
          mma16<IN_DT>(p1, g, 0, acc);
          __builtin_amdgcn_sched_barrier(0);
          d.issue_one(fill, kt + kStages, 2 * g);
          __builtin_amdgcn_sched_barrier(0);
          mma16<IN_DT>(p1, g, 1, acc);
          __builtin_amdgcn_sched_barrier(0);
          d.issue_one(fill, kt + kStages, 2 * g + 1);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < 3; ++u) read16(nxt, fb, 0, 3 * g + u, p0);
          mma16<IN_DT>(p1, g, 2, acc);
          mma16<IN_DT>(p1, g, 3, acc);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else {
      Part8A pa;
      Part8B pb;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) read8_a(smem, fb, mt, pa);
#pragma unroll
      for (int i = 0; i < 8; ++i) pa.b[i >> 2][i & 3] = read8_b(smem, fb, i >> 2, i & 3);
      for (int kt = 0; kt < nk; ++kt) {
        const uint8_t* cur = smem + (kt % kStages) * kStage;
        const uint8_t* nxt = smem + ((kt + 1) % kStages) * kStage;
        const uint32_t fill = lds0 + (kt % kStages) * kStage;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {  // m-subtile g, n-subtiles 0, 1
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int i = 2 * g + u;
            pb.b[i >> 2][i & 3] = read8_b(cur, fb, 2 + (i >> 2), i & 3);
          }
          mma8(pa.a[g], pa.b[0], acc[g][0]);
          mma8(pa.a[g], pa.b[1], acc[g][1]);
          __builtin_amdgcn_sched_barrier(0);
        }
        wait_loads_barrier<kLoads * (kStages - 2)>();  // slab kt+1 landed; slab kt read
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {  // m-subtile g, n-subtiles 2, 3; then its next A
          // each load right behind an MFMA (as in the 16-bit loop)
          mma8(pa.a[g], pb.b[0], acc[g][2]);
          __builtin_amdgcn_sched_barrier(0);
          d.issue_one(fill, kt + kStages, 2 * g);
          __builtin_amdgcn_sched_barrier(0);
          mma8(pa.a[g], pb.b[1], acc[g][3]);
          __builtin_amdgcn_sched_barrier(0);
          d.issue_one(fill, kt + kStages, 2 * g + 1);
          __builtin_amdgcn_sched_barrier(0);
          read8_a(nxt, fb, g, pa);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int i = 2 * g + u;
            pa.b[i >> 2][i & 3] = read8_b(nxt, fb, i >> 2, i & 3);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    wait_loads_barrier<0>();
  }

  // ---- epilogue --------------------------------------------------------------
  // Lane owns output rows wm*128 + mt*32 + lane%32 and, per n-subtile j, the
  // 16 columns wn*128 + j*32 + acc_i(lane, v).  The accumulators stay where
  // the MFMAs left them (AGPRs) and are streamed one m-subtile at a time
  // (sched_barrier keeps the subtiles apart), so at most 64 of them are in
  // VGPRs at once.  Split path: pass 1 takes each row's max over the tile
  // (per wave, then the two waves of a row through LDS); pass 2 writes
  // exp2(y - tile max) into the staging area (in the output type; bf16
  // outputs: f16 times 2^15, split_store_dt) and sums it.
  const int jr = acc_j(lane);
  float* wred = reinterpret_cast<float*>(smem + L::RED_OFF);  // [2][kTM] wave max, then wave sum
  float* tmax = wred + 2 * kTM;                               // [kTM] tile max per row
  uint8_t* stg = smem;
  constexpr int OSZ = L::OSZ;
  auto stage_quad = [&](int m_loc, int n_loc, const f32x4& x) {
    uint8_t* dst = stg + m_loc * L::PITCH + n_loc * OSZ;
    if constexpr (OSZ == 4) {
      *reinterpret_cast<f32x4*>(dst) = x;
    } else {
      uint32_t w0, w1;
      if constexpr (EPI == kEpiSplit)
        pack4<split_store_dt(OUT_DT)>(x * split_store_scale(OUT_DT), &w0, &w1);
      else
        pack4<OUT_DT>(x, &w0, &w1);
      *reinterpret_cast<u32x2*>(dst) = u32x2{w0, w1};
    }
  };
  if constexpr (EPI == kEpiSplit) {
    // y = c2 * acc (log2 domain); columns past N (ragged last tile only)
    // count as -inf.  Instantiated for full tiles and for both signs of c2,
    // so that pass 1 is a max (c2 >= 0) or a min (c2 < 0) of the raw
    // accumulators and pass 2 one fma per exponential.
    const int nvalid = N32 - n0 < (uint32_t)kTN ? (int)(N32 - n0) : kTN;
    auto split_epi = [&](auto full_c, auto neg_c) {
      constexpr bool FULL = decltype(full_c)::value;
      constexpr bool NEG = decltype(neg_c)::value;
      constexpr float kNone = NEG ? INFINITY : -INFINITY;
      auto valid = [&](int j, int v) { return FULL || wn * 128 + j * 32 + acc_i(lane, v) < nvalid; };
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        float ex = kNone;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float a = valid(j, v) ? acc[mt][j][v] : ex;
            ex = NEG ? fminf(ex, a) : fmaxf(ex, a);
          }
        const float o = __shfl_xor(ex, 32);
        ex = NEG ? fminf(ex, o) : fmaxf(ex, o);
        // every column of this wave past N: -inf (exp2 of it is 0)
        if (lane < 32) wred[wn * kTM + wm * 128 + mt * 32 + jr] = ex == kNone ? -INFINITY : ex * p.c2;
        __builtin_amdgcn_sched_barrier(0);
      }
      __syncthreads();
      tmax[t] = fmaxf(wred[t], wred[kTM + t]);  // finite: every tile has a column inside N
      __syncthreads();
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int m_loc = wm * 128 + mt * 32 + jr;
        const float ntm = -tmax[m_loc];
        float sm = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            f32x4 e;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[mt][j][4 * g + u], p.c2, ntm));
              e[u] = valid(j, 4 * g + u) ? x : 0.0f;
              sm += e[u];
            }
            if (L::ROUNDS == 1) stage_quad(m_loc, wn * 128 + j * 32 + acc_i(lane, 4 * g), e);
          }
        sm = wave_xor32_sum(sm);
        if (lane < 32) wred[wn * kTM + m_loc] = sm;
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    using T = std::true_type;
    using F = std::false_type;
    if (nvalid == kTN) {
      if (p.c2 >= 0.0f) split_epi(T{}, F{});
      else split_epi(T{}, T{});
    } else {
      if (p.c2 >= 0.0f) split_epi(F{}, F{});
      else split_epi(F{}, T{});
    }
    __syncthreads();
    store_stat(p.partial + ((int64_t)rbg * kTM + t) * nT32 + nt, tmax[t], wred[t] + wred[kTM + t]);
  }

  // ---- store: stage in LDS (output type), then 16 bytes per thread per step --
  // The ring is free: every load has landed and every wave is past its last
  // fragment read (the K loop ends with a wait and a barrier).  The split
  // path's outputs are re-read by the rescale kernel: ordinary stores.
  uint8_t* o_base = p.out + (uint64_t)bt * p.o_bstride;
  constexpr int EPC = 16 / OSZ;   // elements per 16-byte chunk
  constexpr int CPR = kTN / EPC;  // chunks per tile row
#pragma unroll
  for (int r = 0; r < L::ROUNDS; ++r) {
    // f32 outputs stage 128 rows (one wave row) per round; 16-bit split
    // outputs were staged by pass 2 above
    if (L::ROUNDS == 2 && wm == r) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int m_loc = wm * 128 + mt * 32 + jr;
        const float tm = EPI == kEpiSplit ? tmax[m_loc] : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            f32x4 x;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int v = 4 * g + u;
              if constexpr (EPI == kEpiSplit) {
                const int n_loc = wn * 128 + j * 32 + acc_i(lane, v);
                const int nvalid = N32 - n0 < (uint32_t)kTN ? (int)(N32 - n0) : kTN;
                x[u] = n_loc < nvalid ? __builtin_amdgcn_exp2f(__builtin_fmaf(acc[mt][j][v], p.c2, -tm)) : 0.0f;
              } else {
                x[u] = acc[mt][j][v] * p.lin_scale;
              }
            }
            stage_quad(mt * 32 + jr, wn * 128 + j * 32 + acc_i(lane, 4 * g), x);
          }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (L::ROUNDS == 2 || EPI != kEpiSplit) __syncthreads();
#pragma unroll 4
    for (int idx = t; idx < L::ROWS * CPR; idx += kThreads) {
      const int row = idx / CPR, ch = idx % CPR;
      const int64_t m = (int64_t)row0 + r * L::ROWS + row;
      const int64_t n = (int64_t)n0 + ch * EPC;
      if (m < p.M && n < p.N)
        *reinterpret_cast<u32x4*>(o_base + m * p.ldo_bytes + n * OSZ) =
            *reinterpret_cast<const u32x4*>(stg + row * L::PITCH + ch * 16);
    }
    if (r + 1 < L::ROUNDS) __syncthreads();
  }
}

// -------------------------------------------------------------------------
// Instantiation table
// -------------------------------------------------------------------------
namespace {
template <int IN_DT, int EPI>
const void* wide_by_out(int out_dt) {
  switch (out_dt) {
    case DT_F32: return reinterpret_cast<const void*>(&chain_wide_kernel<IN_DT, DT_F32, EPI>);
    case DT_F16:
      return EPI == kEpiSplit ? reinterpret_cast<const void*>(&chain_wide_kernel<IN_DT, DT_F16, kEpiSplit>)
                              : nullptr;
    case DT_BF16:
      return EPI == kEpiSplit ? reinterpret_cast<const void*>(&chain_wide_kernel<IN_DT, DT_BF16, kEpiSplit>)
                              : nullptr;
  }
  return nullptr;
}
template <int EPI>
const void* wide_by_in(int in_dt, int out_dt) {
  switch (in_dt) {
    case DT_F16: return wide_by_out<DT_F16, EPI>(out_dt);
    case DT_BF16: return wide_by_out<DT_BF16, EPI>(out_dt);
    case DT_FP8: return wide_by_out<DT_FP8, EPI>(out_dt);
  }
  return nullptr;
}
}  // namespace

const void* wide_kernel_symbol(int in_dt, int out_dt, int epi) {
  if (epi == kEpiSplit) return wide_by_in<kEpiSplit>(in_dt, out_dt);
  if (epi == kEpiLogits) return out_dt == DT_F32 ? wide_by_in<kEpiLogits>(in_dt, out_dt) : nullptr;
  return nullptr;
}

int wide_kernel_threads() { return kThreads; }

}  // namespace wtc
