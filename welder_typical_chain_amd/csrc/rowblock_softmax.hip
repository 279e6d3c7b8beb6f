// rowblock_softmax.hip -- the chain for small K (attention scores,
//   out[b] = softmax_row(scale * Q[b] . K[b]^T) with head dim <= 128),
// one workgroup per 128-row block of one batch, all N columns.
//
// When K is small the chain is bound by writing its output, not by the
// MFMAs, so each workgroup computes its logits twice instead of exchanging
// row statistics with other workgroups or rescaling a stored output:
//   pass 1: for every 128-column tile, A.B on MFMA, online row max / sum of
//           exp2 in registers (each wave over its 32 columns of every tile),
//           merged across the 4 column-waves through LDS at the end;
//   pass 2: the same products again, out = exp2(y - max) / sum, stored once.
// The output is written exactly once and nothing else goes to HBM (no
// workspace).  The row block's A goes to LDS once and its MFMA fragments stay
// in registers for both passes; the B column tiles stream through a 3-stage
// LDS ring of direct-to-LDS loads (the same K-major, XOR-swizzled B layout
// and transpose reads as chain_tile_kernel).
//
// 12 waves in two roles, three per SIMD:
//   compute waves 0-7, 2 x 4: wave (wm, wn) owns rows wm*64 .. +63 and
//     columns wn*32 .. +31 of each tile (two 32 x 32 MFMA subtiles); waves w
//     and w + 4 share a SIMD.  For 16-bit outputs they issue no global
//     memory instruction: the MFMAs, the softmax arithmetic and LDS traffic;
//   I/O waves 8-11: the row block's A, every B tile load, and the output
//     stores: 16-bit outputs reach them through an LDS out stage (two, one
//     per tile parity), from which each store instruction writes 4 whole
//     256-byte row segments (full 128-byte lines, non-temporal).
// A wave that issues a load or store waits until the memory pipeline takes
// it; with the I/O waves doing so, the compute waves keep the matrix cores
// and the VALU busy, and with two compute waves per SIMD one issues its
// softmax arithmetic while the other's MFMAs run (one wave alone issues
// VALU work well below the SIMD's rate).  f32 outputs (a 64 KiB tile) are
// stored by the compute waves from registers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "device_common.h"
#include "tile_layout.h"
#include "wtc_kernels.h"

namespace wtc {

namespace rows {

constexpr int BM = 128;             // rows per workgroup
constexpr int BN = 128;             // columns per tile
constexpr int NCW = 8;             // compute waves, 2 x 4 (64 x 32 each)
constexpr int NT = 64 * (NCW + 4);  // threads: 8 compute waves, then 4 I/O waves
constexpr int KS = 8;               // k-steps of 16: K <= 128
constexpr int A_KT = KS / 4;        // A k-tiles of 64 elements (128 bytes) per row
constexpr int A_BYTES = A_KT * BM * 128;  // the row block's A, 32 KiB
constexpr int STAGE = KS * 16 * 256;  // one B tile, 128 k-rows x 256 bytes (32 KiB)
constexpr int OUT_STAGE = BM * 256;   // one tile of 16-bit outputs (32 KiB)
constexpr int S = 3;                // ring stages
constexpr int OUT0 = 0;             // out stage 0: the A region, once A is in registers
constexpr int OUT1 = A_BYTES;       // out stage 1, and the pass-1 statistics merge
constexpr int RING_OFF = OUT1 + OUT_STAGE;
constexpr int BLK = STAGE / 1024;   // 1 KiB load blocks per B tile (32)
constexpr int BPW = BLK / 4;        // B blocks per I/O wave (8)
constexpr int ABPW = A_KT * 16 / 4;  // A blocks per I/O wave (8)
constexpr int SPW = BM / 4 / 4;     // store instructions per I/O wave and tile (8)
constexpr int LDS_BYTES = RING_OFF + S * STAGE;  // 160 KiB
static_assert(LDS_BYTES <= 160 * 1024, "LDS");
static_assert(A_BYTES == OUT_STAGE, "out stage 0 reuses the A region");
static_assert(2 * 4 * BM * 4 <= OUT_STAGE, "row statistics fit in out stage 1");

// the out stage's layout: rows_out_offset (tile_layout.h)
__device__ inline int out_offset(int r, int c) { return rows_out_offset(r, c); }

}  // namespace rows

template <int IN_DT>
__device__ inline f32x16 mfma16(const u32x4& b, const u32x4& a, const f32x16& c) {
  if constexpr (IN_DT == DT_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, b),
                                                  __builtin_bit_cast(f16x8, a), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, b),
                                                   __builtin_bit_cast(bf16x8, a), c, 0, 0, 0);
}

template <int IN_DT, int OUT_DT>
__global__ void __launch_bounds__(rows::NT, 1)
chain_rows_kernel(const ChainParams p) {
  using namespace rows;
  __shared__ __attribute__((aligned(16))) uint8_t smem[LDS_BYTES];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave_u = __builtin_amdgcn_readfirstlane(t >> 6);

  // Row blocks of one batch share B: the XCD remap gives each XCD's L2 a
  // contiguous run of row blocks, i.e. whole batches.
  const uint32_t u = xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t bt = u / (uint32_t)p.nRB;
  const uint32_t rb = u - bt * (uint32_t)p.nRB;
  const uint32_t row0 = rb * BM;
  const uint32_t M = (uint32_t)p.M, N = (uint32_t)p.N, K = (uint32_t)p.K;
  const uint32_t ldo = (uint32_t)p.ldo_bytes;
  const int nT = p.nT;
  const int total = 2 * nT;  // the stream of tiles: pass 1, then pass 2
  constexpr int OSZ = OutTraits<OUT_DT>::SZ;
  constexpr bool STAGED = OSZ == 2;  // outputs leave through the out stages
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.out + bt * p.o_bstride, (uint32_t)p.o_bstride);

  // Barrier schedule, the same count in both roles:
  //   BA      A in LDS;
  //   B(it)   it = 0 .. total+1, at the start of compute step `it`: tile it
  //           in its stage, every wave done with stage (it-1) % S and with
  //           out stage (it-1) & 1 (written in step it-1 for tile it-2,
  //           stored from in I/O step it-1);
  //   BM      between B(nT) and B(nT+1): the pass-1 statistics in LDS.
  if (wave_u >= NCW) {
    // =========================== I/O waves ===================================
    const int v = wave_u - NCW;
    const uint32_t lda = (uint32_t)p.lda_bytes, ldb = (uint32_t)p.ldb_bytes;
    {
      // A: the row block (128 rows x K) into LDS once, as A_KT k-tiles of 64
      // elements in chain_tile_kernel's A-stage layout; chunks past K and
      // rows past M read zero.
      const i32x4 rav = raw_rsrc(p.a + bt * p.a_bstride, (uint32_t)p.a_bstride);
      const uint32_t lds_a = (uint32_t)(uintptr_t)(WTC_LDS uint8_t*)smem;
#pragma unroll
      for (int q = 0; q < ABPW; ++q) {
        const int blk = dma_block(v, q, ABPW);  // 0 .. 16*A_KT-1
        const int kt = blk / 16, b = blk % 16;
        const uint32_t row = row0 + (uint32_t)dma_a_row(b, lane);
        const uint32_t kb = (uint32_t)(kt * kKTileBytes + dma_a_chunk(b, lane) * kChunkBytes);
        dma16(rav, row < M && kb < 2 * K ? row * lda + kb : kOutOfRange,
              lds_a + kt * (BM * 128) + b * 1024);
      }
    }
    // B tile loads: block q of this wave = k-rows 4(BPW v + q) .. +3, 256
    // bytes each.  A lane's k-row is krow0 + 4q for its load q, and its
    // column group does not depend on q.  k-rows past K are clamped to K,
    // whose offset lies past the buffer descriptor (one batch slice of B,
    // < 2 GiB): they read zero.
    const i32x4 rbv = raw_rsrc(p.b + bt * p.b_bstride, (uint32_t)p.b_bstride);
    const uint32_t krow0 = (uint32_t)dma_b_row(dma_block(v, 0, BPW), lane);
    const uint32_t bcol = 8u * (uint32_t)dma_b_chunk(dma_block(v, 0, BPW), lane);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(WTC_LDS uint8_t*)smem + RING_OFF;
    // Tile `it` of the stream into its stage; past the end of the stream
    // (it < total + S) the loads read zero.
    auto issue_load = [&](int it, int q) {
      int jt = it >= nT ? it - nT : it;
      jt = jt >= nT ? jt - nT : jt;
      const uint32_t col = (it < total ? (uint32_t)jt * BN : 0x40000000u) + bcol;
      const uint32_t off = min(krow0 + 4u * (uint32_t)q, K) * ldb + col * 2;
      dma16(rbv, col < N ? off : kOutOfRange, lds0 + (it % S) * STAGE + dma_block(v, q, BPW) * 1024);
    };
    // Stores of stream tile it2 (pass 2, column tile it2 - nT) from out
    // stage it2 & 1: rows v*32 + 4q + lane/16, 16-byte chunk lane % 16.
    auto store_tile = [&](int it2) {
      const uint8_t* os = smem + ((it2 & 1) ? OUT1 : OUT0);
      const int c = lane & 15;
      const uint32_t col = (uint32_t)(it2 - nT) * BN + 8u * (uint32_t)c;
#pragma unroll
      for (int q = 0; q < SPW; ++q) {
        const int r = v * 32 + 4 * q + (lane >> 4);
        const u32x4 x = *reinterpret_cast<const u32x4*>(os + out_offset(r, c));
        const uint32_t row = row0 + (uint32_t)r;
        const uint32_t off = min(row, M) * ldo + col * OSZ;  // rows past M: past the descriptor
        // non-temporal: whole lines, written once and not read back here
        __builtin_amdgcn_raw_buffer_store_b128(x, ro, col < N ? (int)off : (int)kOutOfRange, 0, kCachePolicyNT);
      }
    };
    // I/O step `it` (between B(it) and B(it+1)): the loads of tile it+S-1,
    // BM where it falls, the stores of tile it-2 (ST), then the wait for
    // tile it+1: issued in step it-1 (or the prologue), followed by the
    // stores of step it-1 and this step's loads and stores -- vector memory
    // operations of one wave complete in order.
    auto iostep = [&](int it, auto st_c, auto wait_c, auto merge_c) {
      constexpr bool ST = decltype(st_c)::value;
      constexpr int WAIT = decltype(wait_c)::value;
      constexpr bool MERGE = decltype(merge_c)::value;
#pragma unroll
      for (int q = 0; q < BPW; ++q) issue_load(it + S - 1, q);
      if constexpr (MERGE) asm volatile("s_barrier" ::: "memory");
      if constexpr (ST) store_tile(it - 2);
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(WAIT) : "memory");
    };
    using Y = std::true_type;
    using F = std::false_type;
    using W8 = std::integral_constant<int, BPW>;
    using W16 = std::integral_constant<int, BPW + SPW>;
    using W24 = std::integral_constant<int, BPW + 2 * SPW>;
#pragma unroll
    for (int it = 0; it < S - 1; ++it)
#pragma unroll
      for (int q = 0; q < BPW; ++q) issue_load(it, q);
    wait_loads_barrier<BPW * (S - 1)>();  // BA
    wait_loads_barrier<BPW * (S - 2)>();  // B(0)
    for (int it = 0; it < nT; ++it) iostep(it, F{}, W8{}, F{});
    iostep(nT, F{}, W8{}, Y{});
    if constexpr (STAGED) {
      iostep(nT + 1, F{}, W8{}, F{});
      if (total >= nT + 2) iostep(nT + 2, Y{}, W16{}, F{});  // nT >= 2
      for (int it = nT + 3; it <= total; ++it) iostep(it, Y{}, W24{}, F{});
      // after B(total+1): the last tile's stores
      store_tile(total - 1);
    } else {
      for (int it = nT + 1; it <= total; ++it) iostep(it, F{}, W8{}, F{});
    }
    // every direct-to-LDS load has landed before the workgroup's LDS is freed
    // (no barrier: the compute waves have met their last one)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }

  // ============================= compute waves ===============================
  // Compute wave (wm, wn) owns rows wm*64 .. +63 and columns wn*32 .. +31 of
  // each tile: m-subtiles mt = 0, 1 of 32 x 32.  Waves w and w + 4 share a
  // SIMD, so that one issues its softmax arithmetic while the other's MFMAs
  // run (a wave issues VALU work well below the SIMD's rate on its own).
  const int wm = wave_u >> 2, wn = wave_u & 3;
  const int nw = wn * 32;
  const int jr = acc_j(lane);

  // A fragment of m-subtile mt, k-step s: row wm*64 + mt*32 + lane%32,
  // k = 16s + 8(lane/32) .. +7.
  auto read_a = [&](int mt, int s) {
    return *reinterpret_cast<const u32x4*>(
        smem + (s / 4) * (BM * 128) + a_lds_offset(wm * 64 + mt * 32 + frag_row(lane), frag_chunk(lane, s % 4)));
  };
  // B fragment of k-step s of the tile in stage `st`: columns nw .. nw+31.
  auto read_b = [&](const uint8_t* st, int s) {
    const u32x2 lo = tr_read(st + btr_offset(btr_k(s, 0, lane), btr_n(nw, lane)));
    const u32x2 hi = tr_read(st + btr_offset(btr_k(s, 1, lane), btr_n(nw, lane)));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  const float c2 = p.c2;

  // The body is instantiated for both signs of the logit scale, so that the
  // tile max of y = c2 * acc is a max (c2 >= 0) or a min (c2 < 0) of acc.
  auto body = [&](auto neg_c) {
    constexpr bool NEG = decltype(neg_c)::value;
    // running statistics (log2 domain) of the lane's two rows over its columns
    float rm[2] = {-INFINITY, -INFINITY}, rs[2] = {0.0f, 0.0f};
    float gsub[2] = {0.0f, 0.0f};  // pass 2: row max + log2(row sum)
    float nbase[2] = {0.0f, 0.0f};  // the exponentials' base of the tile being summed
    float ps[2];                    // its running sum, being extended
    f32x16 ACC[2];  // one accumulator per m-subtile
    asm volatile("s_barrier" ::: "memory");  // BA
    // The row block's A fragments (both m-subtiles, all k-steps: 64 VGPRs)
    // are read from LDS once and kept in registers for both passes.
    u32x4 areg[2][KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      areg[0][s] = read_a(0, s);
      areg[1][s] = read_a(1, s);
    }

    // ---- epilogue slice q (0..3) of m-subtile MT of stream tile x ----------
    // EP 1 / 2: pass-1 statistics of a full / ragged tile: the tile maximum
    // and the rescaled running sum in slice 0, the exponentials added in
    // slices 1, 2, the sum kept in slice 3.  EP 3: pass-2 outputs exp2(y - max - log2 sum), four
    // columns per slice; 16-bit outputs are packed, traded with lane ^ 32
    // into 16-byte runs and written to out stage x & 1 (m-subtile 0's runs
    // are held in registers and written in the next step, so that all of a
    // tile's writes fall in one step); f32 outputs are stored directly.
    uint32_t pw[8], hold[8];
    auto epi = [&](auto ep_c, auto mt_c, auto q_c, int x) {
      constexpr int EP = decltype(ep_c)::value;
      constexpr int MT = decltype(mt_c)::value;
      constexpr int Q = decltype(q_c)::value;
      if constexpr (EP == 1 || EP == 2) {
        constexpr bool FULL = EP == 1;
        // column nw + acc_i(lane, v) of the tile is valid when the lane-free
        // part of acc_i is below lim (one register, not one per v)
        const int lim = (int)N - x * BN - nw - 4 * (lane >> 5);
        auto valid = [&](int v) { return FULL || acc_i(0, v) < lim; };
        if constexpr (Q == 0) {
          float mx = NEG ? INFINITY : -INFINITY;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float y = valid(v) ? ACC[MT][v] : mx;
            mx = NEG ? fminf(mx, y) : fmaxf(mx, y);
          }
          mx = NEG ? xor32_min(mx) : xor32_max(mx);
          const float tm = FULL ? mx * c2 : (mx == (NEG ? INFINITY : -INFINITY) ? -INFINITY : mx * c2);
          const float nm = fmaxf(rm[MT], tm);
          nbase[MT] = FULL ? nm : (nm == -INFINITY ? 0.0f : nm);  // all masked so far
          ps[MT] = rs[MT] * __builtin_amdgcn_exp2f(rm[MT] - nbase[MT]);
          rm[MT] = nm;
        } else if constexpr (Q < 3) {
#pragma unroll
          for (int v = 8 * (Q - 1); v < 8 * Q; ++v) {
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(ACC[MT][v], c2, -nbase[MT]));
            ps[MT] += valid(v) ? e : 0.0f;
          }
        } else {
          rs[MT] = ps[MT];
        }
      } else if constexpr (EP == 3) {
        const int r = wm * 64 + MT * 32 + jr;  // row in the block
        float po[4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
          po[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(ACC[MT][4 * Q + v], c2, -gsub[MT]));
        if constexpr (STAGED) {
          pack4<OUT_DT>(f32x4{po[0], po[1], po[2], po[3]}, &pw[2 * Q], &pw[2 * Q + 1]);
          if constexpr (Q == 3) {
            // lane l < 32 now holds columns 8g + 0..3 of the subtile, lane
            // l + 32 columns 8g + 4..7 (words 2g, 2g + 1).  v_permlane32_swap(x,
            // y) leaves {x[0..31], y[0..31]} in x and {x[32..63], y[32..63]}
            // in y, so one swap of words w and w + 2 yields words w and w + 2
            // of a 16-byte run in every lane: l < 32 columns 0-7 and 16-23,
            // l >= 32 columns 8-15 and 24-31.
            const auto q0 = __builtin_amdgcn_permlane32_swap(pw[0], pw[2], false, false);
            const auto q1 = __builtin_amdgcn_permlane32_swap(pw[1], pw[3], false, false);
            const auto q2 = __builtin_amdgcn_permlane32_swap(pw[4], pw[6], false, false);
            const auto q3 = __builtin_amdgcn_permlane32_swap(pw[5], pw[7], false, false);
            const u32x4 run0 = u32x4{q0[0], q1[0], q0[1], q1[1]};
            const u32x4 run1 = u32x4{q2[0], q3[0], q2[1], q3[1]};
            if constexpr (MT == 0) {
#pragma unroll
              for (int w = 0; w < 4; ++w) {
                hold[w] = run0[w];
                hold[4 + w] = run1[w];
              }
            } else {
              uint8_t* os = smem + ((x & 1) ? OUT1 : OUT0);
              const int c0 = wn * 4 + (lane >> 5);  // chunk of run 0; run 1 is c0 + 2
              *reinterpret_cast<u32x4*>(os + out_offset(r, c0)) = run0;
              *reinterpret_cast<u32x4*>(os + out_offset(r, c0 + 2)) = run1;
            }
          }
        } else {
          // f32: lane l < 32 holds columns 8Q + 0..3, lane l + 32 columns 8Q + 4..7
          const uint32_t row = row0 + (uint32_t)r;
          const uint32_t col = (uint32_t)(x - nT) * BN + nw + 8 * Q + 4 * (lane >> 5);
          const uint32_t off = min(row, M) * ldo + col * 4;  // rows past M: past the descriptor
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{po[0], po[1], po[2], po[3]}),
                                                 ro, col < N ? (int)off : (int)kOutOfRange, 0, 0);
        }
      }
    };
    // m-subtile 0's held runs of stream tile x into out stage x & 1
    auto write_hold = [&](int x) {
      uint8_t* os = smem + ((x & 1) ? OUT1 : OUT0);
      const int r = wm * 64 + jr;
      const int c0 = wn * 4 + (lane >> 5);
      *reinterpret_cast<u32x4*>(os + out_offset(r, c0)) = u32x4{hold[0], hold[1], hold[2], hold[3]};
      *reinterpret_cast<u32x4*>(os + out_offset(r, c0 + 2)) = u32x4{hold[4], hold[5], hold[6], hold[7]};
    };

    // Step `it`, in 2 phases after barrier B(it): phase 1 runs the 8 MFMAs
    // of m-subtile 0 of tile it beside the epilogue of m-subtile 1 of tile
    // it-1 (EPA), phase 2 the MFMAs of m-subtile 1 of tile it beside the
    // epilogue of m-subtile 0 of tile it (EPB) -- each epilogue reads an
    // accumulator that no MFMA of its phase writes.  The step's 8 B
    // fragments serve both phases.  Phase 2 is 4 groups of two MFMAs and one
    // epilogue slice, so the matrix core runs while the wave issues the
    // slice; phase 1 issues its epilogue before its MFMAs.  MERGE: the
    // pass-1 statistics of the four column-waves are merged after phase 1
    // (tile it-1 = nT-1 is then complete).
    auto step = [&](auto epa_c, auto epb_c, auto mma_c, auto merge_c, int it) {
      constexpr int EPA = decltype(epa_c)::value;
      constexpr int EPB = decltype(epb_c)::value;
      constexpr bool MMA = decltype(mma_c)::value;  // false: the stream's last step (no tile `it`)
      constexpr bool MERGE = decltype(merge_c)::value;
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // B(it)
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* st = smem + RING_OFF + (it % S) * STAGE;
      u32x4 bf[KS];
      if constexpr (MMA) {
#pragma unroll
        for (int s = 0; s < KS; ++s) bf[s] = read_b(st, s);
      }
      if constexpr (EPA == 3 && STAGED) write_hold(it - 1);
      auto phase = [&](auto ph_c) {
        constexpr int PH = decltype(ph_c)::value;
        constexpr int I = PH - 1;   // m-subtile of the MFMAs
        constexpr int EI = PH & 1;  // m-subtile of the epilogue
        constexpr int EP = PH == 1 ? EPA : EPB;
        const int x = PH == 1 ? it - 1 : it;
        auto group = [&](auto q_c) {
          constexpr int Q = decltype(q_c)::value;
          // Phase 1: the whole epilogue first, while the step's B fragment
          // reads are in flight (an MFMA that waits for its fragment holds
          // up the instructions behind it).
          if constexpr (PH == 1 && Q == 0 && EP != 0) {
            epi(std::integral_constant<int, EP>{}, std::integral_constant<int, EI>{}, std::integral_constant<int, 0>{}, x);
            epi(std::integral_constant<int, EP>{}, std::integral_constant<int, EI>{}, std::integral_constant<int, 1>{}, x);
            epi(std::integral_constant<int, EP>{}, std::integral_constant<int, EI>{}, std::integral_constant<int, 2>{}, x);
            epi(std::integral_constant<int, EP>{}, std::integral_constant<int, EI>{}, std::integral_constant<int, 3>{}, x);
            __builtin_amdgcn_sched_barrier(0);
          }
          if constexpr (MMA) {
#pragma unroll
            for (int s = 2 * Q; s < 2 * Q + 2; ++s) {
              if constexpr (Q == 0) {
                if (s == 0) {
                  f32x16 z;
#pragma unroll
                  for (int v = 0; v < 16; ++v) z[v] = 0.0f;
                  ACC[I] = mfma16<IN_DT>(bf[s], areg[I][s], z);
                } else {
                  ACC[I] = mfma16<IN_DT>(bf[s], areg[I][s], ACC[I]);
                }
              } else {
                ACC[I] = mfma16<IN_DT>(bf[s], areg[I][s], ACC[I]);
              }
            }
          }
          if constexpr (PH == 2 && EP != 0) epi(std::integral_constant<int, EP>{}, std::integral_constant<int, EI>{}, q_c, x);
          __builtin_amdgcn_sched_barrier(0);
        };
        group(std::integral_constant<int, 0>{});
        group(std::integral_constant<int, 1>{});
        group(std::integral_constant<int, 2>{});
        group(std::integral_constant<int, 3>{});
      };
      phase(std::integral_constant<int, 1>{});
      if constexpr (MERGE) {
        // BM: merge the 4 column-waves of each row through out stage 1,
        // which holds no output before step nT + 1.
        float* redmax = reinterpret_cast<float*>(smem + OUT1);  // [4][BM]
        float* redsum = redmax + 4 * BM;                        // [4][BM]
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const float sum = xor32_sum(rs[mt]);
          if (lane < 32) {
            redmax[wn * BM + wm * 64 + mt * 32 + jr] = rm[mt];
            redsum[wn * BM + wm * 64 + mt * 32 + jr] = sum;
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int row = wm * 64 + mt * 32 + jr;
          float gm = redmax[row];
#pragma unroll
          for (int w = 1; w < 4; ++w) gm = fmaxf(gm, redmax[w * BM + row]);
          float gs = 0.0f;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float mw = redmax[w * BM + row];
            gs += mw == -INFINITY ? 0.0f : redsum[w * BM + row] * __builtin_amdgcn_exp2f(mw - gm);
          }
          gsub[mt] = gm + __builtin_amdgcn_logf(gs);  // v_log_f32 is log2
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      phase(std::integral_constant<int, 2>{});
    };
    using Y = std::true_type;
    using F = std::false_type;
    using E0 = std::integral_constant<int, 0>;
    using E1 = std::integral_constant<int, 1>;
    using E2 = std::integral_constant<int, 2>;
    using E3 = std::integral_constant<int, 3>;
    // pass-1 tile x is ragged when it is the last column tile and N % BN != 0
    const bool last_ragged = (int)N - (nT - 1) * BN < BN;
    if (nT == 1 && last_ragged) step(E0{}, E2{}, Y{}, F{}, 0);
    else step(E0{}, E1{}, Y{}, F{}, 0);
    for (int it = 1; it < nT; ++it) {
      if (it == nT - 1 && last_ragged) step(E1{}, E2{}, Y{}, F{}, it);
      else step(E1{}, E1{}, Y{}, F{}, it);
    }
    if (last_ragged) step(E2{}, E3{}, Y{}, Y{}, nT);
    else step(E1{}, E3{}, Y{}, Y{}, nT);
    for (int it = nT + 1; it < total; ++it) step(E3{}, E3{}, Y{}, F{}, it);
    // the last step only finishes tile total-1 (there is no tile `total`)
    step(E3{}, E0{}, F{}, F{}, total);
  };
  if (c2 >= 0.0f)
    body(std::false_type{});
  else
    body(std::true_type{});
  // B(total+1): the last tile's out stage is complete for the I/O waves
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int IN_DT>
static const void* rows_by_out(int out_dt) {
  switch (out_dt) {
    case DT_F32: return reinterpret_cast<const void*>(&chain_rows_kernel<IN_DT, DT_F32>);
    case DT_F16: return reinterpret_cast<const void*>(&chain_rows_kernel<IN_DT, DT_F16>);
    case DT_BF16: return reinterpret_cast<const void*>(&chain_rows_kernel<IN_DT, DT_BF16>);
  }
  return nullptr;
}

const void* rows_kernel_symbol(int in_dt, int out_dt) {
  if (in_dt == DT_F16) return rows_by_out<DT_F16>(out_dt);
  if (in_dt == DT_BF16) return rows_by_out<DT_BF16>(out_dt);
  return nullptr;
}

int rows_kernel_threads() { return rows::NT; }
int rows_kernel_max_k() { return rows::KS * 16; }

}  // namespace wtc
