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
// in registers for both passes; the B column tiles stream through a 4-stage
// LDS ring of direct-to-LDS loads (the same K-major, XOR-swizzled B layout
// and transpose reads as chain_tile_kernel).
//
// 8 waves, 2 x 4: wave (wm, wn) owns rows wm*64 .. +63 and columns
// wn*32 .. +31 of each tile (two 32x32 MFMA subtiles), 2 waves per SIMD.
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
constexpr int WN = 4;               // waves along N
constexpr int NT = 512;             // threads
constexpr int KS = 8;               // k-steps of 16: K <= 128
constexpr int A_KT = KS / 4;        // A k-tiles of 64 elements (128 bytes) per row
constexpr int A_BYTES = A_KT * BM * 128;  // the row block's A, 32 KiB
constexpr int STAGE = KS * 16 * 256;  // one B tile, 128 k-rows x 256 bytes (32 KiB)
constexpr int S = 4;                // ring stages
constexpr int RING_OFF = A_BYTES;
constexpr int BLK = STAGE / 1024;   // 1 KiB load blocks per B tile (32)
constexpr int BPW = BLK / 8;        // B blocks per wave (4)
constexpr int ABPW = A_KT * 16 / 8;  // A blocks per wave (4)
constexpr int LDS_BYTES = RING_OFF + S * STAGE;  // 160 KiB
static_assert(LDS_BYTES <= 160 * 1024, "LDS");
static_assert(2 * WN * BM * 4 <= STAGE, "row statistics fit in one stage");

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
  const int wave = t >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int nw = wn * 32;
  const int jr = acc_j(lane);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);

  // Row blocks of one batch share B: the XCD remap gives each XCD's L2 a
  // contiguous run of row blocks, i.e. whole batches.
  const uint32_t u = xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t bt = u / (uint32_t)p.nRB;
  const uint32_t rb = u - bt * (uint32_t)p.nRB;
  const uint32_t row0 = rb * BM;
  const uint32_t M = (uint32_t)p.M, N = (uint32_t)p.N, K = (uint32_t)p.K;
  const uint32_t lda = (uint32_t)p.lda_bytes, ldb = (uint32_t)p.ldb_bytes;
  const int nT = p.nT;

  // ---- A: the row block (128 rows x K) into LDS once, for both passes -----
  // As A_KT k-tiles of 64 elements in chain_tile_kernel's A-stage layout;
  // chunks past K and rows past M read zero.
  {
    i32x4 rav;
    const i32x4 r = raw_rsrc(p.a + bt * p.a_bstride, (uint32_t)p.a_bstride);
#pragma unroll
    for (int i = 0; i < 4; ++i) rav[i] = __builtin_amdgcn_readfirstlane(r[i]);
    const uint32_t lds_a = (uint32_t)(uintptr_t)(WTC_LDS uint8_t*)smem;
#pragma unroll
    for (int q = 0; q < ABPW; ++q) {
      const int blk = dma_block(wave_u, q, ABPW);  // 0 .. 16*A_KT-1
      const int kt = blk / 16, b = blk % 16;
      const uint32_t row = row0 + (uint32_t)dma_a_row(b, lane);
      const uint32_t kb = (uint32_t)(kt * kKTileBytes + dma_a_chunk(b, lane) * kChunkBytes);
      dma16(rav, row < M && kb < 2 * K ? row * lda + kb : kOutOfRange,
            lds_a + kt * (BM * 128) + b * 1024);
    }
  }
  // A fragment of m-subtile mt, k-step s: row wm*64 + mt*32 + lane%32,
  // k = 16s + 8(lane/32) .. +7.
  auto read_a = [&](int mt, int s) {
    return *reinterpret_cast<const u32x4*>(
        smem + (s / 4) * (BM * 128) + a_lds_offset(wm * 64 + mt * 32 + frag_row(lane), frag_chunk(lane, s % 4)));
  };

  // ---- B tile loads: block q of tile j = k-rows 4q..4q+3, 256 bytes each ---
  i32x4 rbv;
  {
    const i32x4 r = raw_rsrc(p.b + bt * p.b_bstride, (uint32_t)p.b_bstride);
#pragma unroll
    for (int i = 0; i < 4; ++i) rbv[i] = __builtin_amdgcn_readfirstlane(r[i]);
  }
  // A lane's k-row is krow0 + 4q for its load q, and its column group does
  // not depend on q.  k-rows past K are clamped to K, whose offset lies past
  // the buffer descriptor (one batch slice of B, < 2 GiB): they read zero.
  const uint32_t krow0 = (uint32_t)dma_b_row(dma_block(wave_u, 0, BPW), lane);
  const uint32_t bcol = 8u * (uint32_t)dma_b_chunk(dma_block(wave_u, 0, BPW), lane);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(WTC_LDS uint8_t*)smem + RING_OFF;
  const int total = 2 * nT;
  // Tile `it` of the 2*nT-tile stream (pass 1 then pass 2) into its stage;
  // past the end of the stream (it < total + S) the loads read zero.
  auto issue_load = [&](int it, int q) {
    int jt = it >= nT ? it - nT : it;
    jt = jt >= nT ? jt - nT : jt;
    const uint32_t col = (it < total ? (uint32_t)jt * BN : 0x40000000u) + bcol;
    const uint32_t off = min(krow0 + 4u * (uint32_t)q, K) * ldb + col * 2;
    dma16(rbv, col < N ? off : kOutOfRange, lds0 + (it % S) * STAGE + dma_block(wave_u, q, BPW) * 1024);
  };
  // B fragment of k-step s of the tile in stage `st`: columns nw .. nw+31.
  auto read_b = [&](const uint8_t* st, int s) {
    const u32x2 lo = tr_read(st + btr_offset(btr_k(s, 0, lane), btr_n(nw, lane)));
    const u32x2 hi = tr_read(st + btr_offset(btr_k(s, 1, lane), btr_n(nw, lane)));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.out + bt * p.o_bstride, (uint32_t)p.o_bstride);
  const uint32_t ldo = (uint32_t)p.ldo_bytes;
  const float c2 = p.c2;
  constexpr int OSZ = OutTraits<OUT_DT>::SZ;
  // Output stores also count in vmcnt (in order with the loads): a pass-2
  // step leaves NST of them behind its loads, which the waits allow for.
  constexpr int NST = OSZ == 4 ? 8 : 4;

#pragma unroll
  for (int it = 0; it < S - 1; ++it)
#pragma unroll
    for (int q = 0; q < BPW; ++q) issue_load(it, q);

  // The body is instantiated for both signs of the logit scale, so that the
  // tile max of y = c2 * acc is a max (c2 >= 0) or a min (c2 < 0) of acc.
  auto body = [&](auto neg_c) {
    constexpr bool NEG = decltype(neg_c)::value;
    // running statistics (log2 domain) of the lane's two rows over its columns
    float rm[2] = {-INFINITY, -INFINITY}, rs[2] = {0.0f, 0.0f};
    float gsub[2] = {0.0f, 0.0f};  // pass 2: row max + log2(row sum)
    f32x16 ACC[2][2];              // [tile parity][m-subtile]
    // The row block's A fragments (both m-subtiles, all k-steps: 64 VGPRs)
    // are read from LDS once and kept in registers for both passes.  The A
    // loads were issued before the B prologue, so waiting until only the
    // B prologue loads are outstanding means this wave's A is in LDS; the
    // barrier extends that to every wave's share.
    wait_loads_barrier<BPW * (S - 1)>();
    u32x4 areg[2][KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      areg[0][s] = read_a(0, s);
      areg[1][s] = read_a(1, s);
    }

    // Pass-1 statistics of one tile (FULL: no column of the tile is past N),
    // in slices that a step spreads over its load groups: slice 0 the tile
    // maxima of both m-subtiles, slice 1 + mt the exponential sum of m-subtile mt.
    float nbase[2] = {0.0f, 0.0f}, nmax[2] = {0.0f, 0.0f};
    auto ep1 = [&](auto full_c, auto slice_c, const f32x16 (&acc)[2], int j) {
      constexpr bool FULL = decltype(full_c)::value;
      constexpr int SL = decltype(slice_c)::value;
      const int nvalid = (int)N - j * BN;
      if constexpr (SL == 0) {
        float mx[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          mx[mt] = NEG ? INFINITY : -INFINITY;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float x = FULL || nw + acc_i(lane, v) < nvalid ? acc[mt][v] : mx[mt];
            mx[mt] = NEG ? fminf(mx[mt], x) : fmaxf(mx[mt], x);
          }
        }
        const float o0 = __shfl_xor(mx[0], 32), o1 = __shfl_xor(mx[1], 32);
        mx[0] = NEG ? fminf(mx[0], o0) : fmaxf(mx[0], o0);
        mx[1] = NEG ? fminf(mx[1], o1) : fmaxf(mx[1], o1);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const float tm = FULL ? mx[mt] * c2 : (mx[mt] == (NEG ? INFINITY : -INFINITY) ? -INFINITY : mx[mt] * c2);
          nmax[mt] = fmaxf(rm[mt], tm);
          nbase[mt] = FULL ? nmax[mt] : (nmax[mt] == -INFINITY ? 0.0f : nmax[mt]);  // all masked so far
        }
      } else {
        constexpr int mt = SL - 1;
        const float base = nbase[mt];
        float ps[4] = {rs[mt] * __builtin_amdgcn_exp2f(rm[mt] - base), 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[mt][v], c2, -base));
          ps[v & 3] += FULL || nw + acc_i(lane, v) < nvalid ? e : 0.0f;
        }
        rm[mt] = nmax[mt];
        rs[mt] = (ps[0] + ps[1]) + (ps[2] + ps[3]);
      }
    };
    // Pass-2 outputs of one tile: exp2(y - max - log2 sum), stored once, in
    // slices: 2*mt the exponentials of m-subtile mt (packed for 16-bit
    // outputs), 2*mt + 1 their stores.
    uint32_t pw[8];
    float po[16];
    auto ep2 = [&](auto slice_c, const f32x16 (&acc)[2], int j) {
      constexpr int SL = decltype(slice_c)::value;
      constexpr int mt = SL / 2;
      const uint32_t row = row0 + wm * 64 + mt * 32 + jr;
      if constexpr (SL % 2 == 0) {
#pragma unroll
        for (int v = 0; v < 16; ++v)
          po[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[mt][v], c2, -gsub[mt]));
        if constexpr (OSZ != 4) {
#pragma unroll
          for (int g = 0; g < 4; ++g)
            pack4<OUT_DT>(f32x4{po[4 * g], po[4 * g + 1], po[4 * g + 2], po[4 * g + 3]}, &pw[2 * g],
                          &pw[2 * g + 1]);
        }
      } else if constexpr (OSZ == 4) {
        // lane l < 32 holds columns 8g + 0..3, lane l + 32 columns 8g + 4..7
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t col = j * BN + nw + 8 * g + 4 * (lane >> 5);
          const uint32_t off = min(row, M) * ldo + col * 4;  // rows past M: past the descriptor
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4, f32x4{po[4 * g], po[4 * g + 1], po[4 * g + 2], po[4 * g + 3]}),
              ro, col < N ? (int)off : (int)kOutOfRange, 0, 0);
        }
      } else {
        // trade halves with lane ^ 32 so each lane holds two 16-byte runs:
        // l < 32 columns 0-7 and 16-23, l >= 32 columns 8-15 and 24-31.
        // v_permlane32_swap(x, y) leaves {x[0..31], y[0..31]} in x and
        // {x[32..63], y[32..63]} in y, so one swap of words w and w + 2
        // yields words w and w + 2 of the run in every lane, in registers.
        const bool lo = lane < 32;
        const auto q0 = __builtin_amdgcn_permlane32_swap(pw[0], pw[2], false, false);
        const auto q1 = __builtin_amdgcn_permlane32_swap(pw[1], pw[3], false, false);
        const auto q2 = __builtin_amdgcn_permlane32_swap(pw[4], pw[6], false, false);
        const auto q3 = __builtin_amdgcn_permlane32_swap(pw[5], pw[7], false, false);
        const u32x4 run0 = u32x4{q0[0], q1[0], q0[1], q1[1]};
        const u32x4 run1 = u32x4{q2[0], q3[0], q2[1], q3[1]};
        const uint32_t c0 = j * BN + nw + (lo ? 0u : 8u);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t col = c0 + 16u * h;
          const uint32_t off = min(row, M) * ldo + col * 2;  // rows past M: past the descriptor
          __builtin_amdgcn_raw_buffer_store_b128(h ? run1 : run0, ro,
                                                 col < N ? (int)off : (int)kOutOfRange,
                                                 0, 0);
        }
      }
    };

    // Step `it`: MFMAs of tile it into ACC[P] (fragments read from LDS as
    // they are needed), the loads of tile it+S-1, and the epilogue EP of tile
    // it-1 (0 none, 1 pass-1 full, 2 pass-1 ragged, 3 pass 2) from ACC[P^1],
    // all in one basic block so that the scheduler interleaves the
    // epilogue's VALU work with the MFMAs (the matrix core runs an MFMA for
    // 32 cycles while the wave issues other instructions).
    auto step = [&](auto par_c, auto ep_c, int it, auto mma_c) {
      constexpr int P = decltype(par_c)::value;
      constexpr int EP = decltype(ep_c)::value;
      constexpr bool MMA = decltype(mma_c)::value;  // false: the stream's last step (no tile `it`)
      __builtin_amdgcn_sched_barrier(0);
      // tile it landed; every wave is done with stage (it-1)%S
      if (it >= nT + 2)
        wait_loads_barrier<BPW * (S - 2) + NST>();
      else
        wait_loads_barrier<BPW * (S - 2)>();
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* st = smem + RING_OFF + (it % S) * STAGE;
      const int jp = (it - 1) % nT;
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using I3 = std::integral_constant<int, 3>;
      // Group g: load g of tile it+S-1, the MFMAs of k-steps 2g, 2g+1 of tile
      // it, and slice g of the epilogue of tile it-1.  A wave that issues a
      // direct-to-LDS load waits until the memory pipeline takes it; with the
      // loads spread over the step, the matrix core works through those waits.
      auto group = [&](auto g_c) {
        constexpr int g = decltype(g_c)::value;
        static_assert(BPW == 4, "one load per group");
        issue_load(it + S - 1, g);
#pragma unroll
        for (int s2 = 0; s2 < (MMA ? 2 : 0); ++s2) {
          const int s = 2 * g + s2;
          const u32x4 b = read_b(st, s);
          if (s == 0) {
            f32x16 z;
#pragma unroll
            for (int v = 0; v < 16; ++v) z[v] = 0.0f;
            ACC[P][0] = mfma16<IN_DT>(b, areg[0][s], z);
            ACC[P][1] = mfma16<IN_DT>(b, areg[1][s], z);
          } else {
            ACC[P][0] = mfma16<IN_DT>(b, areg[0][s], ACC[P][0]);
            ACC[P][1] = mfma16<IN_DT>(b, areg[1][s], ACC[P][1]);
          }
        }
        if constexpr (EP == 1 || EP == 2) {
          using F = std::integral_constant<bool, EP == 1>;
          if constexpr (g < 3) ep1(F{}, std::integral_constant<int, g>{}, ACC[P ^ 1], jp);
        }
        if constexpr (EP == 3) ep2(std::integral_constant<int, g>{}, ACC[P ^ 1], jp);
        __builtin_amdgcn_sched_barrier(0);
      };
      group(I0{});
      group(I1{});
      group(I2{});
      group(I3{});
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    auto pass1_ep = [&](int it) {  // full or ragged statistics for tile it-1
      return (int)N - ((it - 1) % nT) * BN >= BN;
    };

    using Y = std::true_type;
    step(P0{}, std::integral_constant<int, 0>{}, 0, Y{});
    for (int it = 1; it <= nT; ++it) {
      const bool full = pass1_ep(it);
      if (it & 1) {
        if (full) step(P1{}, std::integral_constant<int, 1>{}, it, Y{});
        else step(P1{}, std::integral_constant<int, 2>{}, it, Y{});
      } else {
        if (full) step(P0{}, std::integral_constant<int, 1>{}, it, Y{});
        else step(P0{}, std::integral_constant<int, 2>{}, it, Y{});
      }
    }
    // Merge the 4 column-waves of each row.  The statistics go to the stage
    // of tile nT once every wave is done reading it (first barrier); it is
    // refilled only after the next step's barrier.  LDS-only barriers: a
    // __syncthreads() would also wait for the tile loads in flight.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float* redmax = reinterpret_cast<float*>(smem + RING_OFF + (nT % S) * STAGE);  // [WN][BM]
    float* redsum = redmax + WN * BM;                                             // [WN][BM]
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      rs[mt] = wave_xor32_sum(rs[mt]);
      if (lane < 32) {
        redmax[wn * BM + wm * 64 + mt * 32 + jr] = rm[mt];
        redsum[wn * BM + wm * 64 + mt * 32 + jr] = rs[mt];
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int row = wm * 64 + mt * 32 + jr;
      float gm = redmax[row];
#pragma unroll
      for (int w = 1; w < WN; ++w) gm = fmaxf(gm, redmax[w * BM + row]);
      float gs = 0.0f;
#pragma unroll
      for (int w = 0; w < WN; ++w) {
        const float mw = redmax[w * BM + row];
        gs += mw == -INFINITY ? 0.0f : redsum[w * BM + row] * __builtin_amdgcn_exp2f(mw - gm);
      }
      gsub[mt] = gm + __builtin_amdgcn_logf(gs);  // v_log_f32 is log2
    }
    for (int it = nT + 1; it < total; ++it) {
      if (it & 1) step(P1{}, std::integral_constant<int, 3>{}, it, Y{});
      else step(P0{}, std::integral_constant<int, 3>{}, it, Y{});
    }
    // the last step only stores tile total-1 (there is no tile `total`)
    if (total & 1) step(P1{}, std::integral_constant<int, 3>{}, total, std::false_type{});
    else step(P0{}, std::integral_constant<int, 3>{}, total, std::false_type{});
  };
  if (c2 >= 0.0f)
    body(std::false_type{});
  else
    body(std::true_type{});
  wait_loads_barrier<0>();
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
