// layout_check.cpp -- CPU replay of one workgroup of chain_tile_kernel (and
// of one k-slab of chain_wide_kernel's 256x256 tile).
//
// Uses the kernel's own index maps (welder_typical_chain_amd/csrc/tile_layout.h)
// to move one k-tile of A and B from "HBM" through the register transpose into
// the LDS stage, read the MFMA fragments back, run a reference model of the
// 32x32xK MFMA (lane l supplies row/column l%32 and k-group l/32; register v of
// the result holds D[8*(v/4) + 4*(l/32) + v%4][l%32]), and map the
// accumulators to output coordinates the way the epilogue does.  Values are
// small integers so the products are exact; the result must equal the plain
// integer matmul.  Also checks that every LDS byte of the stage is written
// exactly once, that the XCD remap is a bijection, and counts LDS bank
// conflicts (64 banks x 4 bytes, 16 lanes per 128-bit access phase).  Also
// replays the row-block kernel's pass-2 output hand-off through its LDS out
// stage (run_rows_out).
//
// Build: g++ -O2 -std=c++17 -I<csrc> layout_check.cpp; prints "OK" and exits 0.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <vector>

#include "tile_layout.h"

using namespace wtc;

static int g_fail = 0;
#define CHECK(c, ...)                           \
  do {                                          \
    if (!(c)) {                                 \
      if (g_fail < 20) std::printf(__VA_ARGS__); \
      ++g_fail;                                 \
    }                                           \
  } while (0)

constexpr int BM = 128, BN = 128;

struct Conflicts {
  int worst = 1;
  void phase(const std::vector<int>& addrs, int bytes_per_lane) {
    // addrs: byte address per lane of one 16-lane phase
    std::map<int, int> use;
    for (int a : addrs)
      for (int d = 0; d < bytes_per_lane / 4; ++d) use[((a / 4) + d) % 64]++;
    for (auto& kv : use) worst = std::max(worst, kv.second);
  }
};

static int64_t elem(const std::vector<uint8_t>& buf, size_t off, int sz) {
  if (sz == 1) return buf[off];
  if (sz == 2) { uint16_t x; std::memcpy(&x, buf.data() + off, 2); return x; }
  uint32_t x; std::memcpy(&x, buf.data() + off, 4); return x;
}

static void run(int sz, const char* name) {
  const int KE = kKTileBytes / sz;  // elements of K in one k-tile
  const int EPC = kChunkBytes / sz;
  // global tiles with small distinct-ish integer values
  std::vector<uint8_t> A((size_t)BM * kKTileBytes), B((size_t)KE * BN * sz);
  for (int m = 0; m < BM; ++m)
    for (int k = 0; k < KE; ++k) {
      uint32_t v = (uint32_t)((m * 7 + k * 3) % 13 + 1);
      std::memcpy(A.data() + (size_t)m * kKTileBytes + k * sz, &v, sz);
    }
  for (int k = 0; k < KE; ++k)
    for (int n = 0; n < BN; ++n) {
      uint32_t v = (uint32_t)((k * 5 + n * 11) % 17 + 1);
      std::memcpy(B.data() + ((size_t)k * BN + n) * sz, &v, sz);
    }
  const int A_STAGE = BM * kKTileBytes;
  std::vector<uint8_t> lds((size_t)A_STAGE + BN * kKTileBytes, 0);
  std::vector<int> cover(lds.size(), 0);
  Conflicts cw_a, cw_b, cr_a, cr_b;

  // ---- A: all 256 threads, 4 passes of one 16-byte chunk each
  for (int j = 0; j < 4; ++j)
    for (int wave = 0; wave < 4; ++wave)
      for (int ph = 0; ph < 4; ++ph) {
        std::vector<int> addrs;
        for (int l = ph * 16; l < ph * 16 + 16; ++l) {
          const int t = wave * 64 + l;
          const int row = a_load_row(t, j), c = a_load_chunk(t);
          const int off = a_lds_offset(row, c);
          addrs.push_back(off);
          std::memcpy(lds.data() + off, A.data() + (size_t)row * kKTileBytes + c * 16, 16);
          for (int b = 0; b < 16; ++b) cover[off + b]++;
        }
        cw_a.phase(addrs, 16);
      }
  // ---- B: all 256 threads transpose an (EPC k) x 4 block into 4 chunks
  for (int c = 0; c < 4; ++c)
    for (int wave = 0; wave < 4; ++wave)
      for (int ph = 0; ph < 4; ++ph) {
        std::vector<int> addrs;
        for (int l = ph * 16; l < ph * 16 + 16; ++l) {
          const int t = wave * 64 + l;
          const int g = b_load_colgroup(t), kc = b_load_chunkrow(t);
          // the loader's k-rows as 16 row-major words, 4 columns per row
          uint32_t words[16];
          const int rows = EPC, row_bytes = 4 * sz;
          for (int r = 0; r < rows; ++r)
            std::memcpy(reinterpret_cast<uint8_t*>(words) + r * row_bytes,
                        B.data() + ((size_t)(kc * EPC + r) * BN + 4 * g) * sz, row_bytes);
          auto rw = [&](int i) { return words[i]; };
          uint32_t unit[4];
          for (int w = 0; w < 4; ++w) unit[w] = b_unit_word(rw, sz, c, w);
          const int off = A_STAGE + b_lds_offset(kc, 4 * g + c, BN);
          addrs.push_back(off);
          std::memcpy(lds.data() + off, unit, 16);
          for (int b = 0; b < 16; ++b) cover[off + b]++;
        }
        cw_b.phase(addrs, 16);
      }
  for (size_t i = 0; i < cover.size(); ++i)
    CHECK(cover[i] == 1, "[%s] LDS byte %zu written %d times\n", name, i, cover[i]);

  // ---- fragments + reference MFMA
  std::vector<int64_t> acc(4 * 4 * 64 * 16, 0);  // [wave][mt*2+nt][lane][v]
  auto ACC = [&](int wave, int mt, int nt, int l, int v) -> int64_t& {
    return acc[(((size_t)wave * 4 + mt * 2 + nt) * 64 + l) * 16 + v];
  };
  const int steps = kChunksPerKTile / 2;  // chunk pairs per k-tile
  for (int wave = 0; wave < 4; ++wave) {
    const int wm = wave >> 1, wn = wave & 1;
    for (int s = 0; s < steps; ++s) {
      // operand bytes per lane: [lane][16]
      std::vector<std::vector<uint8_t>> af(2, std::vector<uint8_t>(64 * 16)), bf(2, std::vector<uint8_t>(64 * 16));
      for (int mt = 0; mt < 2; ++mt)
        for (int ph = 0; ph < 4; ++ph) {
          std::vector<int> addrs;
          for (int l = ph * 16; l < ph * 16 + 16; ++l) {
            const int off = a_lds_offset(wm * 64 + mt * 32 + frag_row(l), frag_chunk(l, s));
            addrs.push_back(off);
            std::memcpy(&af[mt][l * 16], lds.data() + off, 16);
          }
          cr_a.phase(addrs, 16);
        }
      for (int nt = 0; nt < 2; ++nt)
        for (int ph = 0; ph < 4; ++ph) {
          std::vector<int> addrs;
          for (int l = ph * 16; l < ph * 16 + 16; ++l) {
            const int off = A_STAGE + b_lds_offset(frag_chunk(l, s), wn * 64 + nt * 32 + frag_row(l), BN);
            addrs.push_back(off);
            std::memcpy(&bf[nt][l * 16], lds.data() + off, 16);
          }
          cr_b.phase(addrs, 16);
        }
      // D = X . Y with X = B^T fragment (rows i <- lane%32), Y = A^T fragment
      for (int mt = 0; mt < 2; ++mt)
        for (int nt = 0; nt < 2; ++nt) {
          int64_t D[32][32] = {};
          for (int i = 0; i < 32; ++i)
            for (int j = 0; j < 32; ++j)
              for (int g = 0; g < 2; ++g)
                for (int e = 0; e < EPC; ++e)
                  D[i][j] += elem(bf[nt], (size_t)(i + 32 * g) * 16 + e * sz, sz) *
                             elem(af[mt], (size_t)(j + 32 * g) * 16 + e * sz, sz);
          for (int l = 0; l < 64; ++l)
            for (int v = 0; v < 16; ++v) ACC(wave, mt, nt, l, v) += D[acc_i(l, v)][acc_j(l)];
        }
    }
  }
  // ---- epilogue coordinates vs the plain matmul
  std::vector<int> seen(BM * BN, 0);
  for (int wave = 0; wave < 4; ++wave) {
    const int wm = wave >> 1, wn = wave & 1;
    for (int mt = 0; mt < 2; ++mt)
      for (int nt = 0; nt < 2; ++nt)
        for (int l = 0; l < 64; ++l)
          for (int v = 0; v < 16; ++v) {
            const int m = wm * 64 + mt * 32 + acc_j(l);
            const int n = wn * 64 + nt * 32 + acc_i(l, v);
            seen[m * BN + n]++;
            int64_t ref = 0;
            for (int k = 0; k < KE; ++k)
              ref += elem(A, (size_t)m * kKTileBytes + k * sz, sz) * elem(B, ((size_t)k * BN + n) * sz, sz);
            CHECK(ACC(wave, mt, nt, l, v) == ref, "[%s] C[%d][%d] = %lld, want %lld\n", name, m, n,
                  (long long)ACC(wave, mt, nt, l, v), (long long)ref);
            if ((v & 3) != 0)
              CHECK(acc_i(l, v) == acc_i(l, v & ~3) + (v & 3), "[%s] staging run not contiguous\n", name);
          }
  }
  for (int i = 0; i < BM * BN; ++i) CHECK(seen[i] == 1, "[%s] output %d covered %d times\n", name, i, seen[i]);
  std::printf("[%s] lds bank-conflict ways: A write %d, B write %d, A read %d, B read %d\n", name,
              cw_a.worst, cw_b.worst, cr_a.worst, cr_b.worst);
  CHECK(cr_a.worst == 1 && cr_b.worst == 1, "[%s] fragment reads conflict\n", name);
  CHECK(cw_a.worst == 1 && cw_b.worst == 1, "[%s] stage writes conflict\n", name);
}

// DMA staging + ds_read_b64_tr_b16 operand path of the 16-bit kernels.
static void run_dma16() {
  const int KE = 64;  // k per k-tile
  std::vector<uint16_t> A(BM * KE), B(KE * BN);
  for (int m = 0; m < BM; ++m)
    for (int k = 0; k < KE; ++k) A[m * KE + k] = (uint16_t)((m * 7 + k * 3) % 13 + 1);
  for (int k = 0; k < KE; ++k)
    for (int n = 0; n < BN; ++n) B[k * BN + n] = (uint16_t)((k * 5 + n * 11) % 17 + 1);
  std::vector<uint8_t> sa(BM * 128), sb(KE * 256);
  std::vector<int> ca(sa.size(), 0), cb(sb.size(), 0);
  for (int w = 0; w < 8; ++w)  // the 8-wave layout: 2 blocks per wave and operand
    for (int j = 0; j < 2; ++j) {
      const int b = dma_block(w, j, 2);
      for (int i = 0; i < 64; ++i) {
        const int row = dma_a_row(b, i), c = dma_a_chunk(b, i);
        const int dst = b * 1024 + 16 * i;
        CHECK(a_lds_offset(row, c) == dst, "[dma16] A lane %d of block %d lands off-layout\n", i, b);
        std::memcpy(&sa[dst], &A[row * KE + c * 8], 16);
        for (int x = 0; x < 16; ++x) ca[dst + x]++;
        const int kr = dma_b_row(b, i), cc = dma_b_chunk(b, i);
        CHECK(btr_offset(kr, 8 * cc) == dst, "[dma16] B lane %d of block %d lands off-layout\n", i, b);
        std::memcpy(&sb[dst], &B[kr * BN + 8 * cc], 16);
        for (int x = 0; x < 16; ++x) cb[dst + x]++;
      }
    }
  for (size_t i = 0; i < ca.size(); ++i) CHECK(ca[i] == 1 && cb[i] == 1, "[dma16] LDS byte %zu coverage\n", i);
  Conflicts cr;
  for (int wave = 0; wave < 8; ++wave) {  // 2 x 4 waves, 32 columns each
    const int wn = wave & 3;
    for (int s = 0; s < 4; ++s)
      for (int nt = 0; nt < 1; ++nt) {
        const int nb = wn * 32 + nt * 32;
        uint16_t op[64][8];
        for (int h = 0; h < 2; ++h) {
          uint16_t src[64][4];
          std::vector<int> addrs;
          for (int l = 0; l < 64; ++l) {
            const int off = btr_offset(btr_k(s, h, l), btr_n(nb, l));
            std::memcpy(src[l], &sb[off], 8);
            addrs.push_back(off);
            if ((l & 31) == 31) {
              cr.phase(addrs, 8);
              addrs.clear();
            }
          }
          for (int l = 0; l < 64; ++l)  // the transpose, as measured on gfx950
            for (int r = 0; r < 4; ++r) op[l][4 * h + r] = src[16 * (l / 16) + 4 * r + (l % 16) / 4][(l % 16) % 4];
        }
        for (int l = 0; l < 64; ++l)
          for (int e = 0; e < 8; ++e) {
            const int k = 16 * s + 8 * (l >> 5) + e, n = nb + (l & 31);
            CHECK(op[l][e] == B[k * BN + n], "[dma16] B operand lane %d elem %d: got %d want %d\n", l, e, op[l][e],
                  B[k * BN + n]);
            // the A operand of the same lane covers the same k
            const int koff = frag_chunk(l, s) * 8;
            CHECK(koff + e == k, "[dma16] A/B k mismatch lane %d\n", l);
          }
      }
  }
  std::printf("[dma16] tr-read bank-conflict ways: %d\n", cr.worst);
  CHECK(cr.worst == 1, "[dma16] tr reads conflict\n");
}

// DMA staging + ds_read_b64_tr_b8 operand path of the fp8 kernels: the B
// operand bytes of every lane must be the column and k the A operand of the
// same lane pairs with.
static void run_dma8() {
  const int KE = 128;  // fp8 per k-tile
  std::vector<uint8_t> A(BM * KE), B(KE * BN);
  for (int m = 0; m < BM; ++m)
    for (int k = 0; k < KE; ++k) A[m * KE + k] = (uint8_t)((m * 7 + k * 3) % 251);
  for (int k = 0; k < KE; ++k)
    for (int n = 0; n < BN; ++n) B[k * BN + n] = (uint8_t)((k * 5 + n * 11) % 253);
  std::vector<uint8_t> sa(BM * 128), sb(KE * 128);
  std::vector<int> ca(sa.size(), 0), cb(sb.size(), 0);
  for (int w = 0; w < 8; ++w)
    for (int j = 0; j < 2; ++j) {
      const int b = dma_block(w, j, 2);
      for (int i = 0; i < 64; ++i) {
        const int row = dma_a_row(b, i), c = dma_a_chunk(b, i);
        const int dst = b * 1024 + 16 * i;
        CHECK(a_lds_offset(row, c) == dst, "[dma8] A lane %d of block %d lands off-layout\n", i, b);
        std::memcpy(&sa[dst], &A[row * KE + c * 16], 16);
        for (int x = 0; x < 16; ++x) ca[dst + x]++;
        const int kr = dma8_b_row(b, i), cc = dma8_b_chunk(b, i);
        CHECK(btr8_offset(kr, 16 * cc) == dst, "[dma8] B lane %d of block %d lands off-layout\n", i, b);
        std::memcpy(&sb[dst], &B[kr * BN + 16 * cc], 16);
        for (int x = 0; x < 16; ++x) cb[dst + x]++;
      }
    }
  for (size_t i = 0; i < ca.size(); ++i) CHECK(ca[i] == 1 && cb[i] == 1, "[dma8] LDS byte %zu coverage\n", i);
  Conflicts cr;
  for (int wave = 0; wave < 8; ++wave) {
    const int wm = wave >> 2, wn = wave & 3;
    const int nb = wn * 32;
    for (int s = 0; s < 2; ++s) {
      uint8_t bop[64][32], aop[2][64][32];
      for (int q = 0; q < 4; ++q) {
        uint8_t src[64][8];
        std::vector<int> addrs;
        for (int l = 0; l < 64; ++l) {
          const int off = btr8_offset(btr8_k(s, q, l), btr8_n(nb, l));
          std::memcpy(src[l], &sb[off], 8);
          addrs.push_back(off);
          if ((l & 31) == 31) {
            cr.phase(addrs, 8);
            addrs.clear();
          }
        }
        for (int l = 0; l < 64; ++l)  // the transpose, as measured on gfx950
          for (int r = 0; r < 8; ++r) bop[l][8 * q + r] = src[16 * (l / 16) + 2 * r + (l % 16) / 8][(l % 16) % 8];
      }
      for (int mt = 0; mt < 2; ++mt)
        for (int l = 0; l < 64; ++l)
          for (int hh = 0; hh < 2; ++hh) {
            const int row = wm * 64 + mt * 32 + (l & 31);
            const int chunk = 4 * s + 2 * (l >> 5) + hh;
            std::memcpy(&aop[mt][l][16 * hh], &sa[a_lds_offset(row, chunk)], 16);
          }
      for (int l = 0; l < 64; ++l)
        for (int e = 0; e < 32; ++e) {
          const int k = 64 * s + 32 * (l >> 5) + e, n = nb + (l & 31);
          CHECK(bop[l][e] == B[k * BN + n], "[dma8] B operand lane %d byte %d: got %d want %d\n", l, e, bop[l][e],
                B[k * BN + n]);
          for (int mt = 0; mt < 2; ++mt) {
            const int row = wm * 64 + mt * 32 + (l & 31);
            CHECK(aop[mt][l][e] == A[row * KE + k], "[dma8] A operand lane %d byte %d\n", l, e);
          }
        }
    }
  }
  std::printf("[dma8] tr8-read bank-conflict ways: %d\n", cr.worst);
  CHECK(cr.worst == 1, "[dma8] tr8 reads conflict\n");
}

// The 256x256 tile of wide_tile.hip: one 64-byte k-slab of A (256 rows,
// a64 layout) and B (two 128-column halves in the K-major layouts) staged by
// the 4 waves' direct-to-LDS loads (wave w: A blocks 4w..4w+3, B blocks
// 4(w%2)..+3 of half w/2), then every wave's fragment reads from the kernel's
// per-lane bases plus compile-time offsets, checked against the operands
// the MFMA must see (A row / B column of the lane, the same k on both).
static void run_wide(int sz) {
  const char* name = sz == 1 ? "wide8" : "wide16";
  const int KE = 64 / sz;       // k per slab
  const int EPC = 16 / sz;      // elements per chunk
  const int TM = 256, TN = 256;
  std::vector<uint8_t> A((size_t)TM * KE * sz), B((size_t)KE * TN * sz);
  for (size_t i = 0; i < A.size(); ++i) A[i] = (uint8_t)((i * 7 + 3) % 251);
  for (size_t i = 0; i < B.size(); ++i) B[i] = (uint8_t)((i * 13 + 5) % 241);
  auto a_at = [&](int m, int k, int byte) { return A[((size_t)m * KE + k) * sz + byte]; };
  auto b_at = [&](int k, int n, int byte) { return B[((size_t)k * TN + n) * sz + byte]; };
  const int ASTAGE = TM * 64, BHALF = 8192;
  std::vector<uint8_t> st(ASTAGE + 2 * BHALF);
  std::vector<int> cov(st.size(), 0);
  for (int w = 0; w < 4; ++w)
    for (int q = 0; q < 4; ++q)
      for (int i = 0; i < 64; ++i) {
        // A block 4w + q
        const int ba = 4 * w + q;
        const int row = dma64_a_row(ba, i), c = dma64_a_chunk(ba, i);
        CHECK(row == dma64_a_row(4 * w, i) + 16 * q && c == dma64_a_chunk(0, i),
              "[%s] A block step (wave %d q %d lane %d)\n", name, w, q, i);
        const int dst = ba * 1024 + 16 * i;
        CHECK(a64_lds_offset(row, c) == dst, "[%s] A lane %d of block %d lands off-layout\n", name, i, ba);
        for (int x = 0; x < 16; ++x) {
          st[dst + x] = A[(size_t)row * KE * sz + c * 16 + x];
          cov[dst + x]++;
        }
        // B block 4(w%2) + q of half w/2
        const int half = w >> 1, bb = 4 * (w & 1) + q;
        const int kr = sz == 1 ? dma8_b_row(bb, i) : dma_b_row(bb, i);
        const int cc = sz == 1 ? dma8_b_chunk(bb, i) : dma_b_chunk(bb, i);
        const int bdst = bb * 1024 + 16 * i;
        CHECK((sz == 1 ? btr8_offset(kr, 16 * cc) : btr_offset(kr, 8 * cc)) == bdst,
              "[%s] B lane %d of block %d lands off-layout\n", name, i, bb);
        CHECK(kr < KE, "[%s] B k-row %d past the slab\n", name, kr);
        const int n0 = 128 * half + EPC * cc;
        for (int x = 0; x < 16; ++x) {
          st[ASTAGE + half * BHALF + bdst + x] = b_at(kr, n0 + x / sz, x % sz);
          cov[ASTAGE + half * BHALF + bdst + x]++;
        }
      }
  for (size_t i = 0; i < cov.size(); ++i) CHECK(cov[i] == 1, "[%s] LDS byte %zu written %d times\n", name, i, cov[i]);
  Conflicts ca, cb;
  for (int wave = 0; wave < 4; ++wave) {
    const int wm = wave >> 1, wn = wave & 1;
    for (int s = 0; s < (sz == 1 ? 1 : 2); ++s)
      for (int mt = 0; mt < 4; ++mt)
        for (int nt = 0; nt < 4; ++nt) {
          // per lane: the operand bytes of MFMA (s, mt, nt), assembled as the kernel does
          std::vector<int> a_addr[2], b_addr[4];
          for (int l = 0; l < 64; ++l) {
            const int r = frag_row(l);
            const int row = wm * 128 + mt * 32 + r, col = wn * 128 + nt * 32 + r;
            uint8_t aop[32], bop[32];
            const int nbytes = sz == 1 ? 32 : 16;  // operand bytes per lane
            for (int hh = 0; hh < (sz == 1 ? 2 : 1); ++hh) {
              const int chunk = sz == 1 ? frag64_chunk8(l, hh) : frag64_chunk16(l, s);
              const int base = a64_lds_offset(wm * 128 + r, chunk);
              CHECK(a64_lds_offset(row, chunk) == base + mt * 2048, "[%s] A base + 2048*mt (lane %d)\n", name, l);
              std::memcpy(&aop[16 * hh], &st[base + mt * 2048], 16);
              a_addr[hh].push_back(base + mt * 2048);
            }
            for (int e = 0; e < nbytes; ++e) {
              const int kk = sz == 1 ? 32 * (l >> 5) + e : 16 * s + 8 * (l >> 5) + e / 2;
              CHECK(aop[e] == a_at(row, kk, e % sz), "[%s] A operand wave %d lane %d byte %d\n", name, wave, l, e);
            }
            (void)bop;
            (void)col;
          }
          // B: the transpose reads of n-subtile nt (lanes exchange within groups of 16)
          const int qn = sz == 1 ? 4 : 2;
          std::vector<std::vector<uint8_t>> src(qn, std::vector<uint8_t>(64 * 8));
          for (int q = 0; q < qn; ++q)
            for (int l = 0; l < 64; ++l) {
              const int base = wn * BHALF + (sz == 1 ? btr8_offset(btr8_k(0, 0, l), btr8_n(nt * 32, l))
                                                     : btr_offset(btr_k(0, 0, l), btr_n(nt * 32, l)));
              const int off = base + (sz == 1 ? 8 * q * 128 : (16 * s + 4 * q) * 256);
              const int ref = wn * BHALF + (sz == 1 ? btr8_offset(btr8_k(0, q, l), btr8_n(nt * 32, l))
                                                    : btr_offset(btr_k(s, q, l), btr_n(nt * 32, l)));
              CHECK(off == ref, "[%s] B base + k-rows (lane %d q %d)\n", name, l, q);
              std::memcpy(&src[q][8 * l], &st[ASTAGE + off], 8);
              b_addr[q].push_back(ASTAGE + off);
            }
          for (int l = 0; l < 64; ++l) {
            const int col = wn * 128 + nt * 32 + (l & 31);
            for (int q = 0; q < qn; ++q)
              for (int r = 0; r < (sz == 1 ? 8 : 4); ++r) {
                uint8_t got[2];
                int kk;
                if (sz == 1) {  // byte r of lane l: byte l%8 of lane 2r + (l%16)/8 of its group
                  got[0] = src[q][8 * (16 * (l / 16) + 2 * r + (l % 16) / 8) + (l % 16) % 8];
                  kk = 32 * (l >> 5) + 8 * q + r;
                } else {  // element r of lane l: element l%4 of lane 4r + (l%16)/4 of its group
                  const int sl = 16 * (l / 16) + 4 * r + (l % 16) / 4;
                  std::memcpy(got, &src[q][8 * sl + 2 * ((l % 16) % 4)], 2);
                  kk = 16 * s + 8 * (l >> 5) + 4 * q + r;
                }
                for (int byte = 0; byte < sz; ++byte)
                  CHECK(got[byte] == b_at(kk, col, byte), "[%s] B operand wave %d lane %d q %d r %d\n", name, wave,
                        l, q, r);
              }
          }
          for (int hh = 0; hh < 2; ++hh)
            for (size_t p0 = 0; p0 < a_addr[hh].size(); p0 += 16)
              ca.phase(std::vector<int>(a_addr[hh].begin() + p0, a_addr[hh].begin() + p0 + 16), 16);
          for (int q = 0; q < qn; ++q)
            for (size_t p0 = 0; p0 < 64; p0 += 32)
              cb.phase(std::vector<int>(b_addr[q].begin() + p0, b_addr[q].begin() + p0 + 32), 8);
        }
  }
  std::printf("[%s] A-read / B-read bank-conflict ways: %d / %d\n", name, ca.worst, cb.worst);
  CHECK(ca.worst == 1 && cb.worst == 1, "[%s] fragment reads conflict\n", name);
}


// The row-block kernel's pass-2 hand-off of a 128x128 tile of 16-bit outputs
// (chain_rows_kernel): compute wave (wm, wn) holds, per m-subtile mt, the
// 16 values of row l % 32 its lane l keeps in the accumulator layout
// (register v: column acc_i(l, v) of its 32 columns), packs them in pairs
// into 8 words, trades halves with lane l ^ 32 (v_permlane32_swap of words
// w and w + 2 leaves {x[0..31], y[0..31]} in x and {x[32..63], y[32..63]} in
// y) and writes two 16-byte runs at rows_out_offset(row, wn*4 + l/32 + 2h);
// I/O wave v reads row v*32 + 4q + l/16, chunk l % 16, and stores it at
// columns 8 (l % 16) .. +7.  Checks that every read finds its row's 8
// columns in order, that every 16-byte slot is written exactly once, and
// counts bank conflicts of both sides.
static void run_rows_out() {
  struct Word { int row, col0, col1; };
  std::vector<std::vector<Word>> lds(128 * 16);  // 16-byte slots: 4 words
  std::vector<int> writes(128 * 16, 0);
  Conflicts cw, cr;
  for (int wm = 0; wm < 2; ++wm)
    for (int wn = 0; wn < 4; ++wn)
      for (int mt = 0; mt < 2; ++mt) {
        Word pw[64][8];
        for (int l = 0; l < 64; ++l)
          for (int g = 0; g < 4; ++g)
            for (int h = 0; h < 2; ++h)
              pw[l][2 * g + h] = {wm * 64 + mt * 32 + l % 32, wn * 32 + acc_i(l, 4 * g + 2 * h),
                                  wn * 32 + acc_i(l, 4 * g + 2 * h + 1)};
        // q[i][0/1][l]: v_permlane32_swap(pw[a], pw[b]) for (a, b) = (0,2) (1,3) (4,6) (5,7)
        const int ab[4][2] = {{0, 2}, {1, 3}, {4, 6}, {5, 7}};
        Word q[4][2][64];
        for (int i = 0; i < 4; ++i)
          for (int l = 0; l < 64; ++l) {
            q[i][0][l] = l < 32 ? pw[l][ab[i][0]] : pw[l - 32][ab[i][1]];
            q[i][1][l] = l < 32 ? pw[l + 32][ab[i][0]] : pw[l][ab[i][1]];
          }
        for (int h = 0; h < 2; ++h) {
          std::vector<int> addrs;
          for (int l = 0; l < 64; ++l) {
            const int i0 = 2 * h, i1 = 2 * h + 1;
            const std::vector<Word> run = {q[i0][0][l], q[i1][0][l], q[i0][1][l], q[i1][1][l]};
            const int row = wm * 64 + mt * 32 + l % 32, chunk = wn * 4 + l / 32 + 2 * h;
            const int off = rows_out_offset(row, chunk);
            CHECK(off >= 0 && off % 16 == 0 && off < 128 * 256, "rows out: offset %d out of the stage\n", off);
            lds[off / 16] = run;
            writes[off / 16]++;
            addrs.push_back(off);
            if (addrs.size() == 16) {
              cw.phase(addrs, 16);
              addrs.clear();
            }
          }
        }
      }
  for (int sl = 0; sl < 128 * 16; ++sl) CHECK(writes[sl] == 1, "rows out: slot %d written %d times\n", sl, writes[sl]);
  for (int v = 0; v < 4; ++v)
    for (int qq = 0; qq < 8; ++qq) {
      std::vector<int> addrs;
      for (int l = 0; l < 64; ++l) {
        const int r = v * 32 + 4 * qq + l / 16, c = l % 16;
        const int off = rows_out_offset(r, c);
        const std::vector<Word>& run = lds[off / 16];
        CHECK(run.size() == 4, "rows out: empty slot read\n");
        for (int w = 0; w < (int)run.size(); ++w)
          CHECK(run[w].row == r && run[w].col0 == 8 * c + 2 * w && run[w].col1 == 8 * c + 2 * w + 1,
                "rows out: row %d chunk %d word %d holds row %d columns %d,%d\n", r, c, w, run[w].row,
                run[w].col0, run[w].col1);
        addrs.push_back(off);
        if (addrs.size() == 16) {
          cr.phase(addrs, 16);
          addrs.clear();
        }
      }
    }
  std::printf("rows out stage: bank conflict degree write %d read %d\n", cw.worst, cr.worst);
  CHECK(cw.worst == 1 && cr.worst == 1, "rows out: bank conflicts\n");
}

int main() {
  run_rows_out();
  run_dma16();
  run_dma8();
  run_wide(2);
  run_wide(1);
  run(2, "f16/bf16");
  run(1, "fp8");
  run(4, "f32");
  // The direct-to-LDS load plan keeps only block 0's offsets per lane and
  // steps to block b from there: A rows +8 per block with the chunk
  // recomputed as (lane % 8) ^ ((4b + lane / 16) % 8); B rows +4 (16-bit) or
  // +8 (fp8) per block with a block-independent chunk.  Checked for all 32
  // A blocks of a 256-row tile and the 16 B blocks.
  for (int b = 0; b < 32; ++b)
    for (int l = 0; l < 64; ++l) {
      CHECK(dma_a_row(b, l) == dma_a_row(0, l) + 8 * b, "dma_a_row step (b %d lane %d)\n", b, l);
      CHECK(dma_a_chunk(b, l) == ((l & 7) ^ ((4 * b + (l >> 4)) & 7)),
            "dma_a_chunk recomputation (b %d lane %d)\n", b, l);
      CHECK(dma_a_chunk(b, l) == (dma_a_chunk(b & ~1, l) ^ ((b & 1) ? 4 : 0)),
            "dma_a_chunk from the even block (b %d lane %d)\n", b, l);
      if (b < 16) {
        CHECK(dma_b_row(b, l) == dma_b_row(0, l) + 4 * b, "dma_b_row step (b %d lane %d)\n", b, l);
        CHECK(dma_b_chunk(b, l) == dma_b_chunk(0, l), "dma_b_chunk depends on the block\n");
        CHECK(dma8_b_row(b, l) == dma8_b_row(0, l) + 8 * b, "dma8_b_row step (b %d lane %d)\n", b, l);
        CHECK(dma8_b_chunk(b, l) == dma8_b_chunk(0, l), "dma8_b_chunk depends on the block\n");
      }
    }
  // Fragment reads as a per-lane base plus a compile-time offset (the kernel
  // keeps only the bases): A m-subtile mt adds 4096 bytes; 16-bit B k-step s,
  // half h add (16s + 4h) k-rows of 256 bytes; fp8 B k-step s, quad q add
  // (64s + 8q) k-rows of 128 bytes.  For every lane and wave position.
  for (int l = 0; l < 64; ++l)
    for (int wm = 0; wm < 4; ++wm)
      for (int mt = 0; mt < 2; ++mt)
        for (int s = 0; s < 4; ++s) {
          const int r = frag_row(l);
          CHECK(a_lds_offset(wm * 64 + mt * 32 + r, frag_chunk(l, s)) ==
                    a_lds_offset(wm * 64 + r, frag_chunk(l, s)) + mt * 4096,
                "A fragment offset not base + 4096*mt (lane %d)\n", l);
          const int c8 = 4 * (s >> 1) + 2 * (l >> 5) + (s & 1);
          CHECK(a_lds_offset(wm * 64 + mt * 32 + r, c8) == a_lds_offset(wm * 64 + r, c8) + mt * 4096,
                "fp8 A fragment offset not base + 4096*mt (lane %d)\n", l);
        }
  for (int l = 0; l < 64; ++l)
    for (int nw = 0; nw < 128; nw += 32)
      for (int s = 0; s < 4; ++s)
        for (int h = 0; h < 4; ++h) {
          if (h < 2)
            CHECK(btr_offset(btr_k(s, h, l), btr_n(nw, l)) ==
                      btr_offset(btr_k(0, 0, l), btr_n(nw, l)) + (16 * s + 4 * h) * 256,
                  "B fragment offset not base + k-rows (lane %d s %d h %d)\n", l, s, h);
          if (s < 2)
            CHECK(btr8_offset(btr8_k(s, h, l), btr8_n(nw, l)) ==
                      btr8_offset(btr8_k(0, 0, l), btr8_n(nw, l)) + (64 * s + 8 * h) * 128,
                  "fp8 B fragment offset not base + k-rows (lane %d s %d q %d)\n", l, s, h);
        }
  // tile_of_block: every (row block, column tile) exactly once
  for (auto rc : std::vector<std::pair<uint32_t, uint32_t>>{{16, 16}, {8, 256}, {1024, 16}, {2, 3}, {5, 7}, {3, 1}}) {
    const uint32_t R = rc.first, C = rc.second, G = R * C;
    std::set<std::pair<uint32_t, uint32_t>> seen2;
    for (uint32_t b = 0; b < G; ++b) {
      uint32_t r, c;
      tile_of_block(b, G, R, C, &r, &c);
      CHECK(r < R && c < C, "tile_of_block out of range\n");
      seen2.insert({r, c});
    }
    CHECK(seen2.size() == G, "tile_of_block not a bijection for %ux%u\n", R, C);
  }
  for (uint32_t G : {256u, 16384u, 8u, 100u, 7u, 2048u}) {
    std::set<uint32_t> s;
    for (uint32_t b = 0; b < G; ++b) s.insert(xcd_remap(b, G));
    CHECK(s.size() == G && *s.begin() == 0 && *s.rbegin() == G - 1, "xcd_remap not a bijection for %u\n", G);
    if (G % 8 == 0)
      for (uint32_t b = 0; b < G; ++b)
        CHECK(xcd_remap(b, G) / (G / 8) == b % 8, "xcd_remap: tile of block %u off its XCD\n", b);
  }
  if (g_fail) {
    std::printf("FAILED (%d)\n", g_fail);
    return 1;
  }
  std::printf("OK\n");
  return 0;
}
