// layout_check.cpp -- CPU replay of one workgroup of chain_tile_kernel.
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
// conflicts (64 banks x 4 bytes, 16 lanes per 128-bit access phase).
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

int main() {
  run_dma16();
  run_dma8();
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
