// Per-lane LDS byte addresses of every LDS access pattern of one mini-batch
// step of the MLP backward sweep (csrc/ttt_mlp_bwd.hip, mlp_bwd_kernel at
// bf16, F = 64, FF = 256, four waves: HT = 4 hidden tiles per wave, LayerNorm
// backwards split by rows), printed as JSON lines for tests/test_lds_banks.py;
// with --linear, those of the row-split Linear forward
// (csrc/ttt_linear_fwd_rows.hip at F = 64), relative to each shared array's
// start (one offset shared by all lanes of an access leaves its banks'
// conflicts unchanged).  An inactive lane prints as null.
//
// The shared matrices and the 16-bit staging take their addresses from
// csrc/ttt_lds_layout.h, the header the kernel itself builds them from; the
// lane-order exchange slots (LdsLane: base + 16 lane) and the LayerNorm
// parameter reads are restated from the kernel's expressions, named by
// the kernel's variables.
// Each pattern is printed once per wave with its width in bytes and the
// number of times one step of one wave issues it.
//
//   g++ -std=c++17 -O1 -I ttt-triton_amd/csrc tests/lds_banks_dump.cpp -o dump
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "ttt_lds_layout.h"

using namespace ttt::lds;

namespace {

constexpr int F = 64, FF = 256, NW = 4, FT = F / 16, HT = FF / (16 * NW);
// byte offsets of the shared arrays (MlpBwdShared in csrc/ttt_mlp_bwd.hip)
constexpr int W2T = 0, DW1T = 4 * F * FF, XCH = 8 * F * FF;
constexpr int PART = NW * FT * 1024, XCH_BYTES = (NW * FT + 3 * NW) * 1024;
constexpr int LNW = XCH + XCH_BYTES, LNB = LNW + 4 * F, LX = LNB + 4 * F;
constexpr int RS_DZ2 = 0, RS_DTGT = 4096, RS_DZ2T = 8192, RS_LCOL = 2048;

bool first = true;

// a pattern whose name says "write" or "put" is a store
void emit(const char* name, int width, int count, int wave, const std::vector<long>& a) {
  const bool store = std::strstr(name, "write") != nullptr || std::strstr(name, "put") != nullptr;
  std::printf("%s{\"name\": \"%s\", \"width\": %d, \"store\": %d, \"count\": %d, \"wave\": %d, \"addr\": [",
              first ? "" : "\n", name, width, store ? 1 : 0, count, wave);
  for (size_t i = 0; i < a.size(); ++i) {
    if (a[i] < 0)
      std::printf("%snull", i ? ", " : "");
    else
      std::printf("%s%ld", i ? ", " : "", a[i]);
  }
  std::printf("]}");
  first = false;
}

template <typename Fn> std::vector<long> lanes(Fn fn) {
  std::vector<long> a(64);
  for (int l = 0; l < 64; ++l) a[l] = fn(l >> 4, l & 15, l);
  return a;
}

// Layout checks, printed as one JSON line of failures: every map is a
// bijection onto its region, and the pieces a kernel adds up (lane part,
// block start, row step) give the element the access means.
int check() {
  std::vector<std::string> bad;
  auto fail = [&](const std::string& s) {
    if (bad.size() < 20) bad.push_back(s);
  };
  // fp32 block layout: matrices of the shapes the kernels hold
  const int shapes[][2] = {{64, 256}, {256, 64}, {64, 64}, {16, 64}, {32, 32}, {64, 128}, {128, 64}, {48, 16}};
  for (auto& sh : shapes) {
    const int rows = sh[0], cols = sh[1];
    std::vector<int> seen(rows * cols, 0);
    for (int r = 0; r < rows; ++r)
      for (int c = 0; c < cols; ++c) {
        const int e = mat_elem(cols, r, c);
        if (e < 0 || e >= rows * cols) {
          fail("mat_elem out of range");
          continue;
        }
        ++seen[e];
      }
    for (int e = 0; e < rows * cols; ++e)
      if (seen[e] != 1) fail("mat_elem not a bijection at " + std::to_string(rows) + "x" + std::to_string(cols));
    for (int cw = 0; cw < cols; cw += 16)
      for (int r0 = 0; r0 < rows; r0 += 16)
        for (int c0 = 0; c0 + cw < cols; c0 += 16)
          for (int g = 0; g < 4; ++g)
            for (int n = 0; n < 16; ++n) {
              const int k = col_base(cw) + blk_base(cols, r0, c0);
              for (int j = 0; j < 4; ++j)
                if (k + tile_lane(g, n, j) != mat_elem(cols, r0 + 4 * g + j, cw + c0 + n))
                  fail("tile access of the wrong element");
              for (int i = 0; i < 4; ++i)
                if (k + row_lane(g, n) + i != mat_elem(cols, r0 + n, cw + c0 + 4 * g + i))
                  fail("row-vector access of the wrong element");
            }
  }
  // 16-bit transposed frags: the element written for (row 4w + j, feature n
  // of tile lo) is the one frag lane 16 (n >> 2) + 4w + j of tile lo reads at
  // position n & 3; the slots of FT tiles fill tfrag16_bytes without overlap
  for (int ft = 1; ft <= 4; ++ft) {
    std::vector<int> seen(tfrag16_bytes(ft) / 8, 0);
    for (int c = 0; c < ft; ++c)
      for (int l = 0; l < 64; ++l) {
        const int s = tfrag16_slot(c, l);
        if (s < 0 || s >= (int)seen.size())
          fail("tfrag16 slot out of range");
        else
          ++seen[s];
      }
    for (int c = 0; c < ft; ++c)
      for (int w = 0; w < 4; ++w)
        for (int n = 0; n < 16; ++n)
          for (int j = 0; j < 4; ++j)
            if (tfrag16_put_slot(c, w, n) + j != tfrag16_slot(c, 16 * (n >> 2) + 4 * w + j))
              fail("tfrag16 element written to the wrong frag lane");
    int used = 0;
    for (int v : seen) {
      if (v > 1) fail("tfrag16 slots overlap");
      used += v;
    }
    if (used != 64 * ft) fail("tfrag16 slot count");
  }
  // 16-bit row tiles: slots of 4 tiles are a permutation of 0..255
  {
    std::vector<int> seen(256, 0);
    for (int c = 0; c < 4; ++c)
      for (int l = 0; l < 64; ++l) ++seen[crow16_slot(c, l)];
    for (int v : seen)
      if (v != 1) fail("crow16 not a permutation");
  }
  // 16-bit tile rows read back transposed: trow_put and grow_put are
  // permutations of a tile's 64 places, and lane l of the transposing read
  // supplies the place of row 4 (l >> 4) + ((l & 15) >> 2), group l & 3
  for (int o = 0; o < 4; ++o) {
    std::vector<int> a(64, 0), b(64, 0);
    for (int m = 0; m < 16; ++m)
      for (int g = 0; g < 4; ++g) {
        ++a[trow_put(m, g)];
        ++b[grow_put(o, m, g)];
      }
    for (int v : a)
      if (v != 1) fail("trow_put not a permutation");
    for (int v : b)
      if (v != 1) fail("grow_put not a permutation");
    for (int l = 0; l < 64; ++l) {
      const int m = 4 * (l >> 4) + ((l & 15) >> 2), g = l & 3;
      if (trow_get(l) != trow_put(m, g) || grow_get(o, l) != grow_put(o, m, g)) fail("transposing read place");
    }
  }
  std::printf("{\"failures\": [");
  for (size_t i = 0; i < bad.size(); ++i) std::printf("%s\"%s\"", i ? ", " : "", bad[i].c_str());
  std::printf("]}\n");
  return 0;
}

}  // namespace

// One mini-batch step of the row-split Linear forward at F = 64 (four feature
// tiles, two per pair p): waves R0, R1 (the chain), S (the state), O (the
// readout).  Arrays as LinRowsPar / LinRowsShared declare them: wf [16][64]
// 8-byte frags, b [64] fp32, gneg and geta [4][64] 8-byte tile rows, pp
// [2][2][64] 16-byte rows, mt [64] 8-byte frags, gx [2][4][16][20] fp32 (rows
// padded to 20), rc [2][16] fp32, xkt [3][4][64] 8-byte tile rows (one slot
// shown: the three are alike).
int linear_rows() {
  constexpr int LFT = 4, PP = 2, GXT = 16 * 20;
  auto tr = [&](int o) { return lanes([&](int, int, int l) { return 8L * (64 * o + grow_get(o, l)); }); };
  for (int w = 0; w < 2; ++w) {
    for (int o = 0; o < LFT; ++o) emit("G tile transposing read (R)", 8, 1, w, tr(o));
    for (int q = 0; q < PP; ++q) {
      emit("P partial read (R)", 16, 1, w, lanes([&](int, int, int l) { return 16L * (64 * (w * PP + q) + l); }));
      emit("b read (R)", 16, 1, w, lanes([&](int g, int n, int) { return 4L * (16 * (2 * q + (n >> 3)) + 4 * g); }));
    }
    emit("M frag read (R)", 8, 1, w, lanes([&](int, int, int l) { return 8L * l; }));
    for (int q = 0; q < PP; ++q)  // XK_s of token (n & 7) + 8w from the staging ring
      emit("XK row read (R)", 8, 1, w, lanes([&](int g, int n, int) {
             const int o = 2 * q + (n >> 3), t = (n & 7) + 8 * w;
             return 8L * (64 * o + grow_put(o, t, g));
           }));
    for (int q = 0; q < PP; ++q) {
      // -G and -(e o G): lane (g, n) holds token (n & 7) + 8w of tile 2q + (n >> 3)
      emit("G tile row put (R)", 8, 2, w, lanes([&](int g, int n, int) {
             const int o = 2 * q + (n >> 3), t = (n & 7) + 8 * w;
             return 8L * (64 * o + grow_put(o, t, g));
           }));
      emit("G, XH fp32 row write (R)", 16, 2, w, lanes([&](int g, int n, int) {
             const int o = 2 * q + (n >> 3), t = (n & 7) + 8 * w;
             return 4L * (o * GXT + 20 * t + 4 * g);
           }));
    }
    emit("row value write (R)", 4, 2, w,
         lanes([&](int g, int n, int) { return g == 0 && n < 8 ? 4L * ((n & 7) + 8 * w) : -1L; }));
  }
  for (int o = 0; o < LFT; ++o) emit("e G tile transposing read (S)", 8, 1, 2, tr(o));
  for (int i = 0; i < LFT; ++i)
    emit("XK tile transposing read (S)", 8, 1, 2, lanes([&](int, int, int l) { return 8L * (64 * i + grow_get(i, l)); }));
  for (int k = 0; k < LFT * LFT; ++k)
    emit("W frag write (S)", 8, 1, 2, lanes([&](int, int, int l) { return 8L * (64 * k + l); }));
  for (int o = 0; o < LFT; ++o)
    emit("P partial write (S)", 16, 1, 2, lanes([&](int g, int n, int) {
           return 16L * (64 * ((n >> 3) * PP + (o >> 1)) + 16 * g + (n & 7) + 8 * (o & 1));
         }));
  emit("M frag write (S)", 8, 1, 2, lanes([&](int, int, int l) { return 8L * l; }));
  for (int i = 0; i < LFT; ++i)
    emit("XK tile row put (S)", 8, 1, 2, lanes([&](int g, int n, int) { return 8L * (64 * i + grow_put(i, n, g)); }));
  for (int o = 0; o < LFT; ++o)
    for (int j = 0; j < 4; ++j)
      emit("G fp32 read (S)", 4, 1, 2, lanes([&](int g, int n, int) { return 4L * (o * GXT + 20 * (4 * g + j) + n); }));
  for (int o = 0; o < LFT; ++o)
    emit("b write (S)", 4, 1, 2, lanes([&](int g, int n, int) { return g == 0 ? 4L * (16 * o + n) : -1L; }));
  for (int k = 0; k < LFT * LFT; ++k)
    emit("W frag read (O)", 8, 1, 3, lanes([&](int, int, int l) { return 8L * (64 * k + l); }));
  for (int c = 0; c < LFT; ++c)  // XK_{s-1} operand frags (lane (g, n): row n) from the staging ring
    emit("XK frag read (O)", 8, 1, 3, lanes([&](int g, int n, int) { return 8L * (64 * c + grow_put(c, n, g)); }));
  for (int o = 0; o < LFT; ++o) {
    emit("b read (O)", 16, 1, 3, lanes([&](int g, int, int) { return 4L * (16 * o + 4 * g); }));
    emit("G tile transposing read (O)", 8, 1, 3, tr(o));
    for (int j = 0; j < 4; ++j)
      emit("XH fp32 read (O)", 4, 1, 3, lanes([&](int g, int n, int) { return 4L * (4 * GXT + o * GXT + 20 * (4 * g + j) + n); }));
  }
  for (int a = 0; a < 2; ++a)
    emit("row value read (O)", 16, 1, 3, lanes([&](int g, int, int) { return 4L * (16 * a + 4 * g); }));
  std::printf("\n");
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && std::string(argv[1]) == "--check") return check();
  if (argc > 1 && std::string(argv[1]) == "--linear") return linear_rows();
  for (int w = 0; w < NW; ++w) {
    const int hs = 16 * HT * w;
    // W2^T [F][FF] by columns: the wave's view W2t starts at column hs
    const long w2 = W2T + 4L * col_base(hs);
    // dW1^T [FF][F]: the wave's view dW1s starts at row hs
    const long dw1 = DW1T + 4L * hs * F;
    // one instance per block touched: (r0, c0) as the kernel's calls pass them
    for (int c = 0; c < FT; ++c)
      for (int o = 0; o < HT; ++o) {
        // w2_tile / w2_put: W2t.row4(16c, 16o); phase A reads and writes, P reads
        const long k2 = 4L * blk_base(FF, 16 * c, 16 * o);
        emit("W2^T row4 read (A, P)", 16, 2, w, lanes([&](int g, int n, int) { return w2 + k2 + 4L * row_lane(g, n); }));
        emit("W2^T row4 write (A)", 16, 1, w, lanes([&](int g, int n, int) { return w2 + k2 + 4L * row_lane(g, n); }));
        // w2T_frag: W2t.tile(16c, 16o), four rows j; B1 and B2b
        for (int j = 0; j < 4; ++j)
          emit("W2^T tile read (B1, B2b)", 4, 2, w, lanes([&](int g, int n, int) {
                 return w2 + k2 + 4L * tile_lane(g, n, j);
               }));
        // dw1_get / dw1_put: dW1s.row4(16o, 16q) with q = c; Q reads, the update reads and writes
        const long k1 = 4L * blk_base(F, 16 * o, 16 * c);
        emit("dW1^T row4 read (Q, update)", 16, 2, w, lanes([&](int g, int n, int) { return dw1 + k1 + 4L * row_lane(g, n); }));
        emit("dW1^T row4 write (update)", 16, 1, w, lanes([&](int g, int n, int) { return dw1 + k1 + 4L * row_lane(g, n); }));
        // dw1T_frag: dW1s.tile(16o, 16f), f = c; B2b
        for (int j = 0; j < 4; ++j)
          emit("dW1^T tile read (B2b)", 4, 1, w, lanes([&](int g, int n, int) {
                 return dw1 + k1 + 4L * tile_lane(g, n, j);
               }));
      }
    // exchange area, lane-order 16-byte slots (LdsLane, csrc/ttt_tile.h)
    const long xw = XCH + w * FT * 1024, xs16 = XCH + PART + w * 1024;
    for (int b = 0; b < 3; ++b)  // dN1, dN1^T, eta-row partials (xs16.put in N and P)
      emit("exchange put xs16 (N, P)", 16, 1, w, lanes([&](int, int, int l) { return xs16 + b * NW * 1024 + 16L * l; }));
    for (int c = 0; c < FT; ++c)  // dG2 partials (P) and dXK partials (B2b)
      emit("exchange put xw (P, B2b)", 16, 2, w, lanes([&](int, int, int l) { return xw + c * 1024 + 16L * l; }));
    for (int b = 0; b < 3 * NW; ++b)  // B2a: every wave's partials
      emit("exchange get xa (B2a)", 16, 1, w, lanes([&](int, int, int l) { return XCH + PART + b * 1024 + 16L * l; }));
    // row split: xr = 768 (l >> 4) + 256 w + 16 l (LdsLane xr)
    for (int v = 0; v < NW; ++v)
      emit("exchange get xr (B2a)", 16, 1, w,
           lanes([&](int lo, int, int l) { return XCH + 768L * lo + 256 * w + 16L * l + v * FT * 1024; }));
    for (int off : {RS_DZ2, RS_DTGT})
      emit("exchange put xr (LN2)", 16, 1, w,
           lanes([&](int lo, int, int l) { return XCH + 768L * lo + 256 * w + 16L * l + PART + off; }));
    for (int c = 0; c < FT; ++c)  // B2b: dZ2 rows
      emit("exchange get xa (B2b)", 16, 1, w,
           lanes([&](int, int, int l) { return XCH + PART + RS_DZ2 + c * 1024 + 16L * l; }));
    // B3: dtgt of the wave's tile
    emit("exchange get xa (B3)", 16, 1, w, lanes([&](int, int, int l) { return XCH + PART + RS_DTGT + w * 1024 + 16L * l; }));
    for (int v = 0; v < NW; ++v)  // B3: dXK partials of the wave's tile
      emit("exchange get xa (B3)", 16, 1, w, lanes([&](int, int, int l) { return XCH + (v * FT + w) * 1024 + 16L * l; }));
    // transposed dZ2 frags (LN2 writes four 2-byte elements, B2b reads)
    const long t = XCH + PART + RS_DZ2T;
    for (int j = 0; j < 4; ++j)
      emit("dZ2 frag element write (LN2)", 2, 1, w,
           lanes([&](int lo, int n, int) { return t + 8L * tfrag16_put_slot(lo, w, n) + 2 * (n & 3) + 8 * j; }));
    for (int c = 0; c < FT; ++c)
      emit("dZ2 frag read (B2b)", 8, 1, w, lanes([&](int, int, int l) { return t + 8L * tfrag16_slot(c, l); }));
    // readout LayerNorm rows (L): the wave's rows of feature l, then tiles and column sums
    emit("readout dZ2 row write (L)", 8, 1, w, lanes([&](int lo, int n, int) { return LX + 8L * crow16_slot(lo, 16 * w + n); }));
    for (int c = 0; c < FT; ++c)
      emit("readout dZ2 tile read (L)", 8, 1, w, lanes([&](int, int, int l) { return LX + 8L * crow16_slot(c, l); }));
    // column-sum partials: 4 (64 w + 4 n + lo) (the readout LayerNorm backward), read as 16 bytes at 16 (16 v + n)
    emit("readout column sum write (L)", 4, 1, w, lanes([&](int lo, int n, int) { return LX + RS_LCOL + 4L * (64 * w + 4 * n + lo); }));
    for (int v = 0; v < NW; ++v)
      emit("readout column sum read (L)", 16, 1, w, lanes([&](int, int n, int) { return LX + RS_LCOL + 16L * (16 * v + n); }));
    // LayerNorm parameters: src[16 o + n] (ln_param) and lnw[l], lnb[l]
    for (int o = 0; o < FT; ++o)  // lnw (L and LN2) and lnb (LN2): the same banks
      emit("LN parameter read [16o + n]", 4, 3, w, lanes([&](int, int n, int) { return LNW + 4L * (16 * o + n); }));
    emit("LN parameter read [l]", 4, 3, w, lanes([&](int, int, int l) { return LNW + 4L * l; }));
  }
  std::printf("\n");
  return 0;
}
