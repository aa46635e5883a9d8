// Host check of the workspace layouts (pan2_amd/csrc/pm_tiles.hpp: ws_off,
// sm_x_off, and the small apply's LDS unit xt_off): each is a bijection onto [0, rows·ld); a panel of 256 rows starts
// where it does row-major; every 64-column unit of a panel is one contiguous,
// row-ordered block (32 KiB, or 16 KiB for a small X); aligned runs of 4 and 8
// elements are contiguous; the row-major form is r·ld + c.
#include <cstdio>
#include <vector>

#include "../../pan2_amd/csrc/pm_tiles.hpp"

static int bad = 0;
static void fail(const char* what, int r, int c, long long ld) {
  if (bad++ < 10) std::printf("%s: r=%d c=%d ld=%lld\n", what, r, c, ld);
}

// prows: rows per panel (units of 64 columns inside), or 0 for row-major
template <class F>
static void check(const char* name, int rows, int ld, int prows, F off) {
  std::vector<char> seen((size_t)rows * ld, 0);
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < ld; ++c) {
      const long long o = off(r, c);
      if (o < 0 || o >= (long long)rows * ld || seen[o]++) fail(name, r, c, ld);
      if (c % 8 == 0)
        for (int e = 1; e < 8; ++e)
          if (off(r, c + e) != o + e) fail("run of 8", r, c, ld);
      if (prows == 0) {
        if (o != (long long)r * ld + c) fail("row-major form", r, c, ld);
        continue;
      }
      // unit (r / prows, c / 64) starts at its panel's row-major base plus (c/64) units
      const long long unit0 = (long long)(r / prows) * prows * ld + (long long)(c / 64) * prows * 64;
      if (o != unit0 + (r % prows) * 64 + c % 64) fail("unit block", r, c, ld);
    }
  for (int p = 0; prows && p < rows; p += prows)
    if (off(p, 0) != (long long)p * ld) fail("panel base", p, 0, ld);
}

// The apply's X unit in LDS (xt_off, xt_copy_src): a bijection of the 16 KiB
// unit that keeps 8-byte runs whole; the 16 copies (64 lanes of 16 bytes,
// written in order) put every (row, column) where xt_off reads it, and each
// copy reads 8 whole rows; and every 16-lane group of the apply's reads falls
// in 16 distinct bank pairs of a 64-bank, 4-byte LDS (all lanes read 8 bytes).
static void check_apply_unit() {
  std::vector<int> seen(128 * 128, 0);
  for (int k = 0; k < 128; ++k)
    for (int n = 0; n < 64; ++n) {
      const int o = pm::xt_off(k, n);
      if (o < 0 || o + 2 > 128 * 128 || o % 2 || seen[o]++) fail("xt_off bijection", k, n, 64);
      if (n % 4 == 0 && (o % 8 || pm::xt_off(k, n + 3) != o + 6)) fail("xt_off run of 4", k, n, 64);
    }
  for (int q = 0; q < 16; ++q)
    for (int lane = 0; lane < 64; ++lane) {
      const int src = pm::xt_copy_src(q, lane), dst = q * 1024 + lane * 16;
      const int k = src / 128, c = (src % 128) / 16;
      if (src % 16 || k / 8 != q) fail("copy reads its own 8 rows", q, lane, 0);
      for (int e = 0; e < 8; ++e)
        if (pm::xt_off(k, 8 * c + e) != dst + 2 * e) fail("copy lands where xt_off reads", q, lane, e);
    }
  // groups: 16 lanes each, with the row and column they read
  auto groups_ok = [&](const char* what, auto rowcol) {
    for (int v = 0; v < 64; ++v)
      for (int g = 0; g < 4; ++g) {
        std::vector<int> bank(64, 0);
        for (int i = 0; i < 16; ++i) {
          int k, n;
          rowcol(v, g, i, k, n);
          const int o = pm::xt_off(k, n);
          for (int d = 0; d < 2; ++d)
            if (bank[(o / 4 + d) % 64]++) fail(what, v, g, i);
        }
      }
  };
  // transposed fragment (ds_read_b64_tr_b16): lane 16g + i reads row k0 + 4h + i/4, columns n0 + 4(i%4)
  groups_ok("bank spread, transposed read", [](int v, int g, int i, int& k, int& n) {
    const int s = v % 4, h = (v / 4) % 2, n0 = 16 * ((v / 8) % 4);
    k = 32 * s + 8 * g + 4 * h + i / 4;
    n = n0 + 4 * (i % 4);
  });
  // a·X quad: lane 16g + i reads row 64wr + 16m + 4g + i%4, columns (16wc + i) & ~3
  groups_ok("bank spread, a.X quad read", [](int v, int g, int i, int& k, int& n) {
    const int wr = v % 2, m = (v / 2) % 4, wc = (v / 8) % 4;
    k = 64 * wr + 16 * m + 4 * g + i % 4;
    n = (16 * wc + i) & ~3;
  });
  // wide FINAL: lane 16g + i reads row 64wr + 16m + i, columns 16wc + 4g
  groups_ok("bank spread, wide read", [](int v, int g, int i, int& k, int& n) {
    const int wr = v % 2, m = (v / 2) % 4, wc = (v / 8) % 4;
    k = 64 * wr + 16 * m + i;
    n = 16 * wc + 4 * g;
  });
}

int main() {
  for (int rows : {256, 512, 768})
    for (int ld : {64, 128, 256, 320, 1024}) {
      check("panel", rows, ld, 256, [&](int r, int c) { return pm::ws_off(r, c, ld, true); });
      check("row-major", rows, ld, 0, [&](int r, int c) { return pm::ws_off(r, c, ld, false); });
    }
  for (int ld : {256, 512, 768, 4096})
    check("small X", 128, ld, 128, [&](int r, int c) { return pm::sm_x_off(r, c); });
  check("row-major, any ld", 300, 700, 0, [&](int r, int c) { return pm::ws_off(r, c, 700, false); });
  check_apply_unit();
  if (bad) {
    std::printf("FAILED (%d)\n", bad);
    return 1;
  }
  std::printf("OK\n");
  return 0;
}
