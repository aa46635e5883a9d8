// Host check of the workspace layouts (pan2_amd/csrc/pm_tiles.hpp: ws_off,
// sm_x_off): each is a bijection onto [0, rows·ld); a panel of 256 rows starts
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

int main() {
  for (int rows : {256, 512, 768})
    for (int ld : {64, 128, 256, 320, 1024}) {
      check("panel", rows, ld, 256, [&](int r, int c) { return pm::ws_off(r, c, ld, true); });
      check("row-major", rows, ld, 0, [&](int r, int c) { return pm::ws_off(r, c, ld, false); });
    }
  for (int ld : {256, 512, 768, 4096})
    check("small X", 128, ld, 128, [&](int r, int c) { return pm::sm_x_off(r, c); });
  check("row-major, any ld", 300, 700, 0, [&](int r, int c) { return pm::ws_off(r, c, 700, false); });
  if (bad) {
    std::printf("FAILED (%d)\n", bad);
    return 1;
  }
  std::printf("OK\n");
  return 0;
}
