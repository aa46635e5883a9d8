// Host check of the GEMM tile decoders (pan2_amd/csrc/pm_tiles.hpp): every
// work item maps to a distinct in-range tile and every tile is covered, the
// XCD block remap is a permutation, and the K-split rule and its item decode
// keep their invariants.
#include <cstdio>
#include <vector>

#include "../../pan2_amd/csrc/pm_tiles.hpp"

int main() {
  int bad = 0;
  for (int np = 1; np <= 130; ++np) {
    for (int nq = 1; nq <= 130; nq += (nq < 20 ? 1 : 7)) {
      for (int walk = 0; walk < 2; ++walk) {
        std::vector<int> seen(np * nq, 0);
        for (int lt = 0; lt < np * nq; ++lt) {
          int ti, tj;
          if (walk == 0) pm::full_tile(lt, np, nq, ti, tj);
          else pm::full_tile_cols(lt, np, nq, ti, tj);
          if (ti < 0 || ti >= np || tj < 0 || tj >= nq || seen[ti * nq + tj]++) {
            if (bad++ < 5) std::printf("full%s np=%d nq=%d lt=%d -> (%d,%d)\n", walk ? "_cols" : "", np, nq, lt, ti, tj);
          }
        }
      }
    }
    const int nt = np;
    std::vector<int> seen(nt * nt, 0);
    for (int lt = 0; lt < nt * (nt + 1) / 2; ++lt) {
      int ti, tj;
      pm::sym_tile(lt, nt, ti, tj);
      if (ti < 0 || tj >= nt || ti > tj || seen[ti * nt + tj]++) {
        if (bad++ < 5) std::printf("sym nt=%d lt=%d -> (%d,%d)\n", nt, lt, ti, tj);
      }
    }
  }
  for (int nb = 1; nb <= 2100; nb += (nb < 600 ? 1 : 37)) {
    std::vector<int> seen(nb, 0);
    for (int b = 0; b < nb; ++b) {
      const int t = pm::xcd_remap(b, nb);
      if (t < 0 || t >= nb || seen[t]++) {
        if (bad++ < 5) std::printf("xcd nb=%d b=%d -> %d\n", nb, b, t);
      }
    }
  }
  // K-split: the chunk count divides the unit count into chunks of at least
  // kSplitMinUnits units (a multiple of 4), stays within kMaxKSplit and the item
  // budget, is 1 below kSplitMinMp, is the largest such power of two, and
  // split_item covers every (tile, chunk) pair once.
  for (int mp = 256; mp <= 8192; mp += 256) {
    for (int tiles = 1; tiles <= 700; tiles += (tiles < 40 ? 1 : 13)) {
      for (int kt = 4; kt <= 512; kt += 4) {
        const int s = pm::k_split(mp, tiles, kt);
        const bool ok = s >= 1 && s <= pm::kMaxKSplit && (kt / s) % 4 == 0 && (s == 1 || kt / s >= pm::kSplitMinUnits) &&
                        (s == 1 || tiles * s <= pm::kSplitItems) && (mp >= pm::kSplitMinMp || s == 1) &&
                        (s & (s - 1)) == 0;
        // maximal: doubling would break a rule
        const bool maximal = 2 * s > pm::kMaxKSplit || (kt / 4) % (2 * s) != 0 || tiles * 2 * s > pm::kSplitItems ||
                             kt / (2 * s) < pm::kSplitMinUnits || mp < pm::kSplitMinMp;
        if (!ok || !maximal) {
          if (bad++ < 5) std::printf("k_split mp=%d tiles=%d kt=%d -> %d\n", mp, tiles, kt, s);
          continue;
        }
        if (s == 1 || tiles > 64) continue;
        std::vector<int> seen(tiles * s, 0);
        for (int lt = 0; lt < tiles * s; ++lt) {
          int tile, chunk;
          pm::split_item(lt, tiles, tile, chunk);
          if (tile < 0 || tile >= tiles || chunk < 0 || chunk >= s || seen[chunk * tiles + tile]++) {
            if (bad++ < 5) std::printf("split_item tiles=%d s=%d lt=%d -> (%d,%d)\n", tiles, s, lt, tile, chunk);
          }
        }
      }
    }
  }
  // the BASELINE shapes: 1024 x 4096 splits its gram (K = 4096) 4 ways and
  // keeps its K = 1024 products whole; 4096 and 5120 short sides never split
  {
    const int s1[3] = {pm::k_split(1024, 10, 64), pm::k_split(1024, 10, 16), pm::k_split(1024, 64, 16)};
    if (s1[0] != 4 || s1[1] != 1 || s1[2] != 1) {
      ++bad;
      std::printf("k_split 1024x4096: %d %d %d\n", s1[0], s1[1], s1[2]);
    }
    for (int m : {4096, 5120})
      for (int n : {5120, 20480, 30720}) {
        const int nt = m / 256, sym = nt * (nt + 1) / 2, full = nt * (n / 256);
        if (pm::k_split(m, sym, n / 64) != 1 || pm::k_split(m, sym, m / 64) != 1 || pm::k_split(m, full, m / 64) != 1) {
          ++bad;
          std::printf("k_split %dx%d splits\n", m, n);
        }
      }
  }
  std::printf(bad ? "FAIL %d\n" : "OK\n", bad);
  return bad != 0;
}
