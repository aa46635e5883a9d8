// Host check of the GEMM tile decoders (pan2_amd/csrc/pm_tiles.hpp): every
// work item maps to a distinct in-range tile and every tile is covered, and
// the XCD block remap is a permutation.
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
  std::printf(bad ? "FAIL %d\n" : "OK\n", bad);
  return bad != 0;
}
