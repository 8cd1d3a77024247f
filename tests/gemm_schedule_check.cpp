// CPU check of the grouped GEMM tile schedule (csrc/gemm_sched.hpp), built with
// the host compiler alone by tests/test_gemm_schedule.py. Prints "OK" or the
// first failing case and exits non-zero.
//   1. Every tile of a launch is run by exactly one workgroup, whatever the
//      tile count, grid size and chunk size.
//   2. The launcher's grid keeps every workgroup within the LDS row table,
//      for any row table size, group sizes, M and CU count, at the kernel's
//      real tile count (which the launcher bounds from above).
//   3. A group's tile order (panels of M tiles) maps its local tile indices
//      onto its (N tile, M tile) pairs one to one.
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <random>
#include <vector>

#include "../deepseek-v2-lite-cuda_amd/csrc/gemm_sched.hpp"

using namespace dsk;

static int fail(const char* what, long long a, long long b, long long c) {
  std::printf("FAIL %s (%lld, %lld, %lld)\n", what, a, b, c);
  return 1;
}

int main() {
  // 1. coverage: each tile exactly once
  std::vector<int> seen;
  for (int chunk : {1, 7, 11, 16, 22, 33, 64}) {
    for (int nwg = 8; nwg <= 512; nwg += (chunk == kTileChunk ? 8 : 24)) {
      for (int total = 0; total <= 3000; total += (total < 300 ? 1 : 37)) {
        seen.assign(total, 0);
        long long sum = 0;
        for (int x = 0; x < kXcds; ++x) {
          const int xt = sched_xcd_tiles(total, x, chunk);
          for (int slot = 0; slot < nwg / kXcds; ++slot) {
            const int n = sched_slot_tiles(xt, slot, nwg / kXcds);
            sum += n;
            for (int t = 0; t < n; ++t) {
              const int w = sched_tile_index(x, slot, t, nwg / kXcds, chunk);
              if (w < 0 || w >= total) return fail("tile index out of range", nwg, total, w);
              if (seen[w]++) return fail("tile run twice", nwg, total, w);
            }
          }
        }
        if (sum != total) return fail("tiles lost", nwg, total, sum);
      }
    }
  }
  // 2. the launcher's grid respects the row table at the real tile count
  std::mt19937 rng(1234);
  const int BM = 256;
  for (int cus : {8, 80, 256, 304}) {
    for (int rt = 1; rt <= 64; rt = rt < 8 ? rt + 1 : rt * 2) {
      for (int iter = 0; iter < 400; ++iter) {
        const int G = 1 + rng() % 128;
        const int nt = 1 + rng() % 24;
        const int M = rng() % 40000;
        // random group sizes summing to M (the kernel clamps offsets into [0, M])
        std::vector<int> cut(G - 1);
        for (int& c : cut) c = M ? rng() % (M + 1) : 0;
        std::sort(cut.begin(), cut.end());
        long long total = 0;
        int prev = 0;
        for (int g = 0; g < G; ++g) {
          const int end = g + 1 < G ? cut[g] : M;
          total += (long long)((end - prev + BM - 1) / BM) * nt;
          prev = end;
        }
        const long long upper = ((long long)(M + BM - 1) / BM + G) * nt;
        if (total > upper) return fail("tile count above the launcher's bound", M, G, total);
        const int chunk = sched_chunk((int)(rng() % 5), nt);  // 0: the default size
        const long long nwg = sched_workgroups(upper, cus, rt, chunk);
        if (nwg % kXcds || nwg < kXcds) return fail("grid not a multiple of 8", upper, cus, nwg);
        if (sched_max_tiles((int)total, (int)nwg, chunk) > rt)
          return fail("workgroup beyond the row table", total, nwg, rt);
        if (sched_max_tiles((int)upper, (int)nwg, chunk) > rt)
          return fail("bound beyond the row table", upper, nwg, rt);
      }
    }
  }
  // 3. the panel order inside a group is a bijection
  for (int mt = 1; mt <= 4 * kPanelM + 3; ++mt) {
    for (int nc = 1; nc <= 24; ++nc) {
      seen.assign(mt * nc, 0);
      for (int l = 0; l < mt * nc; ++l) {
        int nt = -1, mi = -1;
        sched_group_tile(l, mt, nc, &nt, &mi);
        if (nt < 0 || nt >= nc || mi < 0 || mi >= mt) return fail("group tile out of range", mt, nc, l);
        if (seen[mi * nc + nt]++) return fail("group tile run twice", mt, nc, l);
      }
    }
  }
  std::printf("OK\n");
  return 0;
}
