// Persistent-grid tile schedule of the grouped GEMM kernels, shared by the
// kernels (which decode their tiles from it) and the launchers (which size the
// grid from it). Plain integer arithmetic, also compiled by the host compiler
// alone for the CPU check of the schedule (tests/gemm_schedule_check.cpp).
//
// A launch enumerates T output tiles (group-major, then N tile, then M tile)
// and deals them to the 8 XCDs in chunks of `chunk` consecutive tiles (see
// sched_chunk): chunk c goes to XCD c % 8, so every XCD gets the same mix of
// tile sizes and the M tiles that share a weight tile stay on one XCD (one L2). Workgroup i
// runs on XCD i % 8 in slot i / 8; inside an XCD, the XCD's q-th tile goes to
// slot q % per_xcd in round q / per_xcd, so consecutive tiles run at the same
// time on neighbouring workgroups.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define DSK_HD __host__ __device__ __forceinline__
#else
#define DSK_HD inline
#endif

namespace dsk {

constexpr int kTileChunk = 16;  // tiles dealt to one XCD at a time, by default
constexpr int kXcds = 8;

// Tiles per chunk: kTileChunk, or, when the caller knows the M tiles of a
// typical group (chunk_m_tiles > 0), that many M tiles times the launch's nt N
// tiles, so that one typical group's tiles go to one XCD and its token rows
// are read into one L2. Measured on MI355X in the MoE layer at T = 4096
// (routed groups of two M tiles): GEMM1 (11 N tiles) with chunks of 22 against
// 16 ran 364.6 against 372.9 us and read 1.094 against 1.167 GB past the L2;
// GEMM2 (8 N tiles) with chunks of 22 ran 246.4 against 210.7 us.
DSK_HD int sched_chunk(int chunk_m_tiles, int nt) {
  return chunk_m_tiles > 0 ? chunk_m_tiles * nt : kTileChunk;
}

// Tiles held by XCD `xcd` out of `total`.
DSK_HD int sched_xcd_tiles(int total, int xcd, int chunk) {
  const int n_chunks = (total + chunk - 1) / chunk;
  if (xcd >= n_chunks) return 0;
  int t = ((n_chunks - xcd + kXcds - 1) / kXcds) * chunk;
  if ((n_chunks - 1) % kXcds == xcd) t -= n_chunks * chunk - total;  // partial last chunk
  return t;
}

// Tiles run by workgroup slot `slot` of an XCD that holds xcd_tiles tiles over
// per_xcd workgroups.
DSK_HD int sched_slot_tiles(int xcd_tiles, int slot, int per_xcd) {
  return slot >= xcd_tiles ? 0 : (xcd_tiles - slot + per_xcd - 1) / per_xcd;
}

// Global tile index of the t-th tile of (xcd, slot).
DSK_HD int sched_tile_index(int xcd, int slot, int t, int per_xcd, int chunk) {
  const int q = slot + t * per_xcd;
  return ((q / chunk) * kXcds + xcd) * chunk + q % chunk;
}

// Order of a group's tiles (mt M tiles x nt_count N tiles): N-major inside
// panels of kPanelM M tiles, so that a chunk of 16 consecutive tiles of a large
// group (the shared experts' 16 M tiles at T = 4096) covers 8 M tiles x 2 N
// tiles instead of 16 M tiles x 1 N tile, and fewer XCDs re-read each token
// row; groups of at most kPanelM M tiles (the routed experts) are one panel,
// all M tiles of an N tile side by side, sharing its weights. Measured on
// MI355X at T = 4096: GEMM1 reads 1.165 GB past the L2 per launch against
// 1.238 GB with one panel per group and 1.229 GB with panels of 16, in the same
// time (365.6 against 366.0 us; bitwise the same output).
constexpr int kPanelM = 8;
DSK_HD void sched_group_tile(int local, int mt, int nt_count, int* nt, int* mi) {
  if (mt <= kPanelM) {
    *nt = local / mt;
    *mi = local - *nt * mt;
    return;
  }
  const int p = local / (kPanelM * nt_count);
  const int r = local - p * kPanelM * nt_count;
  const int ps = mt - p * kPanelM < kPanelM ? mt - p * kPanelM : kPanelM;  // last panel may be short
  *nt = r / ps;
  *mi = p * kPanelM + (r - *nt * ps);
}

// The largest number of tiles any workgroup runs (nwg a multiple of 8).
DSK_HD int sched_max_tiles(int total, int nwg, int chunk) {
  int m = 0;
  for (int x = 0; x < kXcds; ++x) {
    const int t = sched_slot_tiles(sched_xcd_tiles(total, x, chunk), 0, nwg / kXcds);
    m = t > m ? t : m;
  }
  return m;
}

// Workgroups (a multiple of 8, at least 8) for a launch of at most `upper`
// tiles on `cus` compute units such that no workgroup runs more than
// row_tiles tiles (the gathered kernels stage each tile's row indices in an
// LDS table of row_tiles tiles). row_tiles <= 0: no limit.
inline int64_t sched_workgroups(int64_t upper, int64_t cus, int row_tiles, int chunk) {
  int64_t nwg = upper < cus ? upper : cus;
  nwg = (nwg + kXcds - 1) / kXcds * kXcds;
  if (nwg < kXcds) nwg = kXcds;
  if (row_tiles > 0) {
    const int64_t chunks = (upper + chunk - 1) / chunk;
    const int64_t xcd_max = (chunks + kXcds - 1) / kXcds * chunk;
    const int64_t per_xcd_min = (xcd_max + row_tiles - 1) / row_tiles;
    if (nwg < kXcds * per_xcd_min) nwg = kXcds * per_xcd_min;
  }
  return nwg;
}

}  // namespace dsk
