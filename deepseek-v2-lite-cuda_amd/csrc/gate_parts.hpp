// Partial router (gate) sums of one wave: the wave computes
//   parts[ks][t][e] = sum over K slice ks of n_parts of x[t, k] * wg[e, k]
// for the 32 tokens of block tb and the 32 experts of block eb, in fp32 on
// the matrix cores (bf16 products are exact in fp32). The route kernel adds
// the planes in a fixed order.
#pragma once

#include "dsk_common.hpp"

namespace dsk {

constexpr int kGateChunk = 8;  // K steps (of 16) loaded before the MFMAs

template <bool TILED>
__device__ __forceinline__ void gate_parts_wave(const uint16_t* __restrict__ x, int64_t ld_x,
                                                const uint16_t* __restrict__ wg,
                                                float* __restrict__ parts, int T, int E, int H,
                                                int tb, int eb, int ks, int n_parts, int lane) {
  const int t0 = tb * 32, e0 = eb * 32;
  const int r32 = lane & 31, h = lane >> 5;
  const int e = min(e0 + r32, E - 1);
  const int t = min(t0 + r32, T - 1);
  const int ksteps = H / 16;
  const int s_beg = ks * ksteps / n_parts;
  const int s_end = (ks + 1) * ksteps / n_parts;
  // row-major weight: row e, 16 elements per K step (each load touches 32
  // rows); fragment-tiled weight: fragment (expert block, K step) is 512
  // consecutive elements, lane-ordered (each load reads 1 KB contiguous)
  const uint16_t* wrow = TILED ? wg + ((int64_t)eb * ksteps) * 512 + lane * 8
                               : wg + (int64_t)e * H + 8 * h;
  constexpr int kWStep = TILED ? 512 : 16;
  const uint16_t* xrow = x + (int64_t)t * ld_x + 8 * h;
  floatx16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  for (int s0 = s_beg; s0 < s_end; s0 += kGateChunk) {
    bf16x8_t wf[kGateChunk], tf[kGateChunk];
#pragma unroll
    for (int u = 0; u < kGateChunk; ++u) {
      const int s = min(s0 + u, s_end - 1);  // past the slice: reload, unused
      wf[u] = *reinterpret_cast<const bf16x8_t*>(wrow + kWStep * s);
      tf[u] = *reinterpret_cast<const bf16x8_t*>(xrow + 16 * s);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kGateChunk; ++u) {
      if (s0 + u >= s_end) tf[u] = bf16x8_t{};  // a reloaded step adds zero
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[u], tf[u], acc, 0, 0, 0);
    }
  }
  const int tok = t0 + r32;
  if (tok >= T) return;
  float* orow = parts + ((int64_t)ks * T + tok) * E;
#pragma unroll
  for (int qg = 0; qg < 4; ++qg) {
    const int eb0 = e0 + 8 * qg + 4 * h;  // lane holds experts eb0 .. eb0+3 of token tok
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (eb0 + c < E) orow[eb0 + c] = acc[4 * qg + c];
  }
}

}  // namespace dsk
