// Softmax and top-K selection of one token on a 16-lane row, shared by the
// route kernel (moe_route.hip) and the small-group GEMM that routes a decode
// step in its prologue (gemm.hip), so both pick the same experts with the same
// weights, bit for bit.
#pragma once

#include <math.h>

#include "dsk_common.hpp"

namespace dsk {

constexpr int kMaxGateParts = 16;  // partial gate-sum planes a logit may be split into

// Token t on one 16-lane row: lane j of the row holds the logits of experts j,
// j+16, j+32, j+48, so every reduction is a 4-value local step plus a 16-lane
// DPP step. The logits are the sum of n_parts partial planes (K slices of the
// gate GEMM) in plane order, plus the optional per-expert bias. Lane j < K of
// the row gets the j-th pick (my_e, my_w: expert and softmax probability,
// descending, NaN as -inf, ties to the lower index). active: t < T (uniform
// over the row); wave_active: some row of the wave is active (the selection
// loop has wave-wide DPP steps).
__device__ __forceinline__ void route_token(const float* __restrict__ logits, int64_t ld,
                                            int n_parts, int64_t part_stride,
                                            const float* __restrict__ bias, int t, bool active,
                                            bool wave_active, int E, int K, int lane, int& my_e,
                                            float& my_w) {
  const int j = lane & 15;
  float xv[4];
  bool taken[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = j + 16 * q;
    taken[q] = e >= E;  // padding experts are never chosen
    float v = -INFINITY;
    if (active && e < E) {
      // all plane loads issued first, then summed in plane order
      const float* src = logits + (int64_t)t * ld + e;
      float pv[kMaxGateParts];
#pragma unroll
      for (int s = 0; s < kMaxGateParts; ++s) pv[s] = s < n_parts ? src[s * part_stride] : 0.f;
      v = pv[0];
#pragma unroll
      for (int s = 1; s < kMaxGateParts; ++s)
        if (s < n_parts) v += pv[s];
      if (bias != nullptr) v += bias[e];
    }
    xv[q] = v;
  }
  const float mx = row16_max(fmaxf(fmaxf(xv[0], xv[1]), fmaxf(xv[2], xv[3])));
  float ex[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) ex[q] = taken[q] ? 0.f : expf(xv[q] - mx);
  const float sum = row16_sum((ex[0] + ex[1]) + (ex[2] + ex[3]));
  my_e = -1;
  my_w = 0.f;
  for (int k = 0; k < K && wave_active; ++k) {
    // local best untaken (NaN counts as -inf; ties -> lower expert index)
    float bv = -INFINITY;
    int bi = 64;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float v = xv[q] == xv[q] ? xv[q] : -INFINITY;
      if (!taken[q] && (v > bv || bi == 64)) {
        bv = v;
        bi = j + 16 * q;
      }
    }
    const float m = row16_max(bv);
    const int win = row16_min((bi < 64 && bv == m) ? bi : 64);
    // probability of the winner, from its owner lane (j = win % 16)
    float pw = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (j + 16 * q == win) {
        taken[q] = true;
        pw = ex[q] / sum;
      }
    pw = __shfl(pw, (lane & ~15) + (win & 15), 64);
    if (j == k) {
      my_e = win;
      my_w = pw;
    }
  }
}


// Routing of one chunk of kRouteChunk tokens by one workgroup, four tokens per
// wave (one per 16-lane row; the workgroup needs a wave per four tokens of the
// chunk). Writes topk idx / weights, the chunk histogram, and (optionally) each
// (token, k)'s rank inside its chunk. With a single chunk (T <= 64) it also
// finishes the job that the scan and permutation kernels do for larger T:
// counts, offsets (including the rows of the always-on groups appended after
// the routed ones), token_map and slot_of.
constexpr int kRouteChunk = 64;  // tokens per routing workgroup (= mask width)

__device__ __forceinline__ void route_chunk_body(
    const float* __restrict__ logits, int64_t ld, int n_parts, int64_t part_stride,
    const float* __restrict__ bias, int T, int E, int K,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    int32_t* __restrict__ blk_hist, int32_t* __restrict__ local_rank,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ token_map, int32_t* __restrict__ slot_of,
    int n_extra_groups, int chunk, bool single_chunk) {
  __shared__ unsigned long long s_mask[64];
  __shared__ int s_off[64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (tid < 64) s_mask[tid] = 0ull;
  __syncthreads();

  const int t0 = chunk * kRouteChunk;
  // Four tokens per wave at once: the 16 lanes of row g hold token
  // tl = 4 * wave + g (route_token).
  const int g = lane >> 4, j = lane & 15;
  const int tl = 4 * wave + g;
  const int t = t0 + tl;
  const bool active = t < T;  // uniform over the 16-lane row
  // waves whose four rows are all past T skip the selection
  const bool wave_active = t0 + 4 * wave < T;
  int my_e;
  float my_w;
  route_token(logits, ld, n_parts, part_stride, bias, t, active, wave_active, E, K, lane, my_e,
              my_w);
  if (active && j < K) {
    topk_idx[(int64_t)t * K + j] = my_e;
    topk_w[(int64_t)t * K + j] = my_w;
    atomicOr(&s_mask[my_e], 1ull << tl);
  } else {
    my_e = -1;
  }
  __syncthreads();

  if (blk_hist != nullptr && tid < E)
    blk_hist[(int64_t)chunk * E + tid] = __popcll(s_mask[tid]);

  const int rank = my_e >= 0 ? __popcll(s_mask[my_e] & ((1ull << tl) - 1ull)) : -1;
  if (local_rank != nullptr && my_e >= 0) local_rank[(int64_t)t * K + j] = rank;

  if (single_chunk && offsets != nullptr) {
    if (wave == 0) {
      const int c = lane < E ? __popcll(s_mask[lane]) : 0;
      const int inc = wave_inclusive_scan(c);
      if (lane < E) {
        offsets[lane] = inc - c;
        s_off[lane] = inc - c;
        if (counts != nullptr) counts[lane] = c;
      }
      if (lane == 63) {
        offsets[E] = inc;
        for (int x = 1; x <= n_extra_groups; ++x) offsets[E + x] = inc + x * T;
      }
    }
    if (token_map != nullptr) {
      __syncthreads();
      if (my_e >= 0) {
        const int slot = s_off[my_e] + rank;
        token_map[slot] = t;
        if (slot_of != nullptr) slot_of[(int64_t)t * K + j] = slot;
      }
      // rows of the always-on groups: group E+x row t is token t
      const int S = T * K;
      for (int r = tid; r < n_extra_groups * T; r += blockDim.x) token_map[S + r] = r % T;
    }
  }
}

}  // namespace dsk
