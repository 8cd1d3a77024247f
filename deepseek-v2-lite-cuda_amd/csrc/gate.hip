// Router (gate) logits on gfx950 matrix cores, fp32 out:
//
//   logits[t, e] = sum_k x[t, k] * wg[e, k]  (+ bias[e])
//
// The reference computes this as F.linear(x.float(), wg.float()) in fp32
// (moe_fused.py:131): the products of bf16 values are exact in fp32 and only
// the summation order differs here (fp32 MFMA accumulation over K slices,
// then a fixed-order sum of the slices), so the logits agree to fp32
// rounding. Fusing it removes the fp32 up-cast copies of x and of the gate
// weight and the torch GEMM launch, which at decode sizes cost more than the
// dot products.
//
// One workgroup per 32 tokens x 32 experts, 16 waves splitting K sixteen ways
// (a decode step has one or two workgroups, so the K split is what spreads
// the loads); each wave issues all loads of a chunk of 8 K steps before its
// MFMAs. The partial sums meet in LDS in a fixed order (waves 1..15 into
// wave 0), so the result is the same on every run.
#include "dsk_internal.hpp"
#include "gate_parts.hpp"

namespace dsk {

constexpr int kGateWaves = 16;

template <bool TILED>
__global__ __launch_bounds__(64 * kGateWaves) void gate_logits_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const uint16_t* __restrict__ wg,
    const float* __restrict__ bias, float* __restrict__ logits, int64_t ld_out, int T, int E,
    int H) {
  __shared__ floatx4_t red[kGateWaves - 1][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t0 = blockIdx.x * 32, e0 = blockIdx.y * 32;
  const int r32 = lane & 31, h = lane >> 5;
  // weights are MFMA operand A (output rows = experts), tokens operand B
  const int e = min(e0 + r32, E - 1);
  const int t = min(t0 + r32, T - 1);
  const int ksteps = H / 16;
  // row-major weight: row e, 16 elements per K step (each load touches 32
  // rows); fragment-tiled weight: fragment (expert block, K step) is 512
  // consecutive elements, lane-ordered (each load reads 1 KB contiguous)
  const uint16_t* wrow = TILED ? wg + ((int64_t)blockIdx.y * ksteps) * 512 + lane * 8
                               : wg + (int64_t)e * H + 8 * h;
  constexpr int kWStep = TILED ? 512 : 16;
  const uint16_t* xrow = x + (int64_t)t * ld_x + 8 * h;
  const int s_beg = wave * ksteps / kGateWaves;
  const int s_end = (wave + 1) * ksteps / kGateWaves;

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

  if (wave > 0) {
#pragma unroll
    for (int qg = 0; qg < 4; ++qg) {
      floatx4_t v;
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = acc[4 * qg + c];
      red[wave - 1][qg][lane] = v;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  const int tok = t0 + r32;
  if (tok >= T) return;
  float* orow = logits + (int64_t)tok * ld_out;
#pragma unroll
  for (int qg = 0; qg < 4; ++qg) {
    floatx4_t v;
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = acc[4 * qg + c];
    for (int w = 0; w < kGateWaves - 1; ++w) v += red[w][qg][lane];
    const int eb = e0 + 8 * qg + 4 * h;  // lane holds experts eb .. eb+3 of token tok
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (eb + c < E) orow[eb + c] = v[c] + (bias != nullptr ? bias[eb + c] : 0.f);
    }
  }
}

// Partial gate sums for the fused layer: one wave per (32 tokens, 32 experts,
// K slice), no LDS and no reduction here; the route kernel adds the n_parts
// planes in a fixed order while it loads the logits. Splitting K over many
// single-wave workgroups is what spreads the 256 KB of gate weight over the
// CUs at decode sizes, where there are only one or two token blocks.
template <bool TILED>
__global__ __launch_bounds__(64) void gate_parts_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const uint16_t* __restrict__ wg,
    float* __restrict__ parts, int T, int E, int H) {
  gate_parts_wave<TILED>(x, ld_x, wg, parts, T, E, H, blockIdx.x, blockIdx.y, blockIdx.z,
                         gridDim.z, threadIdx.x);
}

// K slices for the partial gate sums: more single-wave workgroups at decode
// sizes, one plane when the token blocks already cover the CUs. At most 4: the
// route kernel's loads of the planes sit on the decode step's critical path,
// and 4 planes (8 K steps x 4 per slice) measured 0.6-1.7 us faster per step
// than 16 at T = 1..64 (the gate itself is latency-bound either way).
int gate_parts_count(int T, int E, int H) {
  const int blocks = ((T + 31) / 32) * ((E + 31) / 32);
  int n = 512 / blocks;
  n = n < 1 ? 1 : (n > 4 ? 4 : n);
  return n > H / 16 ? H / 16 : n;
}

int launch_gate_logits(const uint16_t* x, int64_t ld_x, const uint16_t* wg, bool tiled,
                       const float* bias, float* logits, int64_t ld_out, int T, int E, int H,
                       hipStream_t st) {
  dim3 grid((T + 31) / 32, (E + 31) / 32);
  auto kern = tiled ? gate_logits_kernel<true> : gate_logits_kernel<false>;
  hipLaunchKernelGGL(kern, grid, dim3(64 * kGateWaves), 0, st, x, ld_x, wg, bias, logits, ld_out,
                     T, E, H);
  return check_launch("gate_logits_kernel");
}

int launch_gate_parts(const uint16_t* x, int64_t ld_x, const uint16_t* wg, bool tiled,
                      float* parts, int T, int E, int H, int n_parts, hipStream_t st) {
  dim3 grid((T + 31) / 32, (E + 31) / 32, n_parts);
  auto kern = tiled ? gate_parts_kernel<true> : gate_parts_kernel<false>;
  hipLaunchKernelGGL(kern, grid, dim3(64), 0, st, x, ld_x, wg, parts, T, E, H);
  return check_launch("gate_parts_kernel");
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_moe_gate_logits(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* gate_weight,
                                   const float* bias, float* logits, int64_t ld_logits,
                                   int num_tokens, int num_experts, int hidden,
                                   int weight_layout, void* stream) {
  const int T = num_tokens, E = num_experts, H = hidden;
  DSK_REQUIRE(weight_layout == DSK_LAYOUT_ROW_MAJOR ||
                  (weight_layout == DSK_LAYOUT_TILED && E % 32 == 0),
              DSK_ERR_INVALID_ARG,
              "moe_gate: weight_layout must be row-major, or tiled with num_experts % 32 == 0");
  DSK_REQUIRE(T >= 0 && E >= 1 && E <= DSK_MAX_EXPERTS, DSK_ERR_INVALID_ARG,
              "moe_gate: num_experts must be in [1, 64] and num_tokens >= 0");
  DSK_REQUIRE(H > 0 && H % 16 == 0, DSK_ERR_INVALID_ARG,
              "moe_gate: hidden size must be a positive multiple of 16");
  if (T == 0) return DSK_OK;
  DSK_REQUIRE(x && gate_weight && logits, DSK_ERR_NULL_PTR, "moe_gate: NULL pointer");
  DSK_REQUIRE(aligned16(x) && aligned16(gate_weight) && ld_x % 8 == 0, DSK_ERR_ALIGNMENT,
              "moe_gate: x and gate_weight rows must be 16-byte aligned");
  DSK_REQUIRE(ld_x >= H && ld_logits >= E, DSK_ERR_INVALID_ARG,
              "moe_gate: row stride smaller than the row");
  return launch_gate_logits(reinterpret_cast<const uint16_t*>(x), ld_x,
                            reinterpret_cast<const uint16_t*>(gate_weight),
                            weight_layout == DSK_LAYOUT_TILED, bias, logits, ld_logits, T, E, H,
                            as_stream(stream));
}
