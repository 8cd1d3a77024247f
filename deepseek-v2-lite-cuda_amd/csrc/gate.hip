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

namespace dsk {

constexpr int kGateWaves = 16;
constexpr int kGateChunk = 8;  // K steps (of 16) loaded before the MFMAs

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
  const uint16_t* wrow = wg + (int64_t)e * H + 8 * h;
  const uint16_t* xrow = x + (int64_t)t * ld_x + 8 * h;
  const int ksteps = H / 16;
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
      wf[u] = *reinterpret_cast<const bf16x8_t*>(wrow + 16 * s);
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

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_moe_gate_logits(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* gate_weight,
                                   const float* bias, float* logits, int64_t ld_logits,
                                   int num_tokens, int num_experts, int hidden, void* stream) {
  const int T = num_tokens, E = num_experts, H = hidden;
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
  dim3 grid((T + 31) / 32, (E + 31) / 32);
  hipLaunchKernelGGL(gate_logits_kernel, grid, dim3(64 * kGateWaves), 0, as_stream(stream),
                     reinterpret_cast<const uint16_t*>(x), ld_x,
                     reinterpret_cast<const uint16_t*>(gate_weight), bias, logits, ld_logits, T,
                     E, H);
  return check_launch("gate_logits_kernel");
}
