// Fused DeepSeekMoE forward on one GPU: the whole layer (moe.py:77-109) as one
// C call that enqueues 4-6 kernels on the caller's stream and never waits.
//
//   [partial gate sums, dsk_moe_layer_forward only]  ->
//   route (+histogram, ranks)  ->  [scan + permute, one kernel, when T > 64]  ->
//   grouped GEMM1 + SwiGLU (A rows gathered from x through token_map)  ->
//   grouped GEMM2  ->  combine (ascending-expert fp32 sum + shared rows, one
//   bf16 rounding)
//
// The shared expert (intermediate 2*I) is run as n_shared_groups extra groups
// of width I appended after the routed experts: group E+j holds gate/up rows
// [j*I, (j+1)*I) of the shared gate/up weights and the matching column slice of
// the shared down weight. Every token routes to each of them with weight 1.0,
// so the shared expert costs no extra launch and rides the same tile scheduler.
// Slot layout: [0, T*K) routed (expert-major, ascending token), then group E+j
// rows [T*K + j*T, T*K + (j+1)*T) in token order.
#include "dsk_internal.hpp"
#include "route_token.hpp"

#include <algorithm>
#include <atomic>
#include <mutex>

namespace dsk {

struct FusedLayout {
  size_t hist, rank, idx, w, counts, offsets, token_map, slot_of, h, y, total;
};

static FusedLayout fused_layout(int T, int E, int K, int nsh, int H, int I) {
  FusedLayout L{};
  const int nblk = (T + 63) / 64;
  const size_t S = (size_t)T * K;
  const size_t Stot = S + (size_t)nsh * T;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align_up(bytes > 0 ? bytes : 1, 256);
    return o;
  };
  L.hist = take((size_t)nblk * E * 4);
  L.rank = take(S * 4);
  L.idx = take(S * 4);
  L.w = take(S * 4);
  L.counts = take((size_t)E * 4);
  L.offsets = take((size_t)(E + nsh + 1) * 4);
  L.token_map = take(Stot * 4);
  L.slot_of = take(S * 4);
  L.h = take(Stot * I * 2);
  L.y = take(Stot * H * 2);
  L.total = off;
  return L;
}

#ifndef DSK_GROUP_CHUNKS
#define DSK_GROUP_CHUNKS 1
#endif
// M tiles (of 256 rows) of a typical routed group, for dealing the large-group
// GEMMs' tiles to the XCDs one routed group at a time (GemmArgs::chunk_m_tiles),
// or 0 (chunks of the default size) where that deal would not be even: the E
// routed groups make E chunks and the always-on groups (T rows each) must fill
// whole chunks, the count of all chunks a multiple of the 8 XCDs. At T = 4096
// (E = 64, K = 6, 2 always-on groups): 2 M tiles, 64 + 16 chunks.
static int group_chunk_m_tiles(int T, int E, int K, int nsh) {
  if (!DSK_GROUP_CHUNKS || E % 8 != 0) return 0;
  const int64_t avg_rows = ((int64_t)T * K + E - 1) / E;
  const int mt = (int)std::max<int64_t>(1, (avg_rows + 255) / 256);
  const int64_t always_on = (int64_t)nsh * ((T + 255) / 256);  // their M tiles
  if (always_on % mt != 0 || (always_on / mt) % 8 != 0) return 0;
  return mt;
}

// Everything after the gate: route -> permutation -> GEMM1+SwiGLU -> GEMM2 ->
// combine. The router logits are n_parts partial-sum planes (part_stride
// floats apart) plus an optional bias, summed by the route kernel.
static int layer_after_gate(const float* logits, int n_parts, int64_t part_stride,
                            const float* bias, const uint16_t* x, const uint16_t* w1,
                            const uint16_t* w2, uint16_t* out, int T, int E, int K, int nsh,
                            int H, int I, int weight_layout, int32_t* topk_idx_out,
                            float* topk_w_out, int32_t* expert_offsets_out, char* ws,
                            const FusedLayout& L, void* const* stage_events, hipStream_t st) {
  int32_t* hist = reinterpret_cast<int32_t*>(ws + L.hist);
  int32_t* rank = reinterpret_cast<int32_t*>(ws + L.rank);
  int32_t* idx = topk_idx_out ? topk_idx_out : reinterpret_cast<int32_t*>(ws + L.idx);
  float* w = topk_w_out ? topk_w_out : reinterpret_cast<float*>(ws + L.w);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + L.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* token_map = reinterpret_cast<int32_t*>(ws + L.token_map);
  int32_t* slot_of = reinterpret_cast<int32_t*>(ws + L.slot_of);
  uint16_t* h = reinterpret_cast<uint16_t*>(ws + L.h);
  uint16_t* y = reinterpret_cast<uint16_t*>(ws + L.y);
  const int nblk = (T + 63) / 64;
  const int S = T * K;
  const int Stot = S + nsh * T;
  const int G = E + nsh;

  // optional instrumentation: hipEvent_t recorded at the stage boundaries
  auto mark = [&](int i) -> int {
    if (stage_events == nullptr || stage_events[i] == nullptr) return DSK_OK;
    if (hipEventRecord(reinterpret_cast<hipEvent_t>(stage_events[i]), st) != hipSuccess)
      return fail(DSK_ERR_LAUNCH, "moe_fused: hipEventRecord failed");
    return DSK_OK;
  };
  int rc;
  // Decode steps of at most kRouteInGemmTokens tokens: GEMM1's prologue does the
  // routing (every workgroup for itself, workgroup 0 storing the results), so
  // no route launch runs before it.
#ifndef DSK_ROUTE_IN_GEMM
#define DSK_ROUTE_IN_GEMM 1
#endif
  const bool route_in_gemm = DSK_ROUTE_IN_GEMM && nblk == 1 && T <= kRouteInGemmTokens &&
                             Stot <= kRouteInGemmSlots &&
                             n_parts >= 1 && n_parts <= kMaxGateParts;
  if (route_in_gemm) {
    // nothing to launch here
  } else if (nblk == 1) {
    rc = launch_route(logits, E, n_parts, part_stride, bias, T, E, K, idx, w, hist, rank,
                      counts, offsets, token_map, slot_of, nsh, st);
    if (rc) return rc;
  } else {
    rc = launch_route(logits, E, n_parts, part_stride, bias, T, E, K, idx, w, hist, rank,
                      nullptr, nullptr, nullptr, nullptr, 0, st);
    if (rc) return rc;
    rc = launch_scan_permute(hist, nblk, idx, T, K, E, rank, S, counts, offsets, token_map,
                             slot_of, nsh, st);
    if (rc) return rc;
  }

  if ((rc = mark(1))) return rc;

  GemmArgs g1{};
  g1.A = x; g1.lda = H;
  g1.a_rows = token_map; g1.a_rows_limit = T;
  g1.B = w1; g1.ldb = H; g1.b_group_stride = (int64_t)2 * I * H;
  g1.C = h; g1.ldc = I;
  g1.offsets = offsets; g1.G = G;
  g1.M = Stot; g1.N = I; g1.K = H;
  g1.offsets_sorted = 1;  // the route kernels' offsets never decrease
  g1.up_row_offset = I;
  g1.max_group_rows = T;  // a token routes to an expert at most once; shared groups hold T
  g1.b_tiled = weight_layout == DSK_LAYOUT_TILED;
  g1.chunk_m_tiles = group_chunk_m_tiles(T, E, K, nsh);
  if (route_in_gemm) {
    g1.rt_parts = logits;
    g1.rt_n_parts = n_parts;
    g1.rt_part_stride = part_stride;
    g1.rt_bias = bias;
    g1.rt_T = T;
    g1.rt_E = E;
    g1.rt_K = K;
    g1.rt_nsh = nsh;
    g1.rt_idx = idx;
    g1.rt_w = w;
    g1.rt_counts = counts;
    g1.rt_offsets = offsets;
    g1.rt_token_map = token_map;
    g1.rt_slot_of = slot_of;
  }
  if ((rc = run_gemm(g1, true, st))) return rc;
  if ((rc = mark(2))) return rc;

  GemmArgs g2{};
  g2.A = h; g2.lda = I;
  g2.B = w2; g2.ldb = I; g2.b_group_stride = (int64_t)H * I;
  g2.C = y; g2.ldc = H;
  g2.offsets = offsets; g2.G = G;
  g2.M = Stot; g2.N = H; g2.K = I;
  g2.offsets_sorted = 1;
  g2.max_group_rows = T;
  g2.b_tiled = weight_layout == DSK_LAYOUT_TILED;
  g2.chunk_m_tiles = g1.chunk_m_tiles;
  if ((rc = run_gemm(g2, false, st))) return rc;
  if ((rc = mark(3))) return rc;

  rc = launch_combine_slots(y, H, slot_of, w, T, K, H, S, nsh, out, H, st);
  if (rc) return rc;
  if ((rc = mark(4))) return rc;
  if (expert_offsets_out != nullptr) {
    if (hipMemcpyAsync(expert_offsets_out, offsets, (size_t)(E + 1) * 4,
                       hipMemcpyDeviceToDevice, st) != hipSuccess)
      return fail(DSK_ERR_LAUNCH, "moe_fused: offsets copy failed");
  }
  return DSK_OK;
}

static int check_layer_args(const char* who, int T, int E, int K, int nsh, int H, int I,
                            int weight_layout) {
  const std::string w(who);
  DSK_REQUIRE(E >= 1 && E <= DSK_MAX_EXPERTS, DSK_ERR_INVALID_ARG,
              w + ": num_experts must be in [1, 64]");
  DSK_REQUIRE(K >= 1 && K <= DSK_MAX_TOP_K && K <= E, DSK_ERR_INVALID_ARG,
              w + ": top_k must be in [1, min(6, num_experts)]");
  DSK_REQUIRE(nsh >= 0 && E + nsh <= 128, DSK_ERR_INVALID_ARG, w + ": too many shared groups");
  DSK_REQUIRE(T >= 0, DSK_ERR_INVALID_ARG, w + ": num_tokens < 0");
  DSK_REQUIRE(H > 0 && H % 64 == 0 && I > 0 && I % 64 == 0, DSK_ERR_INVALID_ARG,
              w + ": hidden and intermediate sizes must be multiples of 64");
  DSK_REQUIRE(weight_layout == DSK_LAYOUT_ROW_MAJOR || weight_layout == DSK_LAYOUT_TILED,
              DSK_ERR_INVALID_ARG, w + ": unknown weight_layout");
  return DSK_OK;
}

// Partial gate sums of the layer entry live after the fused layout.
static size_t layer_parts_offset(int T, int E, int K, int nsh, int H, int I) {
  return fused_layout(T, E, K, nsh, H, I).total;
}

}  // namespace dsk

using namespace dsk;

extern "C" size_t dsk_moe_fused_workspace_size(int num_tokens, int num_experts, int top_k,
                                               int n_shared_groups, int hidden,
                                               int intermediate) {
  if (num_tokens < 0 || num_experts <= 0 || top_k <= 0 || n_shared_groups < 0) return 0;
  return fused_layout(num_tokens, num_experts, top_k, n_shared_groups, hidden, intermediate)
      .total;
}

extern "C" int dsk_moe_fused_forward(const float* logits, const dsk_bf16* x, const dsk_bf16* w1,
                                     const dsk_bf16* w2, dsk_bf16* out, int num_tokens,
                                     int num_experts, int top_k, int n_shared_groups,
                                     int hidden, int intermediate, int weight_layout,
                                     int32_t* topk_idx_out,
                                     float* topk_w_out, int32_t* expert_offsets_out,
                                     void* workspace, size_t workspace_bytes,
                                     void* const* stage_events, void* stream) {
  const int T = num_tokens, E = num_experts, K = top_k, nsh = n_shared_groups;
  const int H = hidden, I = intermediate;
  int rc = check_layer_args("moe_fused", T, E, K, nsh, H, I, weight_layout);
  if (rc) return rc;
  if (T == 0) return DSK_OK;
  DSK_REQUIRE(logits && x && w1 && w2 && out, DSK_ERR_NULL_PTR, "moe_fused: NULL pointer");
  DSK_REQUIRE(aligned16(x) && aligned16(w1) && aligned16(w2) && aligned16(out),
              DSK_ERR_ALIGNMENT, "moe_fused: tensors must be 16-byte aligned");
  const FusedLayout L = fused_layout(T, E, K, nsh, H, I);
  DSK_REQUIRE(workspace != nullptr && workspace_bytes >= L.total && aligned16(workspace),
              DSK_ERR_WORKSPACE, "moe_fused: workspace too small");
  hipStream_t st = as_stream(stream);
  if (stage_events != nullptr && stage_events[0] != nullptr &&
      hipEventRecord(reinterpret_cast<hipEvent_t>(stage_events[0]), st) != hipSuccess)
    return fail(DSK_ERR_LAUNCH, "moe_fused: hipEventRecord failed");
  return layer_after_gate(logits, 1, 0, nullptr, x, w1, w2, out, T, E, K, nsh, H, I,
                          weight_layout, topk_idx_out, topk_w_out, expert_offsets_out,
                          static_cast<char*>(workspace), L, stage_events, st);
}

extern "C" size_t dsk_moe_layer_workspace_size(int num_tokens, int num_experts, int top_k,
                                               int n_shared_groups, int hidden,
                                               int intermediate) {
  if (num_tokens < 0 || num_experts <= 0 || top_k <= 0 || n_shared_groups < 0 || hidden < 16)
    return 0;
  const size_t parts = (size_t)gate_parts_count(num_tokens, num_experts, hidden) *
                       num_tokens * num_experts * sizeof(float);
  return layer_parts_offset(num_tokens, num_experts, top_k, n_shared_groups, hidden,
                            intermediate) + align_up(parts > 0 ? parts : 1, 256);
}

extern "C" int dsk_moe_layer_forward(const dsk_bf16* x, const dsk_bf16* gate_weight,
                                     const float* gate_bias, const dsk_bf16* w1,
                                     const dsk_bf16* w2, dsk_bf16* out, int num_tokens,
                                     int num_experts, int top_k, int n_shared_groups,
                                     int hidden, int intermediate, int weight_layout,
                                     int32_t* topk_idx_out, float* topk_w_out,
                                     int32_t* expert_offsets_out, void* workspace,
                                     size_t workspace_bytes, void* const* stage_events,
                                     void* stream) {
  const int T = num_tokens, E = num_experts, K = top_k, nsh = n_shared_groups;
  const int H = hidden, I = intermediate;
  int rc = check_layer_args("moe_layer", T, E, K, nsh, H, I, weight_layout);
  if (rc) return rc;
  DSK_REQUIRE(weight_layout == DSK_LAYOUT_ROW_MAJOR || E % 32 == 0, DSK_ERR_INVALID_ARG,
              "moe_layer: a tiled gate weight needs num_experts % 32 == 0");
  if (T == 0) return DSK_OK;
  DSK_REQUIRE(x && gate_weight && w1 && w2 && out, DSK_ERR_NULL_PTR, "moe_layer: NULL pointer");
  DSK_REQUIRE(aligned16(x) && aligned16(gate_weight) && aligned16(w1) && aligned16(w2) &&
                  aligned16(out),
              DSK_ERR_ALIGNMENT, "moe_layer: tensors must be 16-byte aligned");
  DSK_REQUIRE(workspace != nullptr && aligned16(workspace) &&
                  workspace_bytes >= dsk_moe_layer_workspace_size(T, E, K, nsh, H, I),
              DSK_ERR_WORKSPACE, "moe_layer: workspace too small");
  hipStream_t st = as_stream(stream);
  if (stage_events != nullptr && stage_events[0] != nullptr &&
      hipEventRecord(reinterpret_cast<hipEvent_t>(stage_events[0]), st) != hipSuccess)
    return fail(DSK_ERR_LAUNCH, "moe_layer: hipEventRecord failed");
  const FusedLayout L = fused_layout(T, E, K, nsh, H, I);
  char* ws = static_cast<char*>(workspace);
  float* parts = reinterpret_cast<float*>(ws + layer_parts_offset(T, E, K, nsh, H, I));
  // Partial sums over K slices in single-wave workgroups: at decode sizes they
  // spread the gate weight's loads over the CUs, and at T=4096 the full logits
  // (16 waves per 32 x 32 block reducing their K slices in the LDS, one plane)
  // measured slower: gate + route 29.0 against 31.4 us.
  const int n_parts = gate_parts_count(T, E, H);
  rc = launch_gate_parts(x, H, gate_weight, weight_layout == DSK_LAYOUT_TILED, parts, T, E, H,
                         n_parts, st);
  if (rc) return rc;
  return layer_after_gate(parts, n_parts, (int64_t)T * E, gate_bias, x, w1, w2, out, T, E, K,
                          nsh, H, I, weight_layout, topk_idx_out, topk_w_out,
                          expert_offsets_out, ws, L, stage_events, st);
}

// --------------------------------------------------- allocation-free entry --
// dsk_moe_layer_forward_noalloc runs the same kernels as dsk_moe_layer_forward
// with the workspace taken from `scratch`, a file-scope device array that the
// runtime places once per GPU when it loads this library there. The host
// never passes `scratch` itself to a kernel (in host code the name is only a
// stand-in for the symbol): the device address is resolved once per device
// with hipGetSymbolAddress and kept in g_scratch_addr.
namespace dsk {

constexpr size_t kNoAllocScratchBytes = DSK_NOALLOC_SCRATCH_BYTES;  // per GPU
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

static std::atomic<void*> g_scratch_addr[kNoAllocMaxDevices];
static std::mutex g_scratch_mu;

// In-flight tracking of each GPU's scratch: an event recorded on the stream of
// the last eager call after its kernels. A call on another stream of that GPU
// while the event is pending would share the scratch with a running layer, so
// it is refused (calls on one stream are ordered by the stream itself).
struct NoAllocInFlight {
  std::mutex mu;
  hipEvent_t done = nullptr;
  hipStream_t stream = nullptr;
  bool recorded = false;
};
static NoAllocInFlight g_inflight[kNoAllocMaxDevices];

// Device address of `scratch` on device `dev` (which must be current).
static int scratch_address(int dev, void** out) {
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return fail(DSK_ERR_LAUNCH, std::string("moe_layer_noalloc: hipGetSymbolAddress(scratch) "
                                                "failed: ") + hipGetErrorString(e));
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return DSK_OK;
}

}  // namespace dsk

extern "C" int dsk_moe_layer_forward_noalloc(const dsk_bf16* x, const dsk_bf16* gate_weight,
                                             const float* gate_bias, const dsk_bf16* w1,
                                             const dsk_bf16* w2, dsk_bf16* out,
                                             int num_tokens, int num_experts, int top_k,
                                             int n_shared_groups, int hidden,
                                             int intermediate, int weight_layout,
                                             int32_t* topk_idx_out, float* topk_w_out,
                                             int32_t* expert_offsets_out,
                                             void* const* stage_events, void* stream) {
  const int T = num_tokens, E = num_experts, K = top_k, nsh = n_shared_groups;
  const int H = hidden, I = intermediate;
  int rc = check_layer_args("moe_layer_noalloc", T, E, K, nsh, H, I, weight_layout);
  if (rc) return rc;
  const size_t need = dsk_moe_layer_workspace_size(T, E, K, nsh, H, I);
  DSK_REQUIRE(need <= kNoAllocScratchBytes, DSK_ERR_WORKSPACE,
              "moe_layer_noalloc: this layer needs " + std::to_string(need) +
                  " bytes of scratch, more than the " + std::to_string(kNoAllocScratchBytes) +
                  " bytes of the library's static per-GPU scratch; use dsk_moe_layer_forward "
                  "with a caller-allocated workspace");
  if (T == 0) return DSK_OK;
  int dev = -1;
  DSK_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kNoAllocMaxDevices,
              DSK_ERR_LAUNCH, "moe_layer_noalloc: no usable current device");
  hipStream_t st = as_stream(stream);
  if (st != nullptr) {
    int sdev = -1;
    DSK_REQUIRE(hipStreamGetDevice(st, &sdev) == hipSuccess && sdev == dev, DSK_ERR_INVALID_ARG,
                "moe_layer_noalloc: the stream must belong to the current device");
  }
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  DSK_REQUIRE(hipStreamIsCapturing(st, &capture) == hipSuccess, DSK_ERR_LAUNCH,
              "moe_layer_noalloc: hipStreamIsCapturing failed");
  const bool eager = capture == hipStreamCaptureStatusNone;
  NoAllocInFlight& fl = g_inflight[dev];
  std::lock_guard<std::mutex> lock(fl.mu);
  if (fl.done == nullptr) {
    // one-time set-up per device (the scratch address and the in-flight event)
    // is not capturable: the first call on a device must be an eager one
    DSK_REQUIRE(eager, DSK_ERR_INVALID_ARG,
                "moe_layer_noalloc: the first call on a device must not be under stream "
                "capture (it resolves the device's scratch); make one eager call first");
    // the event only tells whether the call's work has run (hipEventQuery); no
    // timing and no system-scope fence, whose cache writeback and invalidate
    // would cost each eager call ~2 us of GPU time
    DSK_REQUIRE(hipEventCreateWithFlags(&fl.done, hipEventDisableTiming |
                                                      hipEventDisableSystemFence) == hipSuccess,
                DSK_ERR_LAUNCH, "moe_layer_noalloc: hipEventCreate failed");
  }
  void* ws = nullptr;
  if ((rc = scratch_address(dev, &ws))) return rc;
  if (eager && fl.recorded && fl.stream != st) {
    const hipError_t q = hipEventQuery(fl.done);
    DSK_REQUIRE(q != hipErrorNotReady, DSK_ERR_INVALID_ARG,
                "moe_layer_noalloc: a call on another stream of this GPU is still running; "
                "the static scratch is shared by every call on a GPU, so calls on different "
                "streams must be serialised (or use dsk_moe_layer_forward with a workspace)");
    DSK_REQUIRE(q == hipSuccess, DSK_ERR_LAUNCH,
                std::string("moe_layer_noalloc: hipEventQuery failed: ") + hipGetErrorString(q));
  }
  rc = dsk_moe_layer_forward(x, gate_weight, gate_bias, w1, w2, out, T, E, K, nsh, H, I,
                             weight_layout, topk_idx_out, topk_w_out, expert_offsets_out, ws,
                             kNoAllocScratchBytes, stage_events, stream);
  if (rc) return rc;
  if (eager) {
    DSK_REQUIRE(hipEventRecord(fl.done, st) == hipSuccess, DSK_ERR_LAUNCH,
                "moe_layer_noalloc: hipEventRecord failed");
    fl.stream = st;
    fl.recorded = true;
  }
  return DSK_OK;
}
