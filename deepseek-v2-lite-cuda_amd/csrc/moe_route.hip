// MoE routing, expert histogram + scan, stable permutation, dispatch gather,
// deterministic combine and SwiGLU for gfx950 (wave64).
//
// Routing semantics follow the reference gate (src/reference/moe.py:33-43):
// fp32 softmax over all experts, top-K without renormalisation. Selection is
// done on the fp32 logits (softmax is monotone) with ties going to the lower
// expert index, and the K winners are emitted in descending order, as the
// reference kernel does (src/kernels/moe/routing.cu:139-198).
//
// The permutation is the oracle's iteration order (moe.py:90-103): expert-major,
// ascending token index inside an expert. It is computed from per-chunk 64-bit
// token masks (one bit per token of a 64-token chunk, one mask per expert):
//   rank inside chunk = popcount(mask[e] & bits below the token),
//   slot = offsets[e] + chunk_base[chunk][e] + rank,
// which is deterministic and needs no atomics beyond LDS bit-ors.
#include "dsk_internal.hpp"
#include "route_token.hpp"

#include <algorithm>
#include <climits>

namespace dsk {

constexpr int kChunk = kRouteChunk;   // tokens per routing workgroup (= mask width)
constexpr int kRouteThreads = 1024;   // 16 waves, 4 tokens each
constexpr int kRouteWaves = kRouteThreads / kWave;
constexpr int kTokPerWave = kChunk / kRouteWaves;  // one per 16-lane row
constexpr int kRankThreads = 256;

// ------------------------------------------------------------------ route --
// One workgroup per chunk of 64 tokens (route_chunk_body, route_token.hpp).
__global__ __launch_bounds__(kRouteThreads) void route_kernel(
    const float* __restrict__ logits, int64_t ld, int n_parts, int64_t part_stride,
    const float* __restrict__ bias, int T, int E, int K,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    int32_t* __restrict__ blk_hist, int32_t* __restrict__ local_rank,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ token_map, int32_t* __restrict__ slot_of,
    int n_extra_groups) {
  route_chunk_body(logits, ld, n_parts, part_stride, bias, T, E, K, topk_idx, topk_w, blk_hist,
                   local_rank, counts, offsets, token_map, slot_of, n_extra_groups, blockIdx.x,
                   gridDim.x == 1);
}

// ------------------------------------------------------------------- rank --
// Chunk histogram + in-chunk stable rank from a given topk_idx (the dispatch
// op receives indices, not logits). Entries with an out-of-range expert, or a
// repeat of an expert earlier in the same row, get rank -1 and are skipped.
__global__ __launch_bounds__(kRankThreads) void rank_kernel(
    const int32_t* __restrict__ idx, int T, int K, int E,
    int32_t* __restrict__ blk_hist, int32_t* __restrict__ local_rank) {
  __shared__ unsigned long long s_mask[64];
  const int tid = threadIdx.x;
  if (tid < 64) s_mask[tid] = 0ull;
  __syncthreads();
  const int t0 = blockIdx.x * kChunk;
  const int npairs = kChunk * K;
  for (int p = tid; p < npairs; p += kRankThreads) {
    const int tl = p / K, k = p - tl * K;
    const int t = t0 + tl;
    if (t >= T) continue;
    const int e = idx[(int64_t)t * K + k];
    bool ok = e >= 0 && e < E;
    for (int j = 0; j < k && ok; ++j) ok = idx[(int64_t)t * K + j] != e;
    if (ok) atomicOr(&s_mask[e], 1ull << tl);
  }
  __syncthreads();
  if (tid < E) blk_hist[(int64_t)blockIdx.x * E + tid] = __popcll(s_mask[tid]);
  for (int p = tid; p < npairs; p += kRankThreads) {
    const int tl = p / K, k = p - tl * K;
    const int t = t0 + tl;
    if (t >= T) continue;
    const int e = idx[(int64_t)t * K + k];
    bool ok = e >= 0 && e < E;
    for (int j = 0; j < k && ok; ++j) ok = idx[(int64_t)t * K + j] != e;
    local_rank[(int64_t)t * K + k] =
        ok ? __popcll(s_mask[e] & ((1ull << tl) - 1ull)) : -1;
  }
}

// ------------------------------------------------------------------- scan --
// Single workgroup of 16 waves; lane = expert. Reduces the chunk histograms
// into counts, the exclusive scan into offsets (plus the always-on groups),
// and the per-chunk exclusive bases of every expert.
constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(kScanThreads) void scan_kernel(
    const int32_t* __restrict__ hist, int nblk, int E,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ blk_base, int n_extra_groups, int extra_rows) {
  __shared__ int s_part[16][64];
  __shared__ int s_tot[64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int seg = (nblk + 15) / 16;
  const int b0 = min(wave * seg, nblk), b1 = min(b0 + seg, nblk);
  int part = 0;
  if (lane < E)
    for (int b = b0; b < b1; ++b) part += hist[(int64_t)b * E + lane];
  s_part[wave][lane] = part;
  __syncthreads();
  int pre = 0;
  for (int w = 0; w < wave; ++w) pre += s_part[w][lane];
  if (blk_base != nullptr && lane < E) {
    int run = pre;
    for (int b = b0; b < b1; ++b) {
      blk_base[(int64_t)b * E + lane] = run;
      run += hist[(int64_t)b * E + lane];
    }
  }
  if (wave == 15) s_tot[lane] = pre + part;
  __syncthreads();
  if (wave == 0) {
    const int c = lane < E ? s_tot[lane] : 0;
    const int inc = wave_inclusive_scan(c);
    if (lane < E) {
      if (counts != nullptr) counts[lane] = c;
      if (offsets != nullptr) offsets[lane] = inc - c;
    }
    if (offsets != nullptr && lane == 63) {
      offsets[E] = inc;
      for (int j = 1; j <= n_extra_groups; ++j) offsets[E + j] = inc + j * extra_rows;
    }
  }
}

// --------------------------------------------------------------- permute ----
// Slot assignment + index outputs, one thread per (token, k) pair, and the
// identity rows of the always-on groups.
__global__ __launch_bounds__(256) void permute_kernel(
    const int32_t* __restrict__ idx, const float* __restrict__ w, int T, int K,
    int E, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ blk_base, const int32_t* __restrict__ local_rank,
    int S, int32_t* __restrict__ token_map, float* __restrict__ dw,
    int32_t* __restrict__ slot_of, int n_extra_groups) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t npairs = (int64_t)T * K;
  if (p < npairs) {
    const int t = (int)(p / K);
    const int e = idx[p];
    const int r = local_rank[p];
    int slot = -1;
    if (e >= 0 && e < E && r >= 0) {
      const int base = blk_base != nullptr ? blk_base[(int64_t)(t / kChunk) * E + e] : 0;
      slot = offsets[e] + base + r;
      if (slot < 0 || slot >= S) slot = -1;
    }
    if (slot >= 0) {
      token_map[slot] = t;
      if (dw != nullptr) dw[slot] = w[p];
    }
    if (slot_of != nullptr) slot_of[p] = slot;
  } else if (p < npairs + (int64_t)n_extra_groups * T) {
    const int64_t q = p - npairs;
    token_map[S + q] = (int)(q % T);
  }
}

// ---------------------------------------------------------- scan+permute ----
// The scan and the permutation in one launch, for the fused layer. Workgroup
// b < ceil(T / 32) owns the (token, k) pairs of tokens 32b .. 32b+31, which lie
// in one 64-token chunk; it reduces the chunk histograms itself (nblk x E
// ints, 16 KB at T = 4096, read from L2) into the expert offsets and its
// chunk's bases, then assigns the slots as permute_kernel does. The sums are
// integer, so every workgroup sees the same offsets; workgroup 0 also writes
// counts and offsets. The workgroups after those write the identity rows of
// the always-on groups.
constexpr int kScanPermThreads = 256;
constexpr int kScanPermSegs = kScanPermThreads / 64;
constexpr int kScanPermTokens = 32;  // tokens per workgroup: K <= 8 pairs each

__global__ __launch_bounds__(kScanPermThreads) void scan_permute_kernel(
    const int32_t* __restrict__ hist, int nblk, const int32_t* __restrict__ idx, int T, int K,
    int E, const int32_t* __restrict__ local_rank, int S, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ token_map,
    int32_t* __restrict__ slot_of, int n_extra_groups) {
  __shared__ int s_all[kScanPermSegs][64];
  __shared__ int s_lo[kScanPermSegs][64];
  __shared__ int s_off[64];
  __shared__ int s_base[64];
  const int tid = threadIdx.x, e = tid & 63, sg = tid >> 6;
  const int n_pair_wgs = (T + kScanPermTokens - 1) / kScanPermTokens;
  if ((int)blockIdx.x >= n_pair_wgs) {  // uniform: rows of the always-on groups
    const int64_t q = (int64_t)(blockIdx.x - n_pair_wgs) * kScanPermThreads + tid;
    if (q < (int64_t)n_extra_groups * T) token_map[S + q] = (int)(q % T);
    return;
  }
  const int t0 = blockIdx.x * kScanPermTokens;
  const int chunk = t0 / kChunk;
  // segment sums of every chunk's histogram, and of the chunks below this one
  const int seg = (nblk + kScanPermSegs - 1) / kScanPermSegs;
  const int b0 = min(sg * seg, nblk), b1 = min(b0 + seg, nblk);
  int all = 0, lo = 0;
  if (e < E) {
    // batches of 8 independent loads, so a batch costs one round trip
    for (int b = b0; b < b1; b += 8) {
      int v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = b + u < b1 ? hist[(int64_t)(b + u) * E + e] : 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        all += v[u];
        lo += b + u < chunk ? v[u] : 0;
      }
    }
  }
  s_all[sg][e] = all;
  s_lo[sg][e] = lo;
  __syncthreads();
  if (sg == 0) {
    int tot = 0, below = 0;
#pragma unroll
    for (int k = 0; k < kScanPermSegs; ++k) {
      tot += s_all[k][e];
      below += s_lo[k][e];
    }
    const int inc = wave_inclusive_scan(tot);  // lanes e >= E hold 0
    s_off[e] = inc - tot;
    s_base[e] = below;
    if (blockIdx.x == 0) {
      if (e < E) {
        if (counts != nullptr) counts[e] = tot;
        offsets[e] = inc - tot;
      }
      if (e == 63) {
        offsets[E] = inc;
        for (int j = 1; j <= n_extra_groups; ++j) offsets[E + j] = inc + j * T;
      }
    }
  }
  __syncthreads();
  const int64_t npairs = (int64_t)T * K;
  const int64_t p = (int64_t)t0 * K + tid;
  if (tid < kScanPermTokens * K && p < npairs) {
    const int ex = idx[p];
    const int r = local_rank[p];
    int slot = -1;
    if (ex >= 0 && ex < E && r >= 0) {
      slot = s_off[ex] + s_base[ex] + r;
      if (slot < 0 || slot >= S) slot = -1;
    }
    if (slot >= 0) token_map[slot] = (int)(p / K);
    if (slot_of != nullptr) slot_of[p] = slot;
  }
}

// -------------------------------------------------------------- dispatch ----
// Row gather dispatched[slot] = x[t]: one wave per (token, k) pair, 16 B/lane.
__global__ __launch_bounds__(256) void gather_rows_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int T, int K, int H,
    const int32_t* __restrict__ slot_of, uint16_t* __restrict__ dispatched) {
  const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (p >= (int64_t)T * K) return;
  const int slot = slot_of[p];
  if (slot < 0) return;
  const int t = (int)(p / K);
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(x + (int64_t)t * ldx);
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(dispatched + (int64_t)slot * H);
  for (int c = lane; c < H / 8; c += 64) dst[c] = src[c];
}

// --------------------------------------------------------------- combine ----
// Fused-path combine: token t's K slots (slot_of) are summed in ascending slot
// order (= ascending expert, the oracle's order, moe.py:90-103), weighted by
// topk_w, then the always-on group rows are added, all in fp32 registers, and
// the result is rounded to bf16 once. One workgroup per token, 8 columns/thread.
constexpr int kMaxK = 8;

__global__ __launch_bounds__(256) void combine_slots_kernel(
    const uint16_t* __restrict__ y, int64_t ldy, const int32_t* __restrict__ slot_of,
    const float* __restrict__ topk_w, int T, int K, int H, int extra_base,
    int n_extra_groups, uint16_t* __restrict__ out, int64_t ldo) {
  const int t = blockIdx.x;
  int s[kMaxK];
  float wt[kMaxK];
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) {
    const int sk = k < K ? slot_of[(int64_t)t * K + k] : -1;
    s[k] = sk >= 0 ? sk : INT_MAX;
    wt[k] = k < K ? topk_w[(int64_t)t * K + k] : 0.f;
  }
  // fixed sorting network (bubble) on compile-time indices: stays in registers
#pragma unroll
  for (int a = 0; a < kMaxK; ++a) {
#pragma unroll
    for (int b = 0; b < kMaxK - 1 - a; ++b) {
      if (s[b] > s[b + 1]) {
        const int ts = s[b]; s[b] = s[b + 1]; s[b + 1] = ts;
        const float tw = wt[b]; wt[b] = wt[b + 1]; wt[b + 1] = tw;
      }
    }
  }
  constexpr int kPreExtra = 2;  // always-on group rows loaded with the slot rows
  for (int c = threadIdx.x; c < H / 8; c += blockDim.x) {
    // every row load of this chunk is issued before the arithmetic, which
    // then runs in the fixed order: slots ascending, then the extra groups
    u32x4_t v[kMaxK], ve[kPreExtra];
#pragma unroll
    for (int k = 0; k < kMaxK; ++k)
      if (s[k] != INT_MAX) v[k] = reinterpret_cast<const u32x4_t*>(y + (int64_t)s[k] * ldy)[c];
#pragma unroll
    for (int g = 0; g < kPreExtra; ++g)
      if (g < n_extra_groups)
        ve[g] = reinterpret_cast<const u32x4_t*>(
            y + ((int64_t)extra_base + (int64_t)g * T + t) * ldy)[c];
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxK; ++k) {
      if (s[k] != INT_MAX) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[2 * j] = fmaf(wt[k], bf16lo(v[k][j]), acc[2 * j]);
          acc[2 * j + 1] = fmaf(wt[k], bf16hi(v[k][j]), acc[2 * j + 1]);
        }
      }
    }
    for (int g = 0; g < n_extra_groups; ++g) {
      u32x4_t vg;
      if (g < kPreExtra) {
        vg = g == 0 ? ve[0] : ve[1];
      } else {
        vg = reinterpret_cast<const u32x4_t*>(
            y + ((int64_t)extra_base + (int64_t)g * T + t) * ldy)[c];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] += bf16lo(vg[j]);
        acc[2 * j + 1] += bf16hi(vg[j]);
      }
    }
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(acc[2 * j], acc[2 * j + 1]);
    reinterpret_cast<u32x4_t*>(out + (int64_t)t * ldo)[c] = o;
  }
}

// Generic combine for an arbitrary token_map (the moe_combine op): build the
// inverse map as CSR (integer atomics only: counts and cursors), then each
// token's list is put in ascending slot order by rank counting and summed.
__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void count_tokens_kernel(const int32_t* __restrict__ token_map, int S,
                                    int T, int32_t* __restrict__ cnt) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= S) return;
  const int t = token_map[s];
  if (t >= 0 && t < T) atomicAdd(&cnt[t], 1);
}

// Exclusive scan of n ints in one workgroup of 1024 threads (contiguous chunk
// per thread). Writes out[0..n] (out[n] = total) and a copy into cursor[0..n).
__global__ __launch_bounds__(kScanThreads) void scan_generic_kernel(
    const int32_t* __restrict__ in, int n, int32_t* __restrict__ out,
    int32_t* __restrict__ cursor) {
  __shared__ int s_wave[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (n + kScanThreads - 1) / kScanThreads;
  const int i0 = min(tid * per, n), i1 = min(i0 + per, n);
  int local = 0;
  for (int i = i0; i < i1; ++i) local += in[i];
  const int inc = wave_inclusive_scan(local);
  if (lane == 63) s_wave[wave] = inc;
  __syncthreads();
  int wpre = 0;
  for (int w = 0; w < wave; ++w) wpre += s_wave[w];
  int run = wpre + inc - local;
  for (int i = i0; i < i1; ++i) {
    out[i] = run;
    if (cursor != nullptr) cursor[i] = run;
    run += in[i];
  }
  if (tid == kScanThreads - 1) out[n] = run;
}

__global__ void scatter_slots_kernel(const int32_t* __restrict__ token_map, int S,
                                     int T, int32_t* __restrict__ cursor,
                                     int32_t* __restrict__ list) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= S) return;
  const int t = token_map[s];
  if (t >= 0 && t < T) list[atomicAdd(&cursor[t], 1)] = s;
}

__global__ __launch_bounds__(256) void combine_lists_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ start,
    const int32_t* __restrict__ list, int32_t* __restrict__ sorted,
    const float* __restrict__ dw, int H, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int st = start[t], n = start[t + 1] - st;
  // slots are distinct, so rank = number of smaller entries is a permutation
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int v = list[st + i];
    int r = 0;
    for (int j = 0; j < n; ++j) r += list[st + j] < v;
    sorted[st + r] = v;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < H / 8; c += blockDim.x) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int i = 0; i < n; ++i) {
      const int s = sorted[st + i];
      const float wt = dw[s];
      const u32x4_t v = reinterpret_cast<const u32x4_t*>(y + (int64_t)s * H)[c];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = fmaf(wt, bf16lo(v[j]), acc[2 * j]);
        acc[2 * j + 1] = fmaf(wt, bf16hi(v[j]), acc[2 * j + 1]);
      }
    }
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(acc[2 * j], acc[2 * j + 1]);
    reinterpret_cast<u32x4_t*>(out + (int64_t)t * H)[c] = o;
  }
}

// ----------------------------------------------------------------- swiglu ---
__device__ __forceinline__ float silu(float x) { return x / (1.f + __expf(-x)); }

__global__ __launch_bounds__(256) void swiglu_vec_kernel(const uint16_t* __restrict__ in,
                                                         uint16_t* __restrict__ out,
                                                         int rows, int I) {
  const int cpr = I / 8;  // 16-byte chunks per output row
  const int64_t total = (int64_t)rows * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cpr;
    const int c = (int)(i - r * cpr);
    const u32x4_t g = reinterpret_cast<const u32x4_t*>(in + r * 2 * I)[c];
    const u32x4_t u = reinterpret_cast<const u32x4_t*>(in + r * 2 * I + I)[c];
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16x2(silu(bf16lo(g[j])) * bf16lo(u[j]), silu(bf16hi(g[j])) * bf16hi(u[j]));
    reinterpret_cast<u32x4_t*>(out + r * I)[c] = o;
  }
}

__global__ void swiglu_scalar_kernel(const uint16_t* __restrict__ in,
                                     uint16_t* __restrict__ out, int rows, int I) {
  const int64_t total = (int64_t)rows * I;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / I;
    const int c = (int)(i - r * I);
    const float g = bf16_to_f32(in[r * 2 * I + c]);
    const float u = bf16_to_f32(in[r * 2 * I + I + c]);
    out[i] = f32_to_bf16(silu(g) * u);
  }
}

// ------------------------------------------------------------ host helpers --
static inline int nchunks(int T) { return (T + kChunk - 1) / kChunk; }

int launch_route(const float* logits, int64_t ld, int n_parts, int64_t part_stride,
                 const float* bias, int T, int E, int K, int32_t* idx,
                 float* w, int32_t* blk_hist, int32_t* local_rank, int32_t* counts,
                 int32_t* offsets, int32_t* token_map, int32_t* slot_of,
                 int n_extra_groups, hipStream_t st) {
  // a single chunk (T <= 64) launches only the waves its tokens need (at
  // least one: wave 0 does the chunk's scan; 64 lanes cover the 64 experts)
  const int threads =
      nchunks(T) == 1 ? kWave * std::max(1, (T + kTokPerWave - 1) / kTokPerWave) : kRouteThreads;
  hipLaunchKernelGGL(route_kernel, dim3(nchunks(T)), dim3(threads), 0, st, logits,
                     ld, n_parts, part_stride, bias, T, E, K, idx, w, blk_hist, local_rank,
                     counts, offsets, token_map, slot_of, n_extra_groups);
  return check_launch("route_kernel");
}

int launch_scan(const int32_t* hist, int nblk, int E, int32_t* counts, int32_t* offsets,
                int32_t* blk_base, int n_extra_groups, int extra_rows, hipStream_t st) {
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(kScanThreads), 0, st, hist, nblk, E,
                     counts, offsets, blk_base, n_extra_groups, extra_rows);
  return check_launch("scan_kernel");
}

int launch_scan_permute(const int32_t* hist, int nblk, const int32_t* idx, int T, int K,
                        int E, const int32_t* local_rank, int S, int32_t* counts,
                        int32_t* offsets, int32_t* token_map, int32_t* slot_of,
                        int n_extra_groups, hipStream_t st) {
  if (T == 0) return DSK_OK;
  if (K > kScanPermThreads / kScanPermTokens || E > 64)
    return fail(DSK_ERR_INVALID_ARG, "scan_permute: needs top_k <= 8 and at most 64 experts");
  const int64_t n_wgs = (T + kScanPermTokens - 1) / kScanPermTokens +
                        ((int64_t)n_extra_groups * T + kScanPermThreads - 1) / kScanPermThreads;
  hipLaunchKernelGGL(scan_permute_kernel, dim3((unsigned)n_wgs), dim3(kScanPermThreads), 0, st,
                     hist, nblk, idx, T, K, E, local_rank, S, counts, offsets, token_map,
                     slot_of, n_extra_groups);
  return check_launch("scan_permute_kernel");
}

int launch_permute(const int32_t* idx, const float* w, int T, int K, int E,
                   const int32_t* offsets, const int32_t* blk_base,
                   const int32_t* local_rank, int S, int32_t* token_map, float* dw,
                   int32_t* slot_of, int n_extra_groups, hipStream_t st) {
  const int64_t n = (int64_t)T * K + (int64_t)n_extra_groups * T;
  if (n == 0) return DSK_OK;
  hipLaunchKernelGGL(permute_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     idx, w, T, K, E, offsets, blk_base, local_rank, S, token_map, dw,
                     slot_of, n_extra_groups);
  return check_launch("permute_kernel");
}

int launch_combine_slots(const uint16_t* y, int64_t ldy, const int32_t* slot_of,
                         const float* topk_w, int T, int K, int H, int extra_base,
                         int n_extra_groups, uint16_t* out, int64_t ldo, hipStream_t st) {
  if (T == 0) return DSK_OK;
  hipLaunchKernelGGL(combine_slots_kernel, dim3(T), dim3(256), 0, st, y, ldy, slot_of,
                     topk_w, T, K, H, extra_base, n_extra_groups, out, ldo);
  return check_launch("combine_slots_kernel");
}

}  // namespace dsk

using namespace dsk;

// =============================================================== C ABI =====
extern "C" size_t dsk_moe_routing_workspace_size(int num_tokens, int num_experts) {
  if (num_tokens <= 0 || num_experts <= 0) return 256;
  return align_up((size_t)nchunks(num_tokens) * num_experts * sizeof(int32_t), 256);
}

extern "C" int dsk_moe_routing(const float* logits, int64_t ld_logits, int32_t* topk_idx,
                               float* topk_w, int32_t* expert_counts, int num_tokens,
                               int num_experts, int top_k, void* workspace,
                               size_t workspace_bytes, void* stream) {
  DSK_REQUIRE(num_experts >= 1 && num_experts <= DSK_MAX_EXPERTS, DSK_ERR_INVALID_ARG,
              "moe_routing: num_experts must be in [1, 64]");
  DSK_REQUIRE(top_k >= 1 && top_k <= DSK_MAX_TOP_K, DSK_ERR_INVALID_ARG,
              "moe_routing: top_k must be in [1, 6]");
  DSK_REQUIRE(top_k <= num_experts, DSK_ERR_INVALID_ARG,
              "moe_routing: top_k must not exceed num_experts");
  DSK_REQUIRE(num_tokens >= 0, DSK_ERR_INVALID_ARG, "moe_routing: num_tokens < 0");
  DSK_REQUIRE(ld_logits >= num_experts, DSK_ERR_INVALID_ARG,
              "moe_routing: ld_logits < num_experts");
  DSK_REQUIRE(expert_counts != nullptr, DSK_ERR_NULL_PTR, "moe_routing: expert_counts is NULL");
  hipStream_t st = as_stream(stream);
  if (num_tokens == 0) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, st, expert_counts,
                       (int64_t)num_experts, 0);
    return check_launch("fill_i32_kernel");
  }
  DSK_REQUIRE(logits && topk_idx && topk_w, DSK_ERR_NULL_PTR, "moe_routing: NULL pointer");
  const int nblk = nchunks(num_tokens);
  if (nblk == 1) {
    // single chunk: the route kernel's own histogram is the count vector
    return launch_route(logits, ld_logits, 1, 0, nullptr, num_tokens, num_experts, top_k,
                        topk_idx, topk_w, expert_counts, nullptr, nullptr, nullptr, nullptr,
                        nullptr, 0, st);
  }
  DSK_REQUIRE(workspace != nullptr &&
                  workspace_bytes >= dsk_moe_routing_workspace_size(num_tokens, num_experts),
              DSK_ERR_WORKSPACE, "moe_routing: workspace too small");
  int32_t* hist = static_cast<int32_t*>(workspace);
  int rc = launch_route(logits, ld_logits, 1, 0, nullptr, num_tokens, num_experts, top_k,
                        topk_idx, topk_w, hist, nullptr, nullptr, nullptr, nullptr, nullptr, 0,
                        st);
  if (rc) return rc;
  return launch_scan(hist, nblk, num_experts, expert_counts, nullptr, nullptr, 0, 0, st);
}

extern "C" int dsk_moe_scan(const int32_t* expert_counts, int32_t* expert_offsets,
                            int num_experts, void* stream) {
  DSK_REQUIRE(num_experts >= 1 && num_experts <= DSK_MAX_EXPERTS, DSK_ERR_INVALID_ARG,
              "moe_scan: num_experts must be in [1, 64]");
  DSK_REQUIRE(expert_counts && expert_offsets, DSK_ERR_NULL_PTR, "moe_scan: NULL pointer");
  return launch_scan(expert_counts, 1, num_experts, nullptr, expert_offsets, nullptr, 0, 0,
                     as_stream(stream));
}

extern "C" size_t dsk_moe_dispatch_workspace_size(int num_tokens, int num_experts,
                                                  int top_k) {
  if (num_tokens <= 0) return 256;
  const size_t nb = (size_t)nchunks(num_tokens) * num_experts * sizeof(int32_t);
  const size_t pairs = (size_t)num_tokens * top_k * sizeof(int32_t);
  return 2 * align_up(nb, 256) + 2 * align_up(pairs, 256);
}

extern "C" int dsk_moe_dispatch(const dsk_bf16* x, int64_t ld_x, const int32_t* topk_idx,
                                const float* topk_w, const int32_t* expert_offsets,
                                dsk_bf16* dispatched, int32_t* token_map,
                                float* dispatched_weights, int num_tokens, int hidden,
                                int num_experts, int top_k, void* workspace,
                                size_t workspace_bytes, void* stream) {
  DSK_REQUIRE(num_experts >= 1 && num_experts <= DSK_MAX_EXPERTS, DSK_ERR_INVALID_ARG,
              "moe_dispatch: num_experts must be in [1, 64]");
  DSK_REQUIRE(top_k >= 1 && top_k <= DSK_MAX_TOP_K, DSK_ERR_INVALID_ARG,
              "moe_dispatch: top_k must be in [1, 6]");
  DSK_REQUIRE(hidden > 0 && hidden % 8 == 0, DSK_ERR_INVALID_ARG,
              "moe_dispatch: hidden_size must be divisible by 8 for 128-bit vectorized access");
  DSK_REQUIRE(num_tokens >= 0, DSK_ERR_INVALID_ARG, "moe_dispatch: num_tokens < 0");
  if (num_tokens == 0) return DSK_OK;
  DSK_REQUIRE(topk_idx && topk_w && expert_offsets && token_map && dispatched_weights,
              DSK_ERR_NULL_PTR, "moe_dispatch: NULL pointer");
  if (dispatched != nullptr) {
    DSK_REQUIRE(x != nullptr, DSK_ERR_NULL_PTR, "moe_dispatch: x is NULL");
    DSK_REQUIRE(aligned16(x) && aligned16(dispatched) && ld_x % 8 == 0 && ld_x >= hidden,
                DSK_ERR_ALIGNMENT, "moe_dispatch: x/dispatched must be 16-byte aligned rows");
  }
  DSK_REQUIRE(workspace != nullptr &&
                  workspace_bytes >= dsk_moe_dispatch_workspace_size(num_tokens, num_experts, top_k),
              DSK_ERR_WORKSPACE, "moe_dispatch: workspace too small");
  hipStream_t st = as_stream(stream);
  const int nblk = nchunks(num_tokens);
  const size_t nb = align_up((size_t)nblk * num_experts * sizeof(int32_t), 256);
  const size_t pairs = align_up((size_t)num_tokens * top_k * sizeof(int32_t), 256);
  char* ws = static_cast<char*>(workspace);
  int32_t* hist = reinterpret_cast<int32_t*>(ws);
  int32_t* base = reinterpret_cast<int32_t*>(ws + nb);
  int32_t* rank = reinterpret_cast<int32_t*>(ws + 2 * nb);
  int32_t* slot_of = reinterpret_cast<int32_t*>(ws + 2 * nb + pairs);
  hipLaunchKernelGGL(rank_kernel, dim3(nblk), dim3(kRankThreads), 0, st, topk_idx,
                     num_tokens, top_k, num_experts, hist, rank);
  int rc = check_launch("rank_kernel");
  if (rc) return rc;
  if (nblk > 1) {
    rc = launch_scan(hist, nblk, num_experts, nullptr, nullptr, base, 0, 0, st);
    if (rc) return rc;
  }
  const int S = num_tokens * top_k;
  rc = launch_permute(topk_idx, topk_w, num_tokens, top_k, num_experts, expert_offsets,
                      nblk > 1 ? base : nullptr, rank, S, token_map, dispatched_weights,
                      slot_of, 0, st);
  if (rc) return rc;
  if (dispatched != nullptr) {
    hipLaunchKernelGGL(gather_rows_kernel, dim3((S + 3) / 4), dim3(256), 0, st, x, ld_x,
                       num_tokens, top_k, hidden, slot_of, dispatched);
    rc = check_launch("gather_rows_kernel");
  }
  return rc;
}

extern "C" size_t dsk_moe_combine_workspace_size(int total_slots, int num_tokens) {
  const size_t t1 = align_up((size_t)(num_tokens + 1) * sizeof(int32_t), 256);
  const size_t s1 = align_up((size_t)(total_slots > 0 ? total_slots : 1) * sizeof(int32_t), 256);
  return 2 * t1 + 2 * s1;
}

extern "C" int dsk_moe_combine(const dsk_bf16* expert_out, const int32_t* token_map,
                               const float* dispatched_weights, dsk_bf16* out,
                               int total_slots, int num_tokens, int hidden,
                               void* workspace, size_t workspace_bytes, void* stream) {
  DSK_REQUIRE(num_tokens > 0, DSK_ERR_INVALID_ARG, "moe_combine: num_tokens must be positive.");
  DSK_REQUIRE(total_slots >= 0, DSK_ERR_INVALID_ARG, "moe_combine: total_slots < 0");
  DSK_REQUIRE(hidden > 0 && hidden % 8 == 0, DSK_ERR_INVALID_ARG,
              "moe_combine: hidden_size must be divisible by 8");
  DSK_REQUIRE(out != nullptr, DSK_ERR_NULL_PTR, "moe_combine: out is NULL");
  DSK_REQUIRE(total_slots == 0 || (expert_out && token_map && dispatched_weights),
              DSK_ERR_NULL_PTR, "moe_combine: NULL pointer");
  DSK_REQUIRE(aligned16(out) && (total_slots == 0 || aligned16(expert_out)),
              DSK_ERR_ALIGNMENT, "moe_combine: rows must be 16-byte aligned");
  DSK_REQUIRE(workspace != nullptr &&
                  workspace_bytes >= dsk_moe_combine_workspace_size(total_slots, num_tokens),
              DSK_ERR_WORKSPACE, "moe_combine: workspace too small");
  hipStream_t st = as_stream(stream);
  const size_t t1 = align_up((size_t)(num_tokens + 1) * sizeof(int32_t), 256);
  const size_t s1 = align_up((size_t)(total_slots > 0 ? total_slots : 1) * sizeof(int32_t), 256);
  char* ws = static_cast<char*>(workspace);
  int32_t* cnt = reinterpret_cast<int32_t*>(ws);          // counts, later cursors
  int32_t* start = reinterpret_cast<int32_t*>(ws + t1);
  int32_t* list = reinterpret_cast<int32_t*>(ws + 2 * t1);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + 2 * t1 + s1);
  const unsigned gT = (unsigned)std::min<int64_t>(((int64_t)num_tokens + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_i32_kernel, dim3(gT), dim3(256), 0, st, cnt, (int64_t)num_tokens, 0);
  int rc = check_launch("fill_i32_kernel");
  if (rc) return rc;
  const unsigned gS = (unsigned)(((int64_t)total_slots + 255) / 256);
  if (total_slots > 0) {
    hipLaunchKernelGGL(count_tokens_kernel, dim3(gS), dim3(256), 0, st, token_map,
                       total_slots, num_tokens, cnt);
    if ((rc = check_launch("count_tokens_kernel"))) return rc;
  }
  hipLaunchKernelGGL(scan_generic_kernel, dim3(1), dim3(kScanThreads), 0, st, cnt,
                     num_tokens, start, cnt);
  if ((rc = check_launch("scan_generic_kernel"))) return rc;
  if (total_slots > 0) {
    hipLaunchKernelGGL(scatter_slots_kernel, dim3(gS), dim3(256), 0, st, token_map,
                       total_slots, num_tokens, cnt, list);
    if ((rc = check_launch("scatter_slots_kernel"))) return rc;
  }
  hipLaunchKernelGGL(combine_lists_kernel, dim3(num_tokens), dim3(256), 0, st, expert_out,
                     start, list, sorted, dispatched_weights, hidden, out);
  return check_launch("combine_lists_kernel");
}

extern "C" int dsk_swiglu(const dsk_bf16* in, dsk_bf16* out, int rows, int intermediate,
                          void* stream) {
  DSK_REQUIRE(intermediate > 0 && intermediate % 2 == 0, DSK_ERR_INVALID_ARG,
              "swiglu: intermediate_size must be even");
  DSK_REQUIRE(rows >= 0, DSK_ERR_INVALID_ARG, "swiglu: rows < 0");
  if (rows == 0) return DSK_OK;
  DSK_REQUIRE(in && out, DSK_ERR_NULL_PTR, "swiglu: NULL pointer");
  hipStream_t st = as_stream(stream);
  if (intermediate % 8 == 0 && aligned16(in) && aligned16(out)) {
    const int64_t total = (int64_t)rows * (intermediate / 8);
    const unsigned g = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(swiglu_vec_kernel, dim3(g), dim3(256), 0, st, in, out, rows,
                       intermediate);
  } else {
    const int64_t total = (int64_t)rows * intermediate;
    const unsigned g = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(swiglu_scalar_kernel, dim3(g), dim3(256), 0, st, in, out, rows,
                       intermediate);
  }
  return check_launch("swiglu_kernel");
}
