// Grouped bf16 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x16_bf16), fp32
// accumulation, used for the MoE expert projections and the MLA dense
// projections.
//
//   C[m, n] = sum_k A[row(m), k] * B_g[n, k]     for m in group g's row range
//
// A is K-contiguous (activations, optionally gathered through a row map so the
// dispatch copy can be skipped), B_g is the K-contiguous nn.Linear weight
// [N, K] of group g (expert), C is row-major. Group row ranges come from a
// device-side offsets array (expert_offsets), so the host never waits for them.
//
// Scheduling: a persistent grid (one workgroup per CU). Output tiles are
// enumerated group-major, then N-tile, then M-tile, and the enumeration is cut
// into 8 contiguous ranges, one per XCD (workgroup i runs on XCD i % 8): the
// M-tiles that share a weight tile run at the same time on the same XCD, so the
// weight tile is fetched from HBM once and re-read from that XCD's L2.
//
// Tile: BM tokens x BN weight rows x 64 (K) per stage, two LDS stages
// (global->register prefetch of stage k+1 overlaps the MFMAs of stage k). LDS
// rows are 128 B with a 16-byte-chunk XOR swizzle (chunk ^ (row & 7)), so both
// the coalesced row stores and the MFMA fragment reads (32 rows x one chunk)
// are bank-conflict free. The weight fragment is MFMA operand A and the token
// fragment operand B, so each lane ends up owning 4 consecutive output columns
// of one token row (8-byte stores).
//
// SWIGLU mode fuses the SwiGLU activation into the epilogue: each wave's
// weight rows are half gate rows (j) and half the matching up rows (I + j), so
// silu(gate) * up is computed from fp32 accumulators held by the same lane.
#include "dsk_internal.hpp"

#include <algorithm>
#include <cstdio>
#include <mutex>

namespace dsk {

constexpr int kMaxGroups = 128;
constexpr int kGemmThreads = 256;
constexpr int kBK = 64;

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + __expf(-x)); }

template <int BM, int BN, int WAVES_M, int WAVES_N, bool SWIGLU>
struct GemmCfg {
  static_assert(WAVES_M * WAVES_N == 4, "4 waves per workgroup");
  static constexpr int WM = BM / WAVES_M;
  static constexpr int WN = BN / WAVES_N;
  static constexpr int TM = WM / 32;
  static constexpr int TN = WN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 block");
  static_assert(!SWIGLU || (TN % 2 == 0), "SwiGLU needs matching gate/up blocks");
  static constexpr int OUT_N = SWIGLU ? BN / 2 : BN;
  static constexpr int A_LOADS = BM * (kBK / 8) / kGemmThreads;  // 16-byte chunks per thread
  static constexpr int B_LOADS = BN * (kBK / 8) / kGemmThreads;
  static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small");
  static constexpr int STAGE_ELEMS = (BM + BN) * kBK;
  static constexpr int LDS_BYTES = 2 * STAGE_ELEMS * 2;
};

template <int BM, int BN, int WAVES_M, int WAVES_N, bool SWIGLU>
__global__ __launch_bounds__(kGemmThreads, 1) void grouped_gemm_kernel(GemmArgs p) {
  using Cfg = GemmCfg<BM, BN, WAVES_M, WAVES_N, SWIGLU>;
  constexpr int WM = Cfg::WM, WN = Cfg::WN, TM = Cfg::TM, TN = Cfg::TN;
  constexpr int OUT_N = Cfg::OUT_N;
  constexpr int A_LOADS = Cfg::A_LOADS, B_LOADS = Cfg::B_LOADS;

  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  __shared__ int s_inc[kMaxGroups];
  __shared__ int s_mb[kMaxGroups];
  __shared__ int s_me[kMaxGroups];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_m = wave / WAVES_N;
  const int wave_n = wave % WAVES_N;
  const int G = p.offsets != nullptr ? p.G : 1;
  const int NT = (p.N + OUT_N - 1) / OUT_N;

  // ---- group table: row ranges and inclusive prefix of tile counts
  if (tid < kMaxGroups) {
    int cnt = 0;
    if (tid < G) {
      int mb = 0, me = p.M;
      if (p.offsets != nullptr) {
        mb = min(max(p.offsets[tid], 0), p.M);
        me = min(max(p.offsets[tid + 1], mb), p.M);
      }
      s_mb[tid] = mb;
      s_me[tid] = me;
      cnt = ((me - mb + BM - 1) / BM) * NT;
    }
    s_inc[tid] = wave_inclusive_scan(cnt);
  }
  __syncthreads();
  const int carry = s_inc[63];
  __syncthreads();
  if (tid >= 64 && tid < kMaxGroups) s_inc[tid] += carry;
  __syncthreads();
  const int total = s_inc[G - 1];

  // ---- XCD-aware persistent enumeration
  const int xcd = blockIdx.x & 7;
  const int q = blockIdx.x >> 3;
  const int per_xcd = gridDim.x >> 3;
  const int share = (total + 7) >> 3;
  const int w_beg = xcd * share;
  const int w_end = min(w_beg + share, total);

  const int ld_chunk = tid & 7;     // 16-byte chunk of a 128-byte LDS row
  const int ld_row = tid >> 3;      // 0..31 (+32*i)
  const int st_off = ld_row * 8 + (ld_chunk ^ (ld_row & 7));  // u32x4 units, +256*i
  u32x4_t* lds4 = reinterpret_cast<u32x4_t*>(lds);
  constexpr int STAGE4 = Cfg::STAGE_ELEMS / 8;
  constexpr int A4 = BM * kBK / 8;
  const int nk = p.K / kBK;
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};

  for (int W = w_beg + q; W < w_end; W += per_xcd) {
    int lo = 0, hi = G - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_inc[mid] > W) hi = mid; else lo = mid + 1;
    }
    const int g = lo;
    const int local = W - (g > 0 ? s_inc[g - 1] : 0);
    const int mb = s_mb[g], me = s_me[g];
    const int mtiles = (me - mb + BM - 1) / BM;
    const int nt = local / mtiles;
    const int mt = local - nt * mtiles;
    const int m0 = mb + mt * BM;
    const int n0 = nt * OUT_N;
    const uint16_t* Bg = p.B + (int64_t)g * p.b_group_stride;

    // ---- per-thread global source rows
    const uint16_t* a_src[A_LOADS];
    bool a_ok[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int m = m0 + ld_row + 32 * i;
      bool ok = m < me;
      int row = m;
      if (ok && p.a_rows != nullptr) {
        row = p.a_rows[m];
        ok = row >= 0 && row < p.a_rows_limit;
      }
      a_ok[i] = ok;
      a_src[i] = p.A + (ok ? (int64_t)row * p.lda : 0) + ld_chunk * 8;
    }
    const uint16_t* b_src[B_LOADS];
    bool b_ok[B_LOADS];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int r = ld_row + 32 * i;
      int brow, col;
      if constexpr (SWIGLU) {
        const int wn = r / WN, w = r % WN;
        constexpr int half = WN / 2;
        col = n0 + wn * half + (w % half);
        brow = (w < half) ? col : p.up_row_offset + col;
      } else {
        col = n0 + r;
        brow = col;
      }
      b_ok[i] = col < p.N;
      b_src[i] = Bg + (b_ok[i] ? (int64_t)brow * p.ldb : 0) + ld_chunk * 8;
    }

    int tm_active = (me - (m0 + wave_m * WM) + 31) / 32;
    tm_active = max(0, min(TM, tm_active));

    floatx16_t acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

    u32x4_t ra[A_LOADS], rb[B_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      ra[i] = a_ok[i] ? *reinterpret_cast<const u32x4_t*>(a_src[i]) : zero4;
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i)
      rb[i] = b_ok[i] ? *reinterpret_cast<const u32x4_t*>(b_src[i]) : zero4;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) lds4[st_off + 256 * i] = ra[i];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) lds4[A4 + st_off + 256 * i] = rb[i];
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
      const bool more = kt + 1 < nk;
      if (more) {
        const int koff = (kt + 1) * kBK;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
          ra[i] = a_ok[i] ? *reinterpret_cast<const u32x4_t*>(a_src[i] + koff) : zero4;
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i)
          rb[i] = b_ok[i] ? *reinterpret_cast<const u32x4_t*>(b_src[i] + koff) : zero4;
      }
      const u32x4_t* As = lds4 + (kt & 1) * STAGE4;
      const u32x4_t* Bs = As + A4;
#pragma unroll
      for (int kk = 0; kk < kBK / 16; ++kk) {
        const int ch = 2 * kk + (lane >> 5);
        bf16x8_t bfr[TN], afr[TM];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int rr = wave_n * WN + 32 * j + (lane & 31);
          bfr[j] = __builtin_bit_cast(bf16x8_t, Bs[rr * 8 + (ch ^ (rr & 7))]);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          if (i < tm_active) {
            const int rr = wave_m * WM + 32 * i + (lane & 31);
            afr[i] = __builtin_bit_cast(bf16x8_t, As[rr * 8 + (ch ^ (rr & 7))]);
          }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          if (i < tm_active) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], afr[i], acc[j][i], 0, 0, 0);
          }
        }
      }
      if (more) {
        u32x4_t* Ad = lds4 + ((kt + 1) & 1) * STAGE4;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) Ad[st_off + 256 * i] = ra[i];
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) Ad[A4 + st_off + 256 * i] = rb[i];
      }
      __syncthreads();
    }

    // ---- epilogue: lane owns token row m = ... + (lane & 31) and 4 consecutive
    // output columns per 4-register group
    constexpr int JN = SWIGLU ? TN / 2 : TN;
    constexpr int WOUT = SWIGLU ? WN / 2 : WN;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if (i >= tm_active) continue;
      const int m = m0 + wave_m * WM + 32 * i + (lane & 31);
      if (m >= me) continue;
      uint16_t* crow = p.C + (int64_t)m * p.ldc;
#pragma unroll
      for (int j = 0; j < JN; ++j) {
#pragma unroll
        for (int qg = 0; qg < 4; ++qg) {
          const int nb = n0 + wave_n * WOUT + 32 * j + 8 * qg + 4 * (lane >> 5);
          float v[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if constexpr (SWIGLU)
              v[c] = silu_f(acc[j][i][4 * qg + c]) * acc[j + TN / 2][i][4 * qg + c];
            else
              v[c] = acc[j][i][4 * qg + c];
          }
          if (nb + 3 < p.N) {
            u32x2_t o;
            o[0] = pack_bf16x2(v[0], v[1]);
            o[1] = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<u32x2_t*>(crow + nb) = o;
          } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (nb + c < p.N) crow[nb + c] = f32_to_bf16(v[c]);
          }
        }
      }
    }
  }
}

// Zero the output rows that no group covers: [0, offsets[0]) and [offsets[G], M).
__global__ __launch_bounds__(256) void zero_uncovered_rows_kernel(
    uint16_t* __restrict__ C, int64_t ldc, int M, int N,
    const int32_t* __restrict__ offsets, int G) {
  const int off0 = min(max(offsets[0], 0), M);
  const int offG = min(max(offsets[G], off0), M);
  const int nrows = off0 + (M - offG);
  for (int i = blockIdx.x; i < nrows; i += gridDim.x) {
    const int row = i < off0 ? i : offG + (i - off0);
    for (int c = threadIdx.x; c < N; c += blockDim.x) C[(int64_t)row * ldc + c] = 0;
  }
}

// ------------------------------------------------------------------ host ----
static int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int BM, int BN, int WAVES_M, int WAVES_N, bool SWIGLU>
static int launch_grouped_gemm(const GemmArgs& a, hipStream_t st) {
  using Cfg = GemmCfg<BM, BN, WAVES_M, WAVES_N, SWIGLU>;
  auto kern = grouped_gemm_kernel<BM, BN, WAVES_M, WAVES_N, SWIGLU>;
  static std::once_flag once;
  std::call_once(once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::LDS_BYTES);
  });
  const int G = a.offsets != nullptr ? a.G : 1;
  const int64_t nt = (a.N + Cfg::OUT_N - 1) / Cfg::OUT_N;
  const int64_t upper = ((int64_t)(a.M + BM - 1) / BM + (a.offsets ? G : 0)) * nt;
  int64_t nwg = std::min<int64_t>(upper, (int64_t)num_cus());
  nwg = std::max<int64_t>(8, (nwg + 7) / 8 * 8);
  hipLaunchKernelGGL(kern, dim3((unsigned)nwg), dim3(kGemmThreads), Cfg::LDS_BYTES, st, a);
  return check_launch("grouped_gemm_kernel");
}

static int validate_gemm(const GemmArgs& a, const char* who) {
  char buf[256];
  if (a.M < 0 || a.N <= 0 || a.K <= 0) {
    snprintf(buf, sizeof buf, "%s: invalid sizes M=%d N=%d K=%d", who, a.M, a.N, a.K);
    return fail(DSK_ERR_INVALID_ARG, buf);
  }
  if (a.K % kBK != 0) {
    snprintf(buf, sizeof buf, "%s: K=%d must be a multiple of %d", who, a.K, kBK);
    return fail(DSK_ERR_INVALID_ARG, buf);
  }
  if (a.offsets != nullptr && (a.G < 1 || a.G > kMaxGroups)) {
    snprintf(buf, sizeof buf, "%s: number of groups %d must be in [1, %d]", who, a.G, kMaxGroups);
    return fail(DSK_ERR_INVALID_ARG, buf);
  }
  if (!a.A || !a.B || !a.C) return fail(DSK_ERR_NULL_PTR, std::string(who) + ": NULL pointer");
  if (!aligned16(a.A) || !aligned16(a.B) || a.lda % 8 || a.ldb % 8 || a.b_group_stride % 8)
    return fail(DSK_ERR_ALIGNMENT, std::string(who) + ": A/B rows must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(a.C) & 7u) || a.ldc % 4)
    return fail(DSK_ERR_ALIGNMENT, std::string(who) + ": C rows must be 8-byte aligned");
  if (a.lda < a.K || a.ldb < a.K)
    return fail(DSK_ERR_INVALID_ARG, std::string(who) + ": leading dimension < K");
  return DSK_OK;
}

// Tile choice: 128 tokens x 256 weight rows, waves side by side along the
// weight rows (each wave 128 x 64), so a wave can skip the 32-row blocks past
// the end of its group.
int run_gemm(const GemmArgs& a, bool swiglu, hipStream_t st) {
  if (a.M == 0) return DSK_OK;
  if (swiglu) return launch_grouped_gemm<128, 256, 1, 4, true>(a, st);
  return launch_grouped_gemm<128, 256, 1, 4, false>(a, st);
}

int zero_uncovered_rows(uint16_t* C, int64_t ldc, int M, int N, const int32_t* offsets,
                        int G, hipStream_t st) {
  if (M == 0) return DSK_OK;
  hipLaunchKernelGGL(zero_uncovered_rows_kernel, dim3(64), dim3(256), 0, st, C, ldc, M, N,
                     offsets, G);
  return check_launch("zero_uncovered_rows_kernel");
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_moe_gemm1(const dsk_bf16* dispatched, const dsk_bf16* packed_w1,
                             dsk_bf16* out, const int32_t* expert_offsets, int total_slots,
                             int num_experts, int hidden, int n_out, void* stream) {
  DSK_REQUIRE(total_slots >= 0, DSK_ERR_INVALID_ARG, "moe_gemm1: total_slots < 0");
  if (total_slots == 0) return DSK_OK;
  DSK_REQUIRE(expert_offsets != nullptr, DSK_ERR_NULL_PTR, "moe_gemm1: expert_offsets is NULL");
  GemmArgs a{};
  a.A = dispatched; a.lda = hidden;
  a.B = packed_w1; a.ldb = hidden; a.b_group_stride = (int64_t)n_out * hidden;
  a.C = out; a.ldc = n_out;
  a.offsets = expert_offsets; a.G = num_experts;
  a.M = total_slots; a.N = n_out; a.K = hidden;
  int rc = validate_gemm(a, "moe_gemm1");
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  if ((rc = zero_uncovered_rows(out, n_out, total_slots, n_out, expert_offsets, num_experts, st)))
    return rc;
  return run_gemm(a, false, st);
}

extern "C" int dsk_moe_gemm1_swiglu(const dsk_bf16* dispatched, const dsk_bf16* packed_w1,
                                    dsk_bf16* out, const int32_t* expert_offsets,
                                    int total_slots, int num_experts, int hidden,
                                    int intermediate, void* stream) {
  DSK_REQUIRE(total_slots >= 0, DSK_ERR_INVALID_ARG, "moe_gemm1_swiglu: total_slots < 0");
  if (total_slots == 0) return DSK_OK;
  DSK_REQUIRE(expert_offsets != nullptr, DSK_ERR_NULL_PTR,
              "moe_gemm1_swiglu: expert_offsets is NULL");
  GemmArgs a{};
  a.A = dispatched; a.lda = hidden;
  a.B = packed_w1; a.ldb = hidden; a.b_group_stride = (int64_t)2 * intermediate * hidden;
  a.C = out; a.ldc = intermediate;
  a.offsets = expert_offsets; a.G = num_experts;
  a.M = total_slots; a.N = intermediate; a.K = hidden;
  a.up_row_offset = intermediate;
  int rc = validate_gemm(a, "moe_gemm1_swiglu");
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  if ((rc = zero_uncovered_rows(out, intermediate, total_slots, intermediate, expert_offsets,
                                num_experts, st)))
    return rc;
  return run_gemm(a, true, st);
}

extern "C" int dsk_moe_gemm2(const dsk_bf16* swiglu_out, const dsk_bf16* w2, dsk_bf16* out,
                             const int32_t* expert_offsets, int total_slots, int num_experts,
                             int intermediate, int hidden, void* stream) {
  DSK_REQUIRE(total_slots >= 0, DSK_ERR_INVALID_ARG, "moe_gemm2: total_slots < 0");
  if (total_slots == 0) return DSK_OK;
  DSK_REQUIRE(expert_offsets != nullptr, DSK_ERR_NULL_PTR, "moe_gemm2: expert_offsets is NULL");
  GemmArgs a{};
  a.A = swiglu_out; a.lda = intermediate;
  a.B = w2; a.ldb = intermediate; a.b_group_stride = (int64_t)hidden * intermediate;
  a.C = out; a.ldc = hidden;
  a.offsets = expert_offsets; a.G = num_experts;
  a.M = total_slots; a.N = hidden; a.K = intermediate;
  int rc = validate_gemm(a, "moe_gemm2");
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  if ((rc = zero_uncovered_rows(out, hidden, total_slots, hidden, expert_offsets, num_experts,
                                st)))
    return rc;
  return run_gemm(a, false, st);
}

extern "C" int dsk_linear(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w, dsk_bf16* out,
                          int64_t ld_out, int M, int K, int N, void* stream) {
  DSK_REQUIRE(M >= 0, DSK_ERR_INVALID_ARG, "linear: M < 0");
  if (M == 0) return DSK_OK;
  GemmArgs a{};
  a.A = x; a.lda = ld_x;
  a.B = w; a.ldb = K; a.b_group_stride = 0;
  a.C = out; a.ldc = ld_out;
  a.offsets = nullptr; a.G = 1;
  a.M = M; a.N = N; a.K = K;
  int rc = validate_gemm(a, "linear");
  if (rc) return rc;
  DSK_REQUIRE(ld_out >= N, DSK_ERR_INVALID_ARG, "linear: ld_out < N");
  return run_gemm(a, false, as_stream(stream));
}

extern "C" int dsk_kv_upproj(const dsk_bf16* normed_kv, int64_t ld_in, const dsk_bf16* weight,
                             dsk_bf16* out, int rows, int kv_lora_rank, int out_dim,
                             void* stream) {
  return dsk_linear(normed_kv, ld_in, weight, out, out_dim, rows, kv_lora_rank, out_dim,
                    stream);
}
