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
// Data movement: BM tokens x BN weight rows x 64 (K) per stage, in a ring of
// kStages LDS stages filled by direct global->LDS DMA (global_load_lds_dwordx4,
// no register staging): while the MFMAs consume stage k, the loads of stages
// k+1 .. k+kStages-1 are in flight. One workgroup barrier per K step.
// LDS rows are 128 B with a 16-byte-chunk XOR swizzle
// chunk ^ (row & 7) ^ ((row >> 3) & 1): with 64 banks of 4 B, 16 lanes of a
// ds_read_b128 (16 rows, one logical chunk) then hit 16 distinct bank quads.
// A DMA instruction writes 1 KB = 8 rows, lane l landing at row l/8, chunk
// l%8, so lane l fetches the logical chunk that the swizzle puts there.
// The weight fragment is MFMA operand A and the token fragment operand B, so
// each lane owns 4 consecutive output columns of one token row (8-byte stores).
//
// SWIGLU mode fuses the SwiGLU activation into the epilogue: each wave's
// weight rows are half gate rows (j) and half the matching up rows (I + j), so
// silu(gate) * up is computed from fp32 accumulators held by the same lane.
#include "dsk_internal.hpp"

#include <algorithm>
#include <cstdio>
#include <mutex>
#include <type_traits>

namespace dsk {

constexpr int kMaxGroups = 128;
constexpr int kGemmThreads = 256;
constexpr int kBK = 64;

// Tile configuration (build-time; tuned on MI355X).
#ifndef DSK_GEMM_BM
#define DSK_GEMM_BM 128
#endif
#ifndef DSK_GEMM_BN
#define DSK_GEMM_BN 256
#endif
#ifndef DSK_GEMM_WAVES_M
#define DSK_GEMM_WAVES_M 1
#endif
#ifndef DSK_GEMM_STAGES
#define DSK_GEMM_STAGES 3
#endif

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + __expf(-x)); }

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// 16-byte slot of (row, logical chunk) in a tile of 128-byte LDS rows.
__device__ __forceinline__ int lds_swz(int row, int chunk) {
  return row * 8 + (chunk ^ (row & 7) ^ ((row >> 3) & 1));
}

// Wait until at most min(ahead, MAXA) * NL vector-memory ops are pending.
template <int MAXA, int NL>
__device__ __forceinline__ void wait_stage_landed(int ahead) {
  if constexpr (MAXA <= 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= MAXA) wait_vmcnt<MAXA * NL>();
    else wait_stage_landed<MAXA - 1, NL>(ahead);
  }
}

// Workgroup barrier without the release/acquire fences of __syncthreads():
// those would wait for every in-flight DMA (vmcnt(0)) and drain the ring. The
// DMA completion this barrier publishes is waited for explicitly (wait_vmcnt)
// by every wave before it arrives; the "memory" clobber keeps the compiler
// from moving LDS accesses across the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Scheduling groups for one K step: NMFMA MFMAs with the NREAD fragment reads
// of the next step placed two after each of the first MFMAs (masks: 0x008 MFMA,
// 0x100 LDS read).
template <int NREAD, int NMFMA, int R = 0>
__device__ __forceinline__ void sched_mfma_reads() {
  constexpr int PAIRS = (NREAD + 1) / 2 < NMFMA ? (NREAD + 1) / 2 : NMFMA;
  if constexpr (R < PAIRS) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, (2 * R + 2 <= NREAD) ? 2 : 1, 0);
    sched_mfma_reads<NREAD, NMFMA, R + 1>();
  } else {
    if constexpr (NMFMA > PAIRS) __builtin_amdgcn_sched_group_barrier(0x008, NMFMA - PAIRS, 0);
    if constexpr (NREAD > 2 * PAIRS)
      __builtin_amdgcn_sched_group_barrier(0x100, NREAD - 2 * PAIRS, 0);
  }
}

// Calls f(std::integral_constant<int, min(v, N)>) for a runtime v in [0, N].
template <int N, class F>
__device__ __forceinline__ void dispatch_count(int v, F&& f) {
  if constexpr (N == 0) {
    f(std::integral_constant<int, 0>{});
  } else {
    if (v >= N) f(std::integral_constant<int, N>{});
    else dispatch_count<N - 1>(v, f);
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, bool SWIGLU>
struct GemmCfg {
  static_assert(WAVES_M * WAVES_N == 4, "4 waves per workgroup");
  static constexpr int WM = BM / WAVES_M;
  static constexpr int WN = BN / WAVES_N;
  static constexpr int TM = WM / 32;
  static constexpr int TN = WN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 block");
  static_assert(!SWIGLU || (TN % 2 == 0), "SwiGLU needs matching gate/up blocks");
  static constexpr int OUT_N = SWIGLU ? BN / 2 : BN;
  // DMA instructions per wave per stage: each moves 8 rows x 128 B
  static constexpr int A_INSTS = BM / 32;
  static constexpr int B_INSTS = BN / 32;
  static_assert(BM % 32 == 0 && BN % 32 == 0, "tile rows must be multiples of 32");
  static constexpr int A_BYTES = BM * kBK * 2;
  static constexpr int STAGE_BYTES = (BM + BN) * kBK * 2;
  static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
  static_assert(LDS_BYTES <= 150 * 1024, "LDS budget");
};

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, bool SWIGLU>
__global__ __launch_bounds__(kGemmThreads, 1) void grouped_gemm_kernel(GemmArgs p) {
  using Cfg = GemmCfg<BM, BN, WAVES_M, WAVES_N, STAGES, SWIGLU>;
  constexpr int kStages = STAGES;
  constexpr int WM = Cfg::WM, WN = Cfg::WN, TM = Cfg::TM, TN = Cfg::TN;
  constexpr int OUT_N = Cfg::OUT_N;
  constexpr int A_INSTS = Cfg::A_INSTS, B_INSTS = Cfg::B_INSTS;
  constexpr int NL = A_INSTS + B_INSTS;  // DMA instructions per thread per stage

  extern __shared__ __attribute__((aligned(1024))) uint16_t lds[];
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

  // DMA lane mapping: row l/8 of an 8-row group g = wave + 4i (so g & 1 is
  // wave & 1), logical chunk = physical chunk ^ swizzle(row)
  const int dma_row = lane >> 3;
  const int dma_chunk = (lane & 7) ^ dma_row ^ (wave & 1);
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const u32x4_t* lds4 = reinterpret_cast<const u32x4_t*>(lds);
  const int nk = p.K / kBK;

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

    // ---- per-lane DMA source rows (out-of-range rows read a valid row; their
    // results land in output rows/columns that are never stored)
    const uint16_t* a_src[A_INSTS];
#pragma unroll
    for (int i = 0; i < A_INSTS; ++i) {
      const int m = m0 + 8 * (wave + 4 * i) + dma_row;
      const int mm = m < me ? m : m0;
      int row = mm;
      if (p.a_rows != nullptr) {
        row = p.a_rows[mm];
        row = (row >= 0 && row < p.a_rows_limit) ? row : 0;
      }
      a_src[i] = p.A + (int64_t)row * p.lda + dma_chunk * 8;
    }
    const uint16_t* b_src[B_INSTS];
#pragma unroll
    for (int i = 0; i < B_INSTS; ++i) {
      const int r = 8 * (wave + 4 * i) + dma_row;
      int brow, col;
      if constexpr (SWIGLU) {
        const int wn = r / WN, w = r % WN;
        constexpr int half = WN / 2;
        col = min(n0 + wn * half + (w % half), p.N - 1);
        brow = (w < half) ? col : p.up_row_offset + col;
      } else {
        col = min(n0 + r, p.N - 1);
        brow = col;
      }
      b_src[i] = Bg + (int64_t)brow * p.ldb + dma_chunk * 8;
    }

    auto issue = [&](int stage, int kt) {
      const int koff = kt * kBK;
      const uint32_t sbase = lds_base + stage * Cfg::STAGE_BYTES;
#pragma unroll
      for (int i = 0; i < A_INSTS; ++i) {
        const uint32_t dst = sbase + (wave + 4 * i) * 1024;
        __builtin_amdgcn_global_load_lds((global_void_t*)(a_src[i] + koff),
                                         (lds_void_t*)(uintptr_t)dst, 16, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < B_INSTS; ++i) {
        const uint32_t dst = sbase + Cfg::A_BYTES + (wave + 4 * i) * 1024;
        __builtin_amdgcn_global_load_lds((global_void_t*)(b_src[i] + koff),
                                         (lds_void_t*)(uintptr_t)dst, 16, 0, 0);
      }
    };

    int tm_active = (me - (m0 + wave_m * WM) + 31) / 32;
    tm_active = max(0, min(TM, tm_active));

    floatx16_t acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

    // prologue: stages 0 .. kStages-2 in flight
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
      if (s < nk) issue(s, s);

    // K loop, specialised on the number of active 32-row blocks of this wave
    // (TMA) so the common full-tile case has no control flow around the MFMAs.
    auto mainloop = [&](auto tma_c) {
      constexpr int TMA = decltype(tma_c)::value;
      for (int kt = 0; kt < nk; ++kt) {
        // stage kt has landed when at most the loads of the stages issued after
        // it (min(kStages - 2, nk - 1 - kt) of them) are pending
        wait_stage_landed<kStages - 2, NL>(nk - 1 - kt);
        lds_barrier();
        if (kt + kStages - 1 < nk) issue((kt + kStages - 1) % kStages, kt + kStages - 1);
        if constexpr (TMA > 0) {
          const int stage = kt % kStages;
          const u32x4_t* As = lds4 + stage * (Cfg::STAGE_BYTES / 16);
          const u32x4_t* Bs = As + Cfg::A_BYTES / 16;
          // fragments of K-step kk are read into register set kk&1 while the
          // MFMAs of step kk-1 run from the other set
          bf16x8_t fb[2][TN], fa[2][TMA];
          auto read_frags = [&](int set, int kk) {
            const int ch = 2 * kk + (lane >> 5);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
              const int rr = wave_n * WN + 32 * j + (lane & 31);
              fb[set][j] = __builtin_bit_cast(bf16x8_t, Bs[lds_swz(rr, ch)]);
            }
#pragma unroll
            for (int i = 0; i < TMA; ++i) {
              const int rr = wave_m * WM + 32 * i + (lane & 31);
              fa[set][i] = __builtin_bit_cast(bf16x8_t, As[lds_swz(rr, ch)]);
            }
          };
          constexpr int KSTEPS = kBK / 16;
          constexpr int NREAD = TN + TMA;   // ds_read_b128 per K-step
          constexpr int NMFMA = TN * TMA;   // MFMAs per K-step
          read_frags(0, 0);
#pragma unroll
          for (int kk = 0; kk < KSTEPS; ++kk) {
            if (kk + 1 < KSTEPS) read_frags((kk + 1) & 1, kk + 1);
#pragma unroll
            for (int i = 0; i < TMA; ++i)
#pragma unroll
              for (int j = 0; j < TN; ++j)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[kk & 1][j], fa[kk & 1][i],
                                                                    acc[j][i], 0, 0, 0);
          }
          // schedule: step-0 reads, then each step's MFMAs with the next step's
          // reads front-loaded (two reads after each of the first MFMAs), so the
          // reads have most of the step's MFMAs to land
          __builtin_amdgcn_sched_group_barrier(0x100, NREAD, 0);
#pragma unroll
          for (int kk = 0; kk < KSTEPS; ++kk) {
            if (kk + 1 < KSTEPS) {
              sched_mfma_reads<NREAD, NMFMA>();
            } else {
              __builtin_amdgcn_sched_group_barrier(0x008, NMFMA, 0);
            }
          }
        }
      }
    };
    dispatch_count<TM>(tm_active, mainloop);
    // all waves are done reading the ring before the next tile's prologue DMA
    __syncthreads();

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

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, bool SWIGLU>
static int launch_grouped_gemm(const GemmArgs& a, hipStream_t st) {
  using Cfg = GemmCfg<BM, BN, WAVES_M, WAVES_N, STAGES, SWIGLU>;
  auto kern = grouped_gemm_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, SWIGLU>;
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
  constexpr int BM = DSK_GEMM_BM, BN = DSK_GEMM_BN, WAVES_M = DSK_GEMM_WAVES_M;
  constexpr int STAGES = DSK_GEMM_STAGES;
  if (swiglu) return launch_grouped_gemm<BM, BN, WAVES_M, 4 / WAVES_M, STAGES, true>(a, st);
  return launch_grouped_gemm<BM, BN, WAVES_M, 4 / WAVES_M, STAGES, false>(a, st);
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
