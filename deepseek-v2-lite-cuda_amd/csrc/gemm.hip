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
// M-tiles that share a weight tile run at about the same time on the same XCD,
// so the weight tile is mostly re-read from that XCD's L2.
//
// Data movement: each workgroup runs one continuous stream of K stages over
// all of its tiles. A stage (BM token rows + BN weight rows, BK deep) lands in
// a ring of STAGES LDS buffers through direct global->LDS DMA
// (global_load_lds_dwordx4, no register staging), issued STAGES-1 stages
// ahead, so the next tile's first stage is in flight while the current one
// finishes and writes its epilogue. One workgroup barrier per stage, placed
// before the last K step: that step's MFMAs then overlap the next stage's
// first fragment reads and the refill DMA of the buffer just released.
//
// The L2->CU path (~48 B/clk per CU measured, for DMA and vector loads alike)
// and its latency, rather than the matrix cores, bound this kernel at small
// tiles, so tiles are as large as the accumulators allow: 256 tokens x 256
// weight rows (128 flops per byte moved), 8 waves of 128 x 64 (two per SIMD,
// so one wave's MFMAs cover the other's waits), BK = 64 so every DMA row is a
// whole 128-byte line, and a 2-deep ring (2 x 64 KB of the 160 KB LDS).
//
// LDS rows are BK*2 bytes with a 16-byte-chunk XOR swizzle chosen so the 16
// lanes that the 64-bank LDS serves together (16 rows, one logical chunk of a
// fragment read) hit 16 distinct bank quads. A DMA instruction writes 1 KB
// (64 lanes x 16 B) = 1024 / (BK*2) rows; lane l lands at a fixed physical
// slot, so it fetches the logical chunk the swizzle puts there.
// The weight fragment is MFMA operand A and the token fragment operand B, so
// each lane owns 4 consecutive output columns of one token row (8-byte stores).
// Partial M tiles skip the MFMAs of 32-row blocks past the group end; the
// variant (all blocks, half, none) is chosen once per tile so the K loop itself
// has no data-dependent branches around the accumulators.
//
// SWIGLU mode fuses the SwiGLU activation into the epilogue: each wave's
// weight rows are half gate rows (j) and half the matching up rows (I + j), so
// silu(gate) * up is computed from fp32 accumulators held by the same lane.
#include "dsk_internal.hpp"
#include "gemm_sched.hpp"
#include "route_token.hpp"

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <mutex>
#include <type_traits>

namespace dsk {

constexpr int kMaxGroups = 128;
constexpr int kLdsPerCU = 160 * 1024;

// Tile configuration (build-time; tuned on MI355X).
#ifndef DSK_GEMM_BM
#define DSK_GEMM_BM 256
#endif
#ifndef DSK_GEMM_BN
#define DSK_GEMM_BN 256
#endif
#ifndef DSK_GEMM_WAVES_M
#define DSK_GEMM_WAVES_M 2
#endif
#ifndef DSK_GEMM_WAVES_N
#define DSK_GEMM_WAVES_N 4
#endif
#ifndef DSK_GEMM_BK
#define DSK_GEMM_BK 64
#endif
#ifndef DSK_GEMM_STAGES
#define DSK_GEMM_STAGES 2
#endif

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// silu(x) = x / (1 + e^-x) with the hardware reciprocal (1 ulp), ample for a
// result that is rounded to bf16.
__device__ __forceinline__ float silu_f(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __expf(-x));
}

// Reads an accumulator register where it is used: the epilogue then moves
// the accumulators to VGPRs a few at a time instead of all at once.
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
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

// Calls f(std::integral_constant<int, n>) for the runtime value n in [0, N].
template <int N, typename F>
__device__ __forceinline__ void dispatch_active(int n, F&& f) {
  if constexpr (N == 0) {
    f(std::integral_constant<int, 0>{});
  } else {
    if (n >= N) f(std::integral_constant<int, N>{});
    else dispatch_active<N - 1>(n, f);
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int BK, int STAGES, bool SWIGLU>
struct GemmCfg {
  static constexpr int NW = WAVES_M * WAVES_N;  // waves per workgroup
  static_assert(NW == 4 || NW == 8, "4 or 8 waves per workgroup");
  static constexpr int THREADS = 64 * NW;
  static_assert(BK == 32 || BK == 64, "BK is 32 or 64");
  static_assert(STAGES >= 2, "the stage stream needs at least 2 LDS buffers");
  static constexpr int WM = BM / WAVES_M;
  static constexpr int WN = BN / WAVES_N;
  static constexpr int TM = WM / 32;
  static constexpr int TN = WN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 block");
  static_assert(!SWIGLU || (TN % 2 == 0), "SwiGLU needs matching gate/up blocks");
  static constexpr int OUT_N = SWIGLU ? BN / 2 : BN;
  static constexpr int CPR = BK / 8;        // 16-byte chunks per LDS row
  static constexpr int RPI = 64 / CPR;      // rows per 1 KB DMA instruction
  // DMA is issued by NI waves only, one per SIMD: a wave stalls while the
  // address unit drains its DMA instructions, and the second wave on the SIMD
  // keeps the matrix core busy meanwhile. The issuers are the last NI waves
  // (the highest wave_m): a partial M tile fills the first waves' rows first,
  // so the issuing waves have the fewest MFMAs.
  static constexpr int NI = 4;
  static constexpr int A_INSTS = BM / (NI * RPI);  // DMA instructions per issuing wave per stage
  static constexpr int B_INSTS = BN / (NI * RPI);
  static_assert(A_INSTS * NI * RPI == BM && B_INSTS * NI * RPI == BN, "tile rows vs DMA rows");
  static constexpr int KSTEPS = BK / 16;
  static constexpr int A_BYTES = BM * BK * 2;
  static constexpr int STAGE_BYTES = (BM + BN) * BK * 2;
  static constexpr int RING_BYTES = STAGES * STAGE_BYTES;
  // tiles per workgroup whose gathered A row indices fit in the LDS left over
  // (4 KB kept for the group table and alignment)
  static constexpr int ROW_TILES = (kLdsPerCU - RING_BYTES - 4096) / (BM * 4);
  static_assert(ROW_TILES >= 1, "no LDS left for the row table");
  static constexpr int LDS_BYTES = RING_BYTES + ROW_TILES * BM * 4;  // dynamic LDS
};

// 16-byte slot of (row, logical chunk) in a tile of CPR-chunk LDS rows.
template <int CPR>
__device__ __forceinline__ int lds_swz(int row, int chunk) {
  if constexpr (CPR == 8) return row * 8 + (chunk ^ (row & 7) ^ ((row >> 3) & 1));
  else return row * 4 + (chunk ^ ((row >> 2) & 3));
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int BK, int STAGES, bool SWIGLU,
          bool GATHER, bool TILED>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1) void grouped_gemm_kernel(GemmArgs p) {
  using Cfg = GemmCfg<BM, BN, WAVES_M, WAVES_N, BK, STAGES, SWIGLU>;
  constexpr int kStages = STAGES;
  constexpr int WM = Cfg::WM, WN = Cfg::WN, TM = Cfg::TM, TN = Cfg::TN;
  constexpr int OUT_N = Cfg::OUT_N;
  constexpr int CPR = Cfg::CPR, RPI = Cfg::RPI;
  constexpr int A_INSTS = Cfg::A_INSTS, B_INSTS = Cfg::B_INSTS;
  constexpr int NL = A_INSTS + B_INSTS;  // DMA instructions per issuing wave per stage
  constexpr int NI = Cfg::NI;
  constexpr int KSTEPS = Cfg::KSTEPS;
  constexpr int NW = Cfg::NW;

  extern __shared__ __attribute__((aligned(1024))) uint16_t lds[];
  __shared__ int s_inc[kMaxGroups];
  __shared__ int s_mb[kMaxGroups];
  __shared__ int s_me[kMaxGroups];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a uniform (scalar) value, so per-wave decisions are branches
  // rather than exec-masked code
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wave_m = wave / WAVES_N;
  const int wave_n = wave % WAVES_N;
  const int G = p.offsets != nullptr ? p.G : 1;
  const int NT = (p.N + OUT_N - 1) / OUT_N;

  // ---- group table: row ranges and inclusive prefix of tile counts. A
  // group of n rows is cut into mt = ceil(n / BM) M tiles of equal size (in
  // 32-row blocks, +-1 block), so the M tiles that share a weight tile
  // progress at the same rate and read it from L2 together.
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
  const int total_tiles = s_inc[G - 1];

  // ---- XCD-aware persistent enumeration (gemm_sched.hpp): tiles dealt to the
  // 8 XCDs in chunks, so the M tiles of one weight tile stay on one XCD
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int per_xcd = gridDim.x >> 3;
  const int chunk = sched_chunk(p.chunk_m_tiles, NT);
  const int ntiles = sched_slot_tiles(sched_xcd_tiles(total_tiles, xcd, chunk), slot, per_xcd);
  if (ntiles == 0) return;  // uniform: no work for this workgroup
  const int nk = p.K / BK;
  const int total = ntiles * nk;  // stages in this workgroup's stream

  struct Tile {
    int g, m0, me, n0;  // rows [m0, me) of group g, output columns from n0
  };
  auto decode = [&](int t) -> Tile {
    const int W = sched_tile_index(xcd, slot, t, per_xcd, chunk);
    int lo = 0, hi = G - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_inc[mid] > W) hi = mid; else lo = mid + 1;
    }
    const int local = W - (lo > 0 ? s_inc[lo - 1] : 0);
    const int mb = s_mb[lo], gme = s_me[lo];
    const int mt = (gme - mb + BM - 1) / BM;
    const int nblk = (gme - mb + 31) / 32;
    int nt, mi;
    sched_group_tile(local, mt, NT, &nt, &mi);
    const int m0 = mb + 32 * (mi * nblk / mt);
    const int me = min(mb + 32 * ((mi + 1) * nblk / mt), gme);
    return Tile{lo, m0, me, nt * OUT_N};
  };

  // DMA lane mapping: lane l lands at row l / CPR of its instruction's row group
  // (RPI rows; group index islot + NI*i), physical chunk l % CPR
  const int islot = wave - (NW - NI);  // issuing slot 0 .. NI-1, negative if not issuing
  const int dma_row = lane / CPR;
  int dma_chunk;
  if constexpr (CPR == 8) dma_chunk = (lane & 7) ^ dma_row ^ (islot & 1);
  else dma_chunk = (lane & 3) ^ ((lane >> 4) & 3);
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const u32x4_t* lds4 = reinterpret_cast<const u32x4_t*>(lds);
  const int row_limit = GATHER ? p.a_rows_limit : p.M;

  // Gathered A rows: the row indices of all of this workgroup's tiles are
  // staged once in the LDS past the ring, so the per-tile lookups are LDS reads
  // (a vector load here would make its first use wait for every DMA issued
  // before it). The launcher sizes the grid so that ntiles <= ROW_TILES.
  // Rows past a group's end read a valid row whose results are never stored.
  int* s_rows = reinterpret_cast<int*>(lds + Cfg::RING_BYTES / 2);
  if constexpr (GATHER) {
    if (ntiles > Cfg::ROW_TILES) return;  // excluded by the launcher
    for (int idx = tid; idx < ntiles * BM; idx += Cfg::THREADS) {
      const Tile t = decode(idx / BM);
      const int m = t.m0 + idx % BM;
      s_rows[idx] = p.a_rows[m < t.me ? m : t.m0];
    }
    __syncthreads();
  }

  // ---- issue side of the stage stream (waves 0 .. NI-1). Sources are kept
  // as 32-bit byte offsets from uniform bases (A, and the tile's weight group),
  // one VGPR each.
  const bool issuer = islot >= 0;
  uint32_t a_off[A_INSTS], b_off[B_INSTS];
  const char* Bg = reinterpret_cast<const char*>(p.B);
  auto set_sources = [&](int t_idx, const Tile& t) {
    Bg = reinterpret_cast<const char*>(p.B + (int64_t)t.g * p.b_group_stride);
    if (!issuer) return;
#pragma unroll
    for (int i = 0; i < A_INSTS; ++i) {
      const int r = RPI * (islot + NI * i) + dma_row;
      int row;
      if constexpr (GATHER) {
        row = s_rows[t_idx * BM + r];
      } else {
        const int m = t.m0 + r;
        row = m < t.me ? m : t.m0;
      }
      row = (row >= 0 && row < row_limit) ? row : 0;
      a_off[i] = (uint32_t)(((int64_t)row * p.lda + dma_chunk * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < B_INSTS; ++i) {
      if constexpr (TILED) {
        // one 1 KB fragment (32 weight rows x 16 k) per instruction: local
        // fragment f = row block * (BK/16) + k step
        const int f = islot + NI * i;
        const int rbl = f / (BK / 16), ksl = f % (BK / 16);
        int rb;
        if constexpr (SWIGLU) {
          const int wn = rbl / TN, wb = rbl % TN;
          const int cb = min(t.n0 / 32 + wn * (TN / 2) + wb % (TN / 2), p.N / 32 - 1);
          rb = wb < TN / 2 ? cb : p.up_row_offset / 32 + cb;
        } else {
          rb = min(t.n0 / 32 + rbl, p.N / 32 - 1);
        }
        b_off[i] = (uint32_t)((((int64_t)rb * (p.K / 16) + ksl) * 512 + lane * 8) * 2);
      } else {
        const int r = RPI * (islot + NI * i) + dma_row;
        int brow, col;
        if constexpr (SWIGLU) {
          const int wn = r / WN, w = r % WN;
          constexpr int half = WN / 2;
          col = min(t.n0 + wn * half + (w % half), p.N - 1);
          brow = (w < half) ? col : p.up_row_offset + col;
        } else {
          col = min(t.n0 + r, p.N - 1);
          brow = col;
        }
        b_off[i] = (uint32_t)(((int64_t)brow * p.ldb + dma_chunk * 8) * 2);
      }
    }
  };
  auto issue = [&](int stage, int kt) {
    if (!issuer) return;
    const uint32_t koff = (uint32_t)kt * BK * 2;  // bytes
    // tiled weights: a stage is BK/16 consecutive fragments of 1 KB
    const uint32_t bkoff = TILED ? (uint32_t)kt * (BK / 16) * 1024 : koff;
    const uint32_t sbase = lds_base + stage * Cfg::STAGE_BYTES;
    const char* A = reinterpret_cast<const char*>(p.A);
#pragma unroll
    for (int i = 0; i < A_INSTS; ++i) {
      const uint32_t dst = sbase + (islot + NI * i) * 1024;
      __builtin_amdgcn_global_load_lds((global_void_t*)(A + (a_off[i] + koff)),
                                       (lds_void_t*)(uintptr_t)dst, 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_INSTS; ++i) {
      const uint32_t dst = sbase + Cfg::A_BYTES + (islot + NI * i) * 1024;
      __builtin_amdgcn_global_load_lds((global_void_t*)(Bg + (b_off[i] + bkoff)),
                                       (lds_void_t*)(uintptr_t)dst, 16, 0, 0);
    }
  };

  int is_tile = 0;      // tile whose stages are being issued
  int is_kt = 0;        // its next stage
  int gs_issue = 0;     // stages issued so far
  set_sources(0, decode(0));
  // Issues the next stage of the stream (if any), switching the DMA sources to
  // the next tile after a tile's last stage.
  auto issue_next = [&]() {
    if (gs_issue >= total) return;
    issue(gs_issue % kStages, is_kt);
    ++gs_issue;
    if (++is_kt == nk) {
      is_kt = 0;
      if (++is_tile < ntiles) set_sources(is_tile, decode(is_tile));
    }
  };

  // ---- compute side
  floatx16_t acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

  bf16x8_t fb[2][TN], fa[2][TM];
  auto read_frags = [&](int set, int stage, int kk) {
    const u32x4_t* As = lds4 + stage * (Cfg::STAGE_BYTES / 16);
    const u32x4_t* Bs = As + Cfg::A_BYTES / 16;
    const int ch = 2 * kk + (lane >> 5);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (TILED) {
        fb[set][j] = __builtin_bit_cast(
            bf16x8_t, Bs[((wave_n * TN + j) * (BK / 16) + kk) * 64 + lane]);
      } else {
        const int rr = wave_n * WN + 32 * j + (lane & 31);
        fb[set][j] = __builtin_bit_cast(bf16x8_t, Bs[lds_swz<CPR>(rr, ch)]);
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int rr = wave_m * WM + 32 * i + (lane & 31);
      fa[set][i] = __builtin_bit_cast(bf16x8_t, As[lds_swz<CPR>(rr, ch)]);
    }
  };

  auto active_blocks = [&](const Tile& t) {
    return max(0, min(TM, (t.me - (t.m0 + wave_m * WM) + 31) / 32));
  };

  // prologue: STAGES stages in flight, stage 0 landed, its first fragments read
#pragma unroll 1
  for (int s = 0; s < kStages; ++s) issue_next();
  wait_stage_landed<kStages - 1, NL>(gs_issue - 1);
  lds_barrier();
  read_frags(0, 0, 0);

  int gc = 0;  // stages consumed
  Tile ct = decode(0);
#pragma unroll 1
  for (int ct_idx = 0; ct_idx < ntiles; ++ct_idx) {
    const int tma = active_blocks(ct);
    // The K loop of one tile, for TMA active 32-row blocks of this wave (the
    // blocks past the tile's rows are skipped). The variant is chosen per
    // tile, so the accumulators never merge between variants inside the loop.
    auto run_tile = [&](auto tma_c) {
      constexpr int TMA = decltype(tma_c)::value;
      constexpr int NREAD = TN + TM;
      constexpr int NMFMA = TN * TMA;
#pragma unroll 1
      for (int kt = 0; kt < nk; ++kt, ++gc) {
        const int stage = gc % kStages;
        // K steps 0 .. KSTEPS-2: MFMAs of step kk, fragments of step kk+1
#pragma unroll
        for (int kk = 0; kk + 1 < KSTEPS; ++kk) {
          read_frags((kk + 1) & 1, stage, kk + 1);
#pragma unroll
          for (int i = 0; i < TMA; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[kk & 1][j], fa[kk & 1][i],
                                                                  acc[j][i], 0, 0, 0);
        }
#pragma unroll
        for (int kk = 0; kk + 1 < KSTEPS; ++kk) sched_mfma_reads<NREAD, NMFMA>();
        // Stage gc+1 must have landed (only later stages may be pending) and
        // every wave must be done reading this stage's buffer before it is
        // refilled with stage gc+STAGES.
        if (gc + 1 < total) {
          wait_stage_landed<kStages - 2, NL>(total - gc - 2);
          __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads done
          lds_barrier();
          issue_next();
        }
        // last K step's MFMAs overlap the next stage's first fragment reads
        // (after the last stage these are harmless, in-bounds LDS reads)
        read_frags(0, (gc + 1) % kStages, 0);
#pragma unroll
        for (int i = 0; i < TMA; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                fb[(KSTEPS - 1) & 1][j], fa[(KSTEPS - 1) & 1][i], acc[j][i], 0, 0, 0);
        sched_mfma_reads<NREAD, NMFMA>();
      }
    };
    dispatch_active<TM>(tma, run_tile);

    // ---- epilogue (the next tile's first stages are already in flight):
    // lane owns token row m = ... + (lane & 31) and 4 consecutive output
    // columns per 4-register group; lanes l and l + 32 hold the same row.
    // One lane-half swap per pair of groups gives lane l columns 0-7 and
    // lane l + 32 columns 8-15 of a 16-column run, so each store instruction
    // writes 16 contiguous bytes per row instead of 8.
    {
      constexpr int JN = SWIGLU ? TN / 2 : TN;
      constexpr int WOUT = SWIGLU ? WN / 2 : WN;
      const bool vec16 = (reinterpret_cast<uintptr_t>(p.C) & 15) == 0 && (p.ldc & 7) == 0;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if (i >= tma) continue;
        const int m = ct.m0 + wave_m * WM + 32 * i + (lane & 31);
        if (m >= ct.me) continue;  // the same for lanes l and l + 32
        uint16_t* crow = p.C + (int64_t)m * p.ldc;
#pragma unroll
        for (int j = 0; j < JN; ++j) {
#pragma unroll
          for (int q2 = 0; q2 < 2; ++q2) {
            uint32_t w[2][2];  // [group 2*q2 + h][packed column pair]
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int qg = 2 * q2 + h;
              float v[4];
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                if constexpr (SWIGLU)
                  v[c] = silu_f(acc_read(acc[j][i][4 * qg + c])) *
                         acc_read(acc[j + TN / 2][i][4 * qg + c]);
                else
                  v[c] = acc_read(acc[j][i][4 * qg + c]);
              }
              w[h][0] = pack_bf16x2(v[0], v[1]);
              w[h][1] = pack_bf16x2(v[2], v[3]);
            }
            // upper lanes of w[0] <-> lower lanes of w[1]
#pragma unroll
            for (int d = 0; d < 2; ++d) {
              const auto r = __builtin_amdgcn_permlane32_swap(w[0][d], w[1][d], false, false);
              w[0][d] = r[0];
              w[1][d] = r[1];
            }
            const int nb = ct.n0 + wave_n * WOUT + 32 * j + 16 * q2 + 8 * (lane >> 5);
            if (nb + 7 < p.N) {
              if (vec16) {
                const u32x4_t o = {w[0][0], w[0][1], w[1][0], w[1][1]};
                *reinterpret_cast<u32x4_t*>(crow + nb) = o;
              } else {
                const u32x2_t lo = {w[0][0], w[0][1]}, hi = {w[1][0], w[1][1]};
                *reinterpret_cast<u32x2_t*>(crow + nb) = lo;
                *reinterpret_cast<u32x2_t*>(crow + nb + 4) = hi;
              }
            } else {
#pragma unroll
              for (int c = 0; c < 8; ++c)
                if (nb + c < p.N)
                  crow[nb + c] = static_cast<uint16_t>(w[c >> 2][(c >> 1) & 1] >> (16 * (c & 1)));
            }
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;
    if (ct_idx + 1 < ntiles) ct = decode(ct_idx + 1);
  }
}

// ------------------------------------------- large groups, tiled weights ----
// Grouped GEMM for fragment-tiled weights, one wave per SIMD. A tile is 256
// token rows x 256 weight rows; each of the 4 waves owns 64 weight rows (two
// 32-row fragments) against all 256 token rows: 8 x 2 blocks of 32 x 32, 256
// fp32 accumulators per lane in the accumulator registers.
//   * Weights go straight from HBM/L2 into registers, two stages (128 K)
//     ahead of their use: a wave's weight rows belong to it alone, and a
//     tiled fragment is one contiguous 1 KB load in MFMA lane order.
//   * Only the token rows go through the LDS: a 4-deep ring of 32 KB stages
//     (256 rows x 64 K) filled by direct global->LDS DMA three stages ahead,
//     read back as 8 fragments per K step by every wave.
//   * Every memory operation of a stage (8 weight loads, 8 DMA instructions
//     per wave) is spread over the stage's MFMAs, so no wave stalls on a burst
//     of issue and the matrix core of each SIMD is fed by a single wave.
//   * One workgroup barrier per stage; all 4 waves do the same work, so no
//     wave waits for another's extra MFMAs.
// The issue cursors (tokens three stages ahead, weights two) run over the
// tile stream of the workgroup, so the next tile's first stages are in flight
// during the epilogue. Past the end of the stream they repeat the last valid
// stage (into a ring slot and registers nobody reads again), which keeps the
// number of memory operations per stage fixed for the vmcnt bookkeeping.
constexpr int kWideWaves = 4;
constexpr int kWideBM = 256;                           // token rows per tile
constexpr int kWideBK = 64;                            // K per stage
constexpr int kWideRing = 4;                           // token stages in the LDS ring
constexpr int kWideStageBytes = kWideBM * kWideBK * 2;  // 32 KB
constexpr int kWideRingBytes = kWideRing * kWideStageBytes;
constexpr int kWideRowTiles = (kLdsPerCU - kWideRingBytes - 4096) / (kWideBM * 4);
constexpr int kWideLdsBytes = kWideRingBytes + kWideRowTiles * kWideBM * 4;
constexpr int kRowScaleParts = 2;  // sum-of-squares partials an RMS row scale adds up


template <bool SWIGLU, bool GATHER>
__global__ __launch_bounds__(64 * kWideWaves, 1) void wide_gemm_kernel(GemmArgs p) {
  constexpr int TM = kWideBM / 32;     // token blocks per tile
  constexpr int TN = 2;                // weight blocks per wave
  constexpr int KSTEPS = kWideBK / 16;
  constexpr int OUT_N = SWIGLU ? 32 * kWideWaves : 64 * kWideWaves;  // output columns per tile
  constexpr int RPI = 8;               // token rows per 1 KB DMA instruction
  constexpr int A_INSTS = kWideBM / (kWideWaves * RPI);  // per wave per stage
  static_assert(A_INSTS == 2 * KSTEPS, "two DMA instructions per K step");
  constexpr int THREADS = 64 * kWideWaves;

  extern __shared__ __attribute__((aligned(1024))) uint16_t lds[];
  __shared__ int s_inc[kMaxGroups];
  __shared__ int s_mb[kMaxGroups];
  __shared__ int s_me[kMaxGroups];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = p.offsets != nullptr ? p.G : 1;
  const int NT = (p.N + OUT_N - 1) / OUT_N;

  // ---- group table (as in grouped_gemm_kernel): row ranges, even M split
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
      cnt = ((me - mb + kWideBM - 1) / kWideBM) * NT;
    }
    s_inc[tid] = wave_inclusive_scan(cnt);
  }
  __syncthreads();
  const int carry = s_inc[63];
  __syncthreads();
  if (tid >= 64 && tid < kMaxGroups) s_inc[tid] += carry;
  __syncthreads();
  const int total_tiles = s_inc[G - 1];

  // ---- XCD-aware persistent enumeration (as in grouped_gemm_kernel)
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int per_xcd = gridDim.x >> 3;
  const int chunk = sched_chunk(p.chunk_m_tiles, NT);
  const int ntiles = sched_slot_tiles(sched_xcd_tiles(total_tiles, xcd, chunk), slot, per_xcd);
  if (ntiles == 0) return;
  const int nk = p.K / kWideBK;  // even (K % 128 == 0, checked by the launcher)
  const int total = ntiles * nk;

  struct Tile {
    int g, m0, me, n0;
  };
  auto decode = [&](int t) -> Tile {
    const int W = sched_tile_index(xcd, slot, t, per_xcd, chunk);
    int lo = 0, hi = G - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_inc[mid] > W) hi = mid; else lo = mid + 1;
    }
    const int local = W - (lo > 0 ? s_inc[lo - 1] : 0);
    const int mb = s_mb[lo], gme = s_me[lo];
    const int mt = (gme - mb + kWideBM - 1) / kWideBM;
    const int nblk = (gme - mb + 31) / 32;
    int nt, mi;
    sched_group_tile(local, mt, NT, &nt, &mi);
    const int m0 = mb + 32 * (mi * nblk / mt);
    const int me = min(mb + 32 * ((mi + 1) * nblk / mt), gme);
    return Tile{lo, m0, me, nt * OUT_N};
  };

  const int dma_row = lane >> 3;
  const int dma_chunk = (lane & 7) ^ dma_row ^ (wave & 1);  // row group wave + 4i: parity wave
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const u32x4_t* lds4 = reinterpret_cast<const u32x4_t*>(lds);
  const int row_limit = GATHER ? p.a_rows_limit : p.M;

  int* s_rows = reinterpret_cast<int*>(lds + kWideRingBytes / 2);
  if constexpr (GATHER) {
    if (ntiles > kWideRowTiles) return;  // excluded by the launcher
    for (int idx = tid; idx < ntiles * kWideBM; idx += THREADS) {
      const Tile t = decode(idx / kWideBM);
      const int m = t.m0 + idx % kWideBM;
      s_rows[idx] = p.a_rows[m < t.me ? m : t.m0];
    }
    __syncthreads();
  }

  // ---- token DMA cursor (three stages ahead of consumption)
  const char* Abase = reinterpret_cast<const char*>(p.A);
  uint32_t a_off[A_INSTS];
  int a_gs = 0, a_tile = 0, a_kt = 0;
  auto set_a = [&](int t_idx) {
    const Tile t = decode(t_idx);
#pragma unroll
    for (int i = 0; i < A_INSTS; ++i) {
      const int r = RPI * (wave + kWideWaves * i) + dma_row;
      int row;
      if constexpr (GATHER) {
        row = s_rows[t_idx * kWideBM + r];
      } else {
        const int m = t.m0 + r;
        row = m < t.me ? m : t.m0;
      }
      row = (row >= 0 && row < row_limit) ? row : 0;
      a_off[i] = (uint32_t)(((int64_t)row * p.lda + dma_chunk * 8) * 2);
    }
  };
  // DMA instructions i0, i0+1 of stage a_gs (ring slot a_gs % kWideRing)
  auto issue_a = [&](int i0) {
    const uint32_t koff = (uint32_t)a_kt * kWideBK * 2;
    const uint32_t dst = lds_base + (a_gs % kWideRing) * kWideStageBytes;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = i0 + u;
      dma_1kb(Abase, a_off[i] + koff, dst + (wave + kWideWaves * i) * 1024);
    }
  };
  auto advance_a = [&]() {
    ++a_gs;
    if (a_gs < total && ++a_kt == nk) {
      a_kt = 0;
      set_a(++a_tile);
    }
  };

  // ---- weight cursor (two stages ahead): fragment (rb, k step) of the tile's
  // group at byte ((rb * K/16 + ks) * 512 + lane * 8) * 2
  const char* b_grp = reinterpret_cast<const char*>(p.B);
  uint32_t b_off[TN];
  int b_gs = 0, b_tile = 0, b_kt = 0;
  auto set_b = [&](int t_idx) {
    const Tile t = decode(t_idx);
    b_grp = reinterpret_cast<const char*>(p.B + (int64_t)t.g * p.b_group_stride);
    const int last = p.N / 32 - 1;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      int rb;
      if constexpr (SWIGLU) {
        const int ob = min(t.n0 / 32 + wave, last);   // output block of this wave
        rb = j == 0 ? ob : p.up_row_offset / 32 + ob;  // gate rows, then up rows
      } else {
        rb = min(t.n0 / 32 + TN * wave + j, last);
      }
      b_off[j] = (uint32_t)((((int64_t)rb * (p.K / 16)) * 512 + lane * 8) * 2);
    }
  };
  auto issue_b = [&](bf16x8_t (&dst)[TN], int k) {
    const uint32_t koff = (uint32_t)(b_kt * KSTEPS + k) * 1024;
#pragma unroll
    for (int j = 0; j < TN; ++j)
      dst[j] = *reinterpret_cast<const bf16x8_t*>(b_grp + (b_off[j] + koff));
  };
  auto advance_b = [&]() {
    ++b_gs;
    if (b_gs < total && ++b_kt == nk) {
      b_kt = 0;
      set_b(++b_tile);
    }
  };

  bf16x8_t fb[2][KSTEPS][TN];  // weight fragments, register set = stage parity
  bf16x8_t fa[2][TM];          // token fragments, double-buffered by K step
  floatx16_t acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

  auto read_a = [&](bf16x8_t (&dst)[TM], int slot_idx, int kk) {
    const u32x4_t* As = lds4 + slot_idx * (kWideStageBytes / 16);
    const int ch = 2 * kk + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i)
      dst[i] = __builtin_bit_cast(bf16x8_t, As[lds_swz<8>(32 * i + (lane & 31), ch)]);
  };

  // ---- prologue: tokens of stages 0-2 and weights of stages 0-1 in flight
  // (order A0 B0 A1 B1 A2: 40 operations per wave), stage 0 landed
  set_a(0);
  set_b(0);
#pragma unroll
  for (int s = 0; s < 3; ++s) {
#pragma unroll
    for (int i = 0; i < A_INSTS; i += 2) issue_a(i);
    advance_a();
    if (s < 2) {
#pragma unroll
      for (int k = 0; k < KSTEPS; ++k) issue_b(fb[s][k], k);
      advance_b();
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt<4 * A_INSTS>();  // everything after A0 may be pending
  lds_barrier();
  read_a(fa[0], 0, 0);

  int gc = 0;  // stages consumed
  Tile ct = decode(0);
#pragma unroll 1
  for (int ct_idx = 0; ct_idx < ntiles; ++ct_idx) {
    // active 32-row token blocks of this tile (uniform). Blocks 0..TM/2-1 are
    // always computed (rows past the tile end are never stored); the others
    // sit behind uniform branches. A copy of the K loop per block count would
    // merge 256 live accumulators at the branch and overflow the registers.
    const int tma = max(1, min(TM, (ct.me - ct.m0 + 31) / 32));
    // Sum-of-squares partials of this tile's token rows (row ct.m0 + 32 i +
    // lane % 32) for the RMS row scale, loaded now and only added up in the
    // epilogue: a use here would make the wave wait for every DMA issued
    // before these loads (the wait counts complete in order).
    float rsc[TM][kRowScaleParts];
    if constexpr (!SWIGLU && !GATHER) {
      if (p.rowscale_ss != nullptr) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = min(ct.m0 + 32 * i + (lane & 31), p.M - 1);
#pragma unroll
          for (int q = 0; q < kRowScaleParts; ++q)
            rsc[i][q] = p.rowscale_ss[min(q, p.rowscale_parts - 1) * p.ld_rowscale + m];
        }
      }
    }
    {
      // one stage: K steps 0..3 on weight set SET; the barrier before the last
      // step publishes the next stage's tokens and frees this stage's slot
      auto stage = [&](auto set_c) {
        constexpr int SET = decltype(set_c)::value;
        const int slot_now = gc % kWideRing;
#pragma unroll
        for (int k = 0; k < KSTEPS; ++k) {
          if (k == KSTEPS - 1) {
            // stage gc+1's tokens landed. Per K step the order is 2 DMA, then 2
            // weight loads, so in steady state 30 operations were issued after
            // the last DMA of that stage (its step's 2 weight loads, one stage
            // of 16, three steps of 4); after the prologue (A0 B0 A1 B1 A2) only
            // 28 follow A1 and A2. 28 is exact there and safe everywhere.
            __builtin_amdgcn_sched_barrier(0);  // no memory operation crosses the count
            wait_vmcnt<16 + 12>();
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): own LDS reads done
            lds_barrier();
            read_a(fa[(k + 1) & 1], (gc + 1) % kWideRing, 0);
          } else {
            read_a(fa[(k + 1) & 1], slot_now, k + 1);
          }
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            if (i < TM / 2 || i < tma) {
#pragma unroll
              for (int j = 0; j < TN; ++j)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[SET][k][j], fa[k & 1][i],
                                                                    acc[j][i], 0, 0, 0);
            }
          }
          issue_a(2 * k);
          issue_b(fb[SET][k], k);
        }
        advance_a();
        advance_b();
        ++gc;
      };
#pragma unroll 1
      for (int kt = 0; kt < nk; kt += 2) {
        stage(std::integral_constant<int, 0>{});
        stage(std::integral_constant<int, 1>{});
      }
    }

    // ---- epilogue through the LDS. A lane holds token row (lane & 31) of
    // each 32-row block and 4 consecutive columns per 4-register group, so
    // direct stores would touch 32 rows per instruction with 8 bytes each.
    // Instead each wave stages one block of its output (64 columns = 128 B
    // per row; SwiGLU: 32 columns = 64 B) in its own 4 KB of the ring slot
    // just consumed, and reads it back so that CHUNKS consecutive lanes hold
    // one row segment: every store instruction writes whole row segments.
    // The slot is free until the next tile's DMA, which the barrier after
    // the epilogue holds back. The staging swizzle (16-byte chunk XOR row
    // bits, 8-byte half XOR row bit 4) keeps the 8-byte writes and the
    // 16-byte reads free of bank conflicts.
    {
      constexpr int ROW_BYTES = SWIGLU ? 64 : 128;
      constexpr int CHUNKS = ROW_BYTES / 16;
      constexpr int ROWS_PER_INST = 64 / CHUNKS;
      constexpr int JN = SWIGLU ? 1 : TN;
      auto swz = [](int row) { return SWIGLU ? (row >> 2) & 3 : (row >> 1) & 7; };
      char* stage_lds = reinterpret_cast<char*>(lds) + ((gc - 1) % kWideRing) * kWideStageBytes +
                        wave * 4096;
      const int r32 = lane & 31, h = lane >> 5;
      const int col0 = SWIGLU ? ct.n0 + 32 * wave : ct.n0 + 64 * wave;  // this wave's columns
      const int rl = lane / CHUNKS, cl = lane % CHUNKS;
      constexpr bool kRowOps = !SWIGLU && !GATHER;
      const bool scale_rows = kRowOps && p.rowscale_ss != nullptr;
      // whole tile inside the sum-of-squares column range (256-aligned bounds)
      const bool sum_rows = kRowOps && p.rowsq_out != nullptr && ct.n0 >= p.rowsq_c0 &&
                            ct.n0 < p.rowsq_c1;
      // per-wave row partials of the sums of squares, behind the ring (the
      // gathered kernels' row table, unused here)
      float* s_ss = reinterpret_cast<float*>(lds + kWideRingBytes / 2);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if (i >= tma) continue;
        float rs = 1.f;
        if constexpr (kRowOps) {
          if (scale_rows) {
            float ss = rsc[i][0];
#pragma unroll
            for (int q = 1; q < kRowScaleParts; ++q)
              if (q < p.rowscale_parts) ss += rsc[i][q];
            rs = rsqrtf(ss * (1.f / p.rowscale_cols) + p.rowscale_eps);
          }
        }
#pragma unroll
        for (int j = 0; j < JN; ++j) {
#pragma unroll
          for (int qg = 0; qg < 4; ++qg) {
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              if constexpr (SWIGLU)
                v[c] = silu_f(acc_read(acc[0][i][4 * qg + c])) * acc_read(acc[1][i][4 * qg + c]);
              else
                v[c] = acc_read(acc[j][i][4 * qg + c]) * rs;
            }
            u32x2_t o;
            o[0] = pack_bf16x2(v[0], v[1]);
            o[1] = pack_bf16x2(v[2], v[3]);
            const int chunk = SWIGLU ? qg : 4 * j + qg;
            const int off = r32 * ROW_BYTES + ((chunk ^ swz(r32)) * 16) + ((h ^ ((r32 >> 4) & 1)) * 8);
            *reinterpret_cast<u32x2_t*>(stage_lds + off) = o;
          }
        }
#pragma unroll
        for (int q = 0; q < 32 / ROWS_PER_INST; ++q) {
          const int rr = q * ROWS_PER_INST + rl;
          u32x4_t d = *reinterpret_cast<const u32x4_t*>(stage_lds + rr * ROW_BYTES +
                                                        ((cl ^ swz(rr)) * 16));
          if ((rr >> 4) & 1) d = u32x4_t{d[2], d[3], d[0], d[1]};  // halves were swapped
          const int m = ct.m0 + 32 * i + rr;
          const int col = col0 + 8 * cl;
          if (m < ct.me && col < p.N)
            *reinterpret_cast<u32x4_t*>(p.C + (int64_t)m * p.ldc + col) = d;
          if constexpr (kRowOps) {
            if (sum_rows) {
              // squares of the stored (bf16) values, summed over the row's 8
              // lanes (quad swaps, then the half-row mirror)
              float sq = 0.f;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float lo = bf16lo(d[e]), hi = bf16hi(d[e]);
                sq = fmaf(lo, lo, sq);
                sq = fmaf(hi, hi, sq);
              }
              sq += dpp_f32<0xB1>(0.f, sq);
              sq += dpp_f32<0x4E>(0.f, sq);
              sq += dpp_f32<0x141>(0.f, sq);
              if (cl == 0) s_ss[wave * kWideBM + 32 * i + rr] = sq;
            }
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging reads done
      lds_barrier();                       // before the next DMA into the slot
      if constexpr (kRowOps) {
        if (sum_rows) {
          // the tile's row sums, the four waves' column ranges added in order
          const int t = tid;  // 256 threads, one token row each
          const int m = ct.m0 + t;
          if (t < 32 * tma && m < ct.me) {
            const float ss = ((s_ss[t] + s_ss[kWideBM + t]) + s_ss[2 * kWideBM + t]) +
                             s_ss[3 * kWideBM + t];
            p.rowsq_out[(int64_t)((ct.n0 - p.rowsq_c0) / (64 * kWideWaves)) * p.ld_rowsq + m] = ss;
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;
    if (ct_idx + 1 < ntiles) ct = decode(ct_idx + 1);
  }
}

// ------------------------------------------------------- small groups ----
// Grouped GEMM for groups of at most 32*MT rows (decode-shaped layers: T <= 64
// tokens, so every expert holds at most T rows). The work is streaming the
// active experts' weights once from HBM, so the kernel is built for memory
// parallelism rather than reuse:
//   * one workgroup per (group, 64 weight rows): for SwiGLU the 32 gate rows
//     and the matching 32 up rows of 32 output columns, otherwise 64
//     consecutive rows; the workgroups are handed to the non-empty groups in
//     order and the rest exit at once, so idle experts cost no bandwidth;
//   * the 4 waves split K four ways; each lane loads its MFMA fragments of
//     weights and tokens straight from global memory into registers (no LDS,
//     no barrier in the K loop), one batch of K steps ahead of the MFMAs, so
//     even a handful of active experts keeps enough loads in flight for HBM
//     latency; with fragment-tiled weights every load is 1 KB contiguous;
//   * the partial sums meet in LDS once at the end, in a fixed order (waves
//     1-3 into wave 0), and wave 0 applies the epilogue (SwiGLU from fp32
//     accumulators);
//   * when so few (group, 64-row) units exist that they do not cover the CUs
//     (a projection of one or a few tokens), plain products switch to 32
//     weight rows and 8 waves per workgroup (NB = 1, NW = 8): twice the
//     workgroups, each splitting K eight ways.
// The weights are MFMA operand A and the tokens operand B, as in the large
// kernel, so the output layout per lane is the same (4 consecutive columns).
constexpr int kSkinnyWaves = 4;  // waves per workgroup, each one slice of K
constexpr int kSkinnyThreads = 64 * kSkinnyWaves;
constexpr int kSkinnyMaxRows = 64;  // largest group the small-group kernel is chosen for
// K steps (of 16) per load batch: 4 for one 32-row token block; 2 for two,
// whose token fragments double the registers per step (measured on MI355X at
// T=64: 117 us against 125 us per layer step with 4)
template <int MT>
constexpr int skinny_batch() { return MT == 1 ? 4 : 2; }

// Routing of a decode step (at most kRouteInGemmTokens tokens) in the prologue
// of the small-group SwiGLU kernel, as route_kernel does it for one chunk: the
// 16-lane row g of wave w picks the experts of token 4 w + g (route_token);
// 64-bit expert masks in the LDS give each (token, k) its stable slot (expert-
// major, ascending token) and the offsets of the routed groups, followed by
// the always-on groups of T rows each. Every workgroup computes the same
// integers from the same planes; workgroup 0 also stores them for the kernels
// after this one.
__device__ __forceinline__ void skinny_route_prologue(const GemmArgs& p,
                                                      unsigned long long* rt_mask, int* rt_off,
                                                      int* rt_tok, int lane, int wave,
                                                      bool store) {
  const int T = p.rt_T, E = p.rt_E, K = p.rt_K, nsh = p.rt_nsh;
  if (threadIdx.x < 64) rt_mask[threadIdx.x] = 0ull;
  __syncthreads();
  const int j = lane & 15;
  const int tl = 4 * wave + (lane >> 4);
  int my_e;
  float my_w;
  route_token(p.rt_parts, E, p.rt_n_parts, p.rt_part_stride, p.rt_bias, tl, tl < T,
              4 * wave < T, E, K, lane, my_e, my_w);
  if (tl < T && j < K) {
    atomicOr(&rt_mask[my_e], 1ull << tl);
    if (store) {
      p.rt_idx[tl * K + j] = my_e;
      p.rt_w[tl * K + j] = my_w;
    }
  } else {
    my_e = -1;
  }
  __syncthreads();
  if (wave == 0) {
    const int c = lane < E ? __popcll(rt_mask[lane]) : 0;
    const int inc = wave_inclusive_scan(c);
    if (lane < E) {
      rt_off[lane] = inc - c;
      if (store) {
        p.rt_offsets[lane] = inc - c;
        p.rt_counts[lane] = c;
      }
    }
    if (lane == 63) {
      for (int x = 0; x <= nsh; ++x) {
        rt_off[E + x] = inc + x * T;
        if (store) p.rt_offsets[E + x] = inc + x * T;
      }
    }
  }
  __syncthreads();
  if (my_e >= 0) {
    const int slot = rt_off[my_e] + __popcll(rt_mask[my_e] & ((1ull << tl) - 1ull));
    rt_tok[slot] = tl;
    if (store) {
      p.rt_token_map[slot] = tl;
      p.rt_slot_of[tl * K + j] = slot;
    }
  }
  // rows of the always-on groups: group E+x row t is token t
  const int S = T * K;
  for (int r = threadIdx.x; r < nsh * T; r += blockDim.x) {
    rt_tok[S + r] = r % T;
    if (store) p.rt_token_map[S + r] = r % T;
  }
  __syncthreads();
}

// NB: 32-row weight blocks per workgroup (SwiGLU with NB = 2: a gate and an up
// block of 32 output columns; SwiGLU with NB = 1: one block whose rows 0-15 are
// the gate rows and 16-31 the up rows of 16 output columns);
// NW: waves per workgroup, each one slice of K.
// The kernel body, on workgroup `bid` of the small-group grid (a device function
// so that other launches can host the same work in extra workgroups).
template <int MT, bool SWIGLU, bool GATHER, bool TILED, int NB = 2, int NW = kSkinnyWaves>
__device__ __forceinline__ void skinny_gemm_body(const GemmArgs& p, int n_blocks, int bid) {
  static_assert(NB == 2 || NB == 1, "one or two 32-row weight blocks");
  // SwiGLU in 16-column units: gate row r and up row r + 16 of the block meet in
  // one lane (accumulator i holds block row 8 (i / 4) + 4 h + i % 4)
  constexpr bool kHalfUnit = SWIGLU && NB == 1;
  static_assert(NW == 4 || NW == 8, "reduction written for 4 or 8 waves");
  // partial sums of the upper half of the waves (8 waves), then of waves 1..3
  __shared__ floatx4_t red[NW == 8 ? 4 : 3][NB][MT][4][64];
  // routing in the prologue (SwiGLU with gathered rows only): expert masks of
  // the step's tokens, group offsets and the slot -> token map
  constexpr bool kCanRoute = SWIGLU && GATHER && NW == 4;
  __shared__ unsigned long long rt_mask[kCanRoute ? 64 : 1];
  __shared__ int rt_off[kCanRoute ? kMaxGroups + 1 : 1];
  __shared__ int rt_tok[kCanRoute ? kRouteInGemmSlots : 1];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  bool routed = false;
  if constexpr (kCanRoute) {
    if (p.rt_parts != nullptr) {
      routed = true;
      skinny_route_prologue(p, rt_mask, rt_off, rt_tok, lane, wave, bid == 0);
    }
  }
  auto group_offset = [&](int i) { return routed ? rt_off[i] : p.offsets[i]; };
  int g = bid / n_blocks;
  const int nb = bid - g * n_blocks;
  int mb = 0, me = p.M;
  if (p.offsets != nullptr) {
    // The grid holds n_blocks workgroups for each of min(G, M) group ordinals
    // (no more groups than rows can be busy), but only non-empty groups have
    // work: workgroup ordinal g takes the g-th non-empty group. The busy
    // workgroups thus come first in dispatch order, and the idle ones, all at
    // the end of the grid, do not hold workgroup slots between them.
    const int G = p.G;
    int ord = g;
    g = -1;
    for (int base = 0; base < G; base += 64) {
      const int gi = base + lane;
      int lo = 0, hi = 0;
      if (gi < G) {
        lo = min(max(group_offset(gi), 0), p.M);
        hi = min(max(group_offset(gi + 1), lo), p.M);
      }
      const bool busy = hi > lo;
      const uint64_t mask = __ballot(busy);
      const int count = __popcll(mask);
      if (ord < count) {  // uniform
        const int rank = __popcll(mask & ((1ull << lane) - 1ull));
        const int src = __ffsll((unsigned long long)__ballot(busy && rank == ord)) - 1;
        g = base + src;
        mb = __builtin_amdgcn_readfirstlane(__shfl(lo, src, 64));
        me = __builtin_amdgcn_readfirstlane(__shfl(hi, src, 64));
        break;
      }
      ord -= count;
    }
    if (g < 0) return;  // uniform: past the non-empty groups
  }
  if (mb >= me) return;  // uniform: empty group

  const int r32 = lane & 31;
  const int h = lane >> 5;
  // Loads address a uniform base (scalar registers) plus a 32-bit per-lane
  // byte offset, so each load needs one VGPR of address and the K steps of a
  // batch become immediate offsets. Offsets stay below 4 GiB: one group's
  // weights, and at most 64 token rows of A.
  const char* Bg = reinterpret_cast<const char*>(p.B + (int64_t)g * p.b_group_stride);
  // per-group bases of A and C (batched products: groups of M rows each)
  const char* Ab = reinterpret_cast<const char*>(p.A + (int64_t)g * p.a_group_stride);
  uint16_t* const Cg = p.C + (int64_t)g * p.c_group_stride;
  // K steps (of 16) of this wave: an even split of K/16 over the waves
  const int ksteps = p.K / 16;
  const int s_beg = wave * ksteps / NW;
  const int nsteps = (wave + 1) * ksteps / NW - s_beg;
  const int k_beg = s_beg * 16;
  // Byte offset of this lane's fragment data at k_beg in each weight block.
  // Row-major weights: row r32 of the block, 32 bytes per K step (each load
  // instruction touches 32 rows). Tiled weights: the 1 KB fragment of the
  // block at this K step, lane-contiguous, 1 KB per K step (each load
  // instruction reads 1 KB of consecutive bytes).
  constexpr uint32_t kStepBytes = TILED ? 1024 : 32;
  uint32_t woff[NB];
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) {
    if constexpr (TILED && kHalfUnit) {
      // 16 gate rows from one half of a 32-row fragment, 16 up rows from the
      // same half of the matching up fragment (N % 32 == 0 for tiled weights)
      const int u = min(nb, p.N / 16 - 1);
      const int rb = (r32 < 16 ? 0 : p.up_row_offset / 32) + u / 2;
      const int src = (u & 1) * 16 + (r32 & 15) + 32 * h;  // lane of that row in the fragment
      woff[blk] = (uint32_t)((((int64_t)rb * (p.K / 16) + k_beg / 16) * 512 + src * 8) * 2);
    } else if constexpr (TILED) {
      int rb;
      if constexpr (SWIGLU) {
        const int cb = min(nb, p.N / 32 - 1);
        rb = blk == 0 ? cb : p.up_row_offset / 32 + cb;
      } else {
        rb = min(nb * NB + blk, p.N / 32 - 1);
      }
      woff[blk] = (uint32_t)((((int64_t)rb * (p.K / 16) + k_beg / 16) * 512 + lane * 8) * 2);
    } else {
      int row;
      if constexpr (kHalfUnit) {
        const int col = min(nb * 16 + (r32 & 15), p.N - 1);
        row = r32 < 16 ? col : p.up_row_offset + col;
      } else if constexpr (SWIGLU) {
        const int col = min(nb * 32 + r32, p.N - 1);
        row = blk == 0 ? col : p.up_row_offset + col;
      } else {
        row = min(nb * 32 * NB + blk * 32 + r32, p.N - 1);
      }
      woff[blk] = (uint32_t)(((int64_t)row * p.ldb + 8 * h + k_beg) * 2);
    }
  }
  const int row_limit = GATHER ? p.a_rows_limit : p.M;

  for (int m0 = mb; m0 < me; m0 += 32 * MT) {
    uint32_t toff[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + mt * 32 + r32;
      const int mm = m < me ? m : m0;
      int row = GATHER ? (routed ? rt_tok[mm] : p.a_rows[mm]) : mm;
      row = (row >= 0 && row < row_limit) ? row : 0;
      toff[mt] = (uint32_t)(((int64_t)row * p.lda + 8 * h + k_beg) * 2);
    }
    floatx16_t acc[NB][MT];
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[blk][mt][r] = 0.f;

    // Software pipeline over batches of skinny_batch<MT>() K steps: the loads of
    // batch b+1 are in flight while batch b's MFMAs run (two register
    // buffers, unrolled by two so they are indexed statically). The
    // scheduling barriers keep the compiler from interleaving loads and
    // MFMAs, which would leave only a few loads in flight.
    constexpr int U = skinny_batch<MT>();
    bf16x8_t wa[U][NB], ta[U][MT], wb[U][NB], tb[U][MT];
    auto load = [&](bf16x8_t (&wf)[U][NB], bf16x8_t (&tf)[U][MT], int s) {
      const uint32_t ks = (uint32_t)s * 32;  // byte offset of K step s in a token row
      const uint32_t kw_s = (uint32_t)s * kStepBytes;
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
          wf[u][blk] = __builtin_nontemporal_load(  // read once: stream past the caches
              reinterpret_cast<const bf16x8_t*>(Bg + (woff[blk] + kw_s) + kStepBytes * u));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          tf[u][mt] = *reinterpret_cast<const bf16x8_t*>(Ab + (toff[mt] + ks) + 32 * u);
      }
    };
    auto compute = [&](const bf16x8_t (&wf)[U][NB], const bf16x8_t (&tf)[U][MT], int n) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u >= n) break;
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[blk][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[u][blk], tf[u][mt],
                                                                   acc[blk][mt], 0, 0, 0);
      }
    };
    const int nbatch = nsteps / U;
    if (nbatch > 0) {
      load(wa, ta, 0);
      int b = 0;
      for (; b + 2 <= nbatch; b += 2) {
        load(wb, tb, (b + 1) * U);
        __builtin_amdgcn_sched_barrier(0);
        compute(wa, ta, U);
        __builtin_amdgcn_sched_barrier(0);
        // past the last batch this reloads the last one (cache hits, unused),
        // which keeps the loop free of conditional loads
        load(wa, ta, min(b + 2, nbatch - 1) * U);
        __builtin_amdgcn_sched_barrier(0);
        compute(wb, tb, U);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (b < nbatch) compute(wa, ta, U);
    }
    // remaining K steps (nsteps not a multiple of the batch)
    for (int s = nbatch * U; s < nsteps; ++s) {
      bf16x8_t w1[1][NB], t1[1][MT];
      const uint32_t ks = (uint32_t)s * 32;
#pragma unroll
      for (int blk = 0; blk < NB; ++blk)
        w1[0][blk] = __builtin_nontemporal_load(
            reinterpret_cast<const bf16x8_t*>(Bg + (woff[blk] + s * kStepBytes)));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        t1[0][mt] = *reinterpret_cast<const bf16x8_t*>(Ab + (toff[mt] + ks));
#pragma unroll
      for (int blk = 0; blk < NB; ++blk)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[blk][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1[0][blk], t1[0][mt],
                                                                 acc[blk][mt], 0, 0, 0);
    }

    // ---- reduce the K slices (upper half of the waves into the lower half,
    // then waves 1..3 into wave 0), epilogue by wave 0 one group of 4 output
    // columns at a time, so few values are live at once
    auto stash = [&](int slot) {
#pragma unroll
      for (int blk = 0; blk < NB; ++blk)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int qg = 0; qg < 4; ++qg) {
            floatx4_t v;
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = acc[blk][mt][4 * qg + c];
            red[slot][blk][mt][qg][lane] = v;
          }
    };
    if constexpr (NW == 8) {
      if (wave >= 4) stash(wave - 4);
      __syncthreads();
      if (wave < 4) {
#pragma unroll
      for (int blk = 0; blk < NB; ++blk)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int qg = 0; qg < 4; ++qg) {
            const floatx4_t v = red[wave][blk][mt][qg][lane];
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[blk][mt][4 * qg + c] += v[c];
          }
      }
      __syncthreads();
    }
    if (wave >= 1 && wave < 4) stash(wave - 1);
    __syncthreads();
    if (wave == 0) {
      auto total = [&](int blk, int mt, int qg) {
        floatx4_t v = red[0][blk][mt][qg][lane] + red[1][blk][mt][qg][lane] +
                      red[2][blk][mt][qg][lane];
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] += acc_read(acc[blk][mt][4 * qg + c]);
        return v;
      };
      // a workgroup's 32 or 64 columns lie on one side of the split (n_split % 64 == 0)
      const bool second = !SWIGLU && p.C2 != nullptr && nb * 32 * NB >= p.n_split;
      const int col0 = second ? p.n_split : 0;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = m0 + mt * 32 + r32;
        uint16_t* crow = second ? p.C2 + (int64_t)m * p.ldc2 : Cg + (int64_t)m * p.ldc;
        constexpr int JN = SWIGLU ? 1 : NB;
        constexpr int QG = kHalfUnit ? 2 : 4;  // half units: groups 0-1 gate, 2-3 up
#pragma unroll
        for (int j = 0; j < JN; ++j) {
#pragma unroll
          for (int qg = 0; qg < QG; ++qg) {
            const int nbase = kHalfUnit ? nb * 16 : SWIGLU ? nb * 32 : nb * 32 * NB + j * 32;
            const int n = nbase + 8 * qg + 4 * h;
            float v[4];
            if constexpr (kHalfUnit) {
              const floatx4_t gt = total(0, mt, qg), up = total(0, mt, qg + 2);
#pragma unroll
              for (int c = 0; c < 4; ++c) v[c] = silu_f(gt[c]) * up[c];
            } else if constexpr (SWIGLU) {
              const floatx4_t gt = total(0, mt, qg), up = total(1, mt, qg);
#pragma unroll
              for (int c = 0; c < 4; ++c) v[c] = silu_f(gt[c]) * up[c];
            } else {
              const floatx4_t t = total(j, mt, qg);
#pragma unroll
              for (int c = 0; c < 4; ++c) v[c] = t[c];
            }
            if (m < me) {
              if (n + 3 < p.N) {
                u32x2_t o;
                o[0] = pack_bf16x2(v[0], v[1]);
                o[1] = pack_bf16x2(v[2], v[3]);
                *reinterpret_cast<u32x2_t*>(crow + (n - col0)) = o;
              } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                  if (n + c < p.N) crow[n - col0 + c] = f32_to_bf16(v[c]);
              }
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    __syncthreads();  // red is reused by the next row chunk
  }
}

template <int MT, bool SWIGLU, bool GATHER, bool TILED, int NB = 2, int NW = kSkinnyWaves>
__global__ __launch_bounds__(64 * NW) void skinny_gemm_kernel(GemmArgs p, int n_blocks) {
  skinny_gemm_body<MT, SWIGLU, GATHER, TILED, NB, NW>(p, n_blocks, blockIdx.x);
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
constexpr int kMaxDevices = 64;

// The device the calling thread has current, or -1 outside [0, kMaxDevices).
static int current_device() {
  int dev = 0;
  return hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices ? dev : -1;
}

// CU count of the current device, queried once per device (any thread).
static int num_cus() {
  static std::atomic<int> cached[kMaxDevices];  // static storage: starts at 0
  const int dev = current_device();
  if (dev < 0) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Raises a kernel's dynamic LDS limit on the current device; `once` is the
// caller's per-kernel flag array, one flag per device.
static void allow_lds(std::once_flag (&once)[kMaxDevices], const void* kern, int bytes) {
  const int dev = current_device();
  if (dev < 0) return;
  std::call_once(once[dev], [&] {
    (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  });
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int BK, int STAGES, bool SWIGLU,
          bool GATHER, bool TILED>
static int launch_grouped_gemm(const GemmArgs& a, hipStream_t st) {
  using Cfg = GemmCfg<BM, BN, WAVES_M, WAVES_N, BK, STAGES, SWIGLU>;
  auto kern = grouped_gemm_kernel<BM, BN, WAVES_M, WAVES_N, BK, STAGES, SWIGLU, GATHER, TILED>;
  static std::once_flag once[kMaxDevices];
  allow_lds(once, reinterpret_cast<const void*>(kern), Cfg::LDS_BYTES);
  const int G = a.offsets != nullptr ? a.G : 1;
  const int64_t nt = (a.N + Cfg::OUT_N - 1) / Cfg::OUT_N;
  // upper bound on the kernel's tile count (a group of n rows has ceil(n/BM) M tiles)
  const int64_t upper = ((int64_t)(a.M + BM - 1) / BM + (a.offsets ? G : 0)) * nt;
  const int chunk = sched_chunk(a.chunk_m_tiles, (int)nt);
  const int64_t nwg = sched_workgroups(upper, num_cus(), GATHER ? Cfg::ROW_TILES : 0, chunk);
  // the gathered kernel stages every tile's row indices in an LDS table of
  // ROW_TILES tiles and computes nothing if its share is larger
  if (GATHER &&
      (upper > INT32_MAX || sched_max_tiles((int)upper, (int)nwg, chunk) > Cfg::ROW_TILES))
    return fail(DSK_ERR_INVALID_ARG, "grouped_gemm: a workgroup's tiles exceed the LDS row table");
  hipLaunchKernelGGL(kern, dim3((unsigned)nwg), dim3(Cfg::THREADS), Cfg::LDS_BYTES, st, a);
  return check_launch("grouped_gemm_kernel");
}

template <bool SWIGLU, bool GATHER>
static int launch_wide_gemm(const GemmArgs& a, hipStream_t st) {
  auto kern = wide_gemm_kernel<SWIGLU, GATHER>;
  static std::once_flag once[kMaxDevices];
  allow_lds(once, reinterpret_cast<const void*>(kern), kWideLdsBytes);
  constexpr int OUT_N = SWIGLU ? 32 * kWideWaves : 64 * kWideWaves;
  const int G = a.offsets != nullptr ? a.G : 1;
  const int64_t nt = (a.N + OUT_N - 1) / OUT_N;
  const int64_t upper = ((int64_t)(a.M + kWideBM - 1) / kWideBM + (a.offsets ? G : 0)) * nt;
  const int chunk = sched_chunk(a.chunk_m_tiles, (int)nt);
  const int64_t nwg = sched_workgroups(upper, num_cus(), GATHER ? kWideRowTiles : 0, chunk);
  if (GATHER &&
      (upper > INT32_MAX || sched_max_tiles((int)upper, (int)nwg, chunk) > kWideRowTiles))
    return fail(DSK_ERR_INVALID_ARG, "wide_gemm: a workgroup's tiles exceed the LDS row table");
  hipLaunchKernelGGL(kern, dim3((unsigned)nwg), dim3(64 * kWideWaves), kWideLdsBytes, st, a);
  return check_launch("wide_gemm_kernel");
}

template <int MT, bool SWIGLU, bool GATHER, bool TILED>
static int launch_skinny_gemm(const GemmArgs& a, hipStream_t st) {
  // groups: by offsets, or a batch of G equal groups of M rows (per-group bases)
  const int G = a.offsets != nullptr || a.a_group_stride != 0 || a.c_group_stride != 0 ? a.G : 1;
  // group ordinals launched: with non-decreasing offsets, at most one busy
  // group per row; offsets from a caller may overlap, so every group gets one
  const int64_t GL = a.offsets != nullptr && a.offsets_sorted
                         ? std::min<int64_t>(G, std::max(a.M, 1)) : G;
  if constexpr (!SWIGLU) {
    // Few groups with rows (a decode step's projections: one group, one token):
    // 32-row blocks and 8 waves per workgroup, so the weights stream through
    // twice the workgroups with twice the loads in flight in each.
    const int64_t busy = a.offsets != nullptr ? std::min<int64_t>(G, std::max(a.M, 1)) : G;
    if (busy * ((a.N + 63) / 64) < (int64_t)num_cus()) {
      const int n_blocks = (a.N + 31) / 32;
      hipLaunchKernelGGL((skinny_gemm_kernel<MT, SWIGLU, GATHER, TILED, 1, 8>),
                         dim3((unsigned)(GL * n_blocks)), dim3(64 * 8), 0, st, a, n_blocks);
      return check_launch("skinny_gemm_kernel");
    }
  }
  if constexpr (SWIGLU) {
    // Fewer than two 32-column workgroups per CU (a one-token step: 8 groups x
    // 44): a CU's fetch rate bounds each workgroup's weight stream, so the CUs
    // that hold two set the launch time. 16-column units halve the bytes per
    // workgroup and spread them over the CUs more evenly. Measured on MI355X:
    // GEMM1 at T = 1 27.7 -> 25.2 us (bitwise the same output); at T = 2-4 (704
    // or more workgroups) unchanged, at T = 16 1.4 us and at T = 64 11 us slower.
    if (GL * ((a.N + 31) / 32) < 2 * (int64_t)num_cus()) {
      const int n_blocks = (a.N + 15) / 16;
      hipLaunchKernelGGL((skinny_gemm_kernel<MT, true, GATHER, TILED, 1, kSkinnyWaves>),
                         dim3((unsigned)(GL * n_blocks)), dim3(kSkinnyThreads), 0, st, a,
                         n_blocks);
      return check_launch("skinny_gemm_kernel");
    }
  }
  const int n_blocks = SWIGLU ? (a.N + 31) / 32 : (a.N + 63) / 64;
  const int64_t grid = GL * n_blocks;
  hipLaunchKernelGGL((skinny_gemm_kernel<MT, SWIGLU, GATHER, TILED>), dim3((unsigned)grid),
                     dim3(kSkinnyThreads), 0, st, a, n_blocks);
  return check_launch("skinny_gemm_kernel");
}

template <bool SWIGLU, bool GATHER, bool TILED>
static int launch_skinny(const GemmArgs& a, int rows, hipStream_t st) {
  if (rows <= 32) return launch_skinny_gemm<1, SWIGLU, GATHER, TILED>(a, st);
  return launch_skinny_gemm<2, SWIGLU, GATHER, TILED>(a, st);
}

static int validate_gemm(const GemmArgs& a, const char* who) {
  char buf[256];
  if (a.M < 0 || a.N <= 0 || a.K <= 0) {
    snprintf(buf, sizeof buf, "%s: invalid sizes M=%d N=%d K=%d", who, a.M, a.N, a.K);
    return fail(DSK_ERR_INVALID_ARG, buf);
  }
  if (a.K % DSK_GEMM_BK != 0) {
    snprintf(buf, sizeof buf, "%s: K=%d must be a multiple of %d", who, a.K, DSK_GEMM_BK);
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
  if (a.lda < a.K || (!a.b_tiled && a.ldb < a.K))
    return fail(DSK_ERR_INVALID_ARG, std::string(who) + ": leading dimension < K");
  if (a.b_tiled && (a.N % 32 || a.up_row_offset % 32))
    return fail(DSK_ERR_INVALID_ARG,
                std::string(who) + ": tiled weights need N and the up-row offset in multiples of 32");
  // the kernels address A rows by 32-bit byte offsets from A
  const int64_t a_extent = (int64_t)(a.a_rows != nullptr ? a.a_rows_limit : a.M) * a.lda * 2;
  if (a_extent > (int64_t)UINT32_MAX)
    return fail(DSK_ERR_INVALID_ARG, std::string(who) + ": A operand larger than 4 GiB");
  return DSK_OK;
}

// Kernel choice: groups known to hold at most 64 rows (decode) go to the
// weight-streaming kernel, everything else to the 256 x 256 tile kernel.
template <bool SWIGLU, bool GATHER, bool TILED>
static int run_gemm_t(const GemmArgs& a, hipStream_t st) {
  // groups of at most 64 rows (decode): weight streaming kernel
  const int rows = a.max_group_rows > 0 ? std::min(a.max_group_rows, a.M) : a.M;
  // routing in the prologue exists only in the small-group SwiGLU kernel with gathered rows
  DSK_REQUIRE(a.rt_parts == nullptr ||
                  (SWIGLU && GATHER && rows <= kSkinnyMaxRows && a.offsets != nullptr &&
                   a.rt_T >= 1 && a.rt_T <= kRouteInGemmTokens && a.M <= kRouteInGemmSlots),
              DSK_ERR_INVALID_ARG, "grouped GEMM: routing in the prologue needs a small SwiGLU step");
  if (rows <= kSkinnyMaxRows) return launch_skinny<SWIGLU, GATHER, TILED>(a, rows, st);
#ifndef DSK_GEMM_WIDE
#define DSK_GEMM_WIDE 1
#endif
  // fragment-tiled weights with K % 128 == 0 and 16-byte aligned output rows:
  // one wave per SIMD, weights straight to registers. Measured on MI355X at
  // T=4096: 234 us against 251 us for the down projection, but 448 against
  // 418 us for the gathered SwiGLU projection (368 against 360 us in steady
  // state), which stays on the 8-wave kernel.
  if (DSK_GEMM_WIDE && TILED && !(SWIGLU && GATHER) && a.K % (2 * kWideBK) == 0 &&
      aligned16(a.C) && a.ldc % 8 == 0)
    return launch_wide_gemm<SWIGLU, GATHER>(a, st);
  constexpr int BM = DSK_GEMM_BM, BN = DSK_GEMM_BN, WM = DSK_GEMM_WAVES_M;
  constexpr int BK = DSK_GEMM_BK, ST = DSK_GEMM_STAGES;
  constexpr int WN = DSK_GEMM_WAVES_N;
  return launch_grouped_gemm<BM, BN, WM, WN, BK, ST, SWIGLU, GATHER, TILED>(a, st);
}

int run_gemm(const GemmArgs& a, bool swiglu, hipStream_t st) {
  if (a.M == 0) return DSK_OK;
  if (a.rowsq_out != nullptr || a.rowscale_ss != nullptr) {
    // row statistics live in the one-wave-per-SIMD kernel's epilogue only
    DSK_REQUIRE(a.b_tiled && !swiglu && a.a_rows == nullptr && a.offsets == nullptr &&
                    a.K % (2 * kWideBK) == 0 && aligned16(a.C) && a.ldc % 8 == 0,
                DSK_ERR_INVALID_ARG,
                "linear row statistics: need a tiled weight, K % 128 == 0 and 16-byte aligned "
                "output rows");
    DSK_REQUIRE(a.rowsq_out == nullptr ||
                    (a.rowsq_c0 >= 0 && a.rowsq_c0 < a.rowsq_c1 && a.rowsq_c1 <= a.N &&
                     a.rowsq_c0 % 256 == 0 && a.rowsq_c1 % 256 == 0 && a.ld_rowsq >= a.M),
                DSK_ERR_INVALID_ARG,
                "linear_rowsq: the column range must be 256-aligned inside [0, N) and "
                "ld_rowsq >= M");
    DSK_REQUIRE(a.rowscale_ss == nullptr ||
                    (a.rowscale_parts >= 1 && a.rowscale_parts <= kRowScaleParts &&
                     a.rowscale_cols > 0 && a.ld_rowscale >= a.M),
                DSK_ERR_INVALID_ARG,
                "linear_rowscale: need 1 or 2 parts, cols > 0 and ld_rowscale >= M");
    return launch_wide_gemm<false, false>(a, st);
  }
  const bool g = a.a_rows != nullptr;
  if (a.b_tiled) {
    if (swiglu) return g ? run_gemm_t<true, true, true>(a, st) : run_gemm_t<true, false, true>(a, st);
    return g ? run_gemm_t<false, true, true>(a, st) : run_gemm_t<false, false, true>(a, st);
  }
  if (swiglu) return g ? run_gemm_t<true, true, false>(a, st) : run_gemm_t<true, false, false>(a, st);
  return g ? run_gemm_t<false, true, false>(a, st) : run_gemm_t<false, false, false>(a, st);
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

extern "C" int dsk_linear_ex(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w,
                             int weight_layout, dsk_bf16* out, int64_t ld_out, int M, int K,
                             int N, void* stream) {
  DSK_REQUIRE(weight_layout == DSK_LAYOUT_ROW_MAJOR || weight_layout == DSK_LAYOUT_TILED,
              DSK_ERR_INVALID_ARG, "linear: weight_layout must be row-major or tiled");
  if (weight_layout == DSK_LAYOUT_ROW_MAJOR)
    return dsk_linear(x, ld_x, w, out, ld_out, M, K, N, stream);
  DSK_REQUIRE(M >= 0, DSK_ERR_INVALID_ARG, "linear: M < 0");
  if (M == 0) return DSK_OK;
  GemmArgs a{};
  a.A = x; a.lda = ld_x;
  a.B = w; a.ldb = K; a.b_group_stride = 0;
  a.C = out; a.ldc = ld_out;
  a.offsets = nullptr; a.G = 1;
  a.M = M; a.N = N; a.K = K;
  a.b_tiled = 1;
  int rc = validate_gemm(a, "linear");
  if (rc) return rc;
  DSK_REQUIRE(ld_out >= N, DSK_ERR_INVALID_ARG, "linear: ld_out < N");
  return run_gemm(a, false, as_stream(stream));
}

static int linear_rowstats(const char* who, const dsk_bf16* x, int64_t ld_x,
                           const dsk_bf16* w_tiled, dsk_bf16* out, int64_t ld_out, int M, int K,
                           int N, GemmArgs& a, void* stream) {
  DSK_REQUIRE(M >= 0, DSK_ERR_INVALID_ARG, std::string(who) + ": M < 0");
  if (M == 0) return DSK_OK;
  a.A = x; a.lda = ld_x;
  a.B = w_tiled; a.ldb = K; a.b_group_stride = 0;
  a.C = out; a.ldc = ld_out;
  a.offsets = nullptr; a.G = 1;
  a.M = M; a.N = N; a.K = K;
  a.b_tiled = 1;
  int rc = validate_gemm(a, who);
  if (rc) return rc;
  DSK_REQUIRE(ld_out >= N, DSK_ERR_INVALID_ARG, std::string(who) + ": ld_out < N");
  return run_gemm(a, false, as_stream(stream));
}

extern "C" int dsk_linear_rowsq(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w_tiled,
                                dsk_bf16* out, int64_t ld_out, int M, int K, int N,
                                float* row_sumsq, int64_t ld_rowsq, int col_begin, int col_end,
                                void* stream) {
  DSK_REQUIRE(row_sumsq != nullptr, DSK_ERR_NULL_PTR, "linear_rowsq: row_sumsq is NULL");
  GemmArgs a{};
  a.rowsq_out = row_sumsq; a.ld_rowsq = ld_rowsq;
  a.rowsq_c0 = col_begin; a.rowsq_c1 = col_end;
  return linear_rowstats("linear_rowsq", x, ld_x, w_tiled, out, ld_out, M, K, N, a, stream);
}

extern "C" int dsk_linear_rowscale(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w_tiled,
                                   dsk_bf16* out, int64_t ld_out, int M, int K, int N,
                                   const float* row_sumsq, int64_t ld_rowsq, int n_parts,
                                   int n_cols, float eps, void* stream) {
  DSK_REQUIRE(row_sumsq != nullptr, DSK_ERR_NULL_PTR, "linear_rowscale: row_sumsq is NULL");
  GemmArgs a{};
  a.rowscale_ss = row_sumsq; a.ld_rowscale = ld_rowsq;
  a.rowscale_parts = n_parts; a.rowscale_cols = n_cols; a.rowscale_eps = eps;
  return linear_rowstats("linear_rowscale", x, ld_x, w_tiled, out, ld_out, M, K, N, a, stream);
}

extern "C" int dsk_linear_split(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w_tiled,
                                dsk_bf16* out0, int64_t ld_out0, dsk_bf16* out1,
                                int64_t ld_out1, int M, int K, int N, int n_split,
                                void* stream) {
  DSK_REQUIRE(M >= 0, DSK_ERR_INVALID_ARG, "linear_split: M < 0");
  DSK_REQUIRE(n_split > 0 && n_split < N && n_split % 64 == 0, DSK_ERR_INVALID_ARG,
              "linear_split: n_split must be a multiple of 64 in (0, N)");
  DSK_REQUIRE(ld_out0 >= n_split && ld_out1 >= N - n_split, DSK_ERR_INVALID_ARG,
              "linear_split: ld_out0 < n_split or ld_out1 < N - n_split");
  DSK_REQUIRE(out1 != nullptr, DSK_ERR_NULL_PTR, "linear_split: NULL pointer");
  DSK_REQUIRE((reinterpret_cast<uintptr_t>(out1) & 7u) == 0 && ld_out1 % 4 == 0,
              DSK_ERR_ALIGNMENT, "linear_split: out1 rows must be 8-byte aligned");
  if (M == 0) return DSK_OK;
  GemmArgs a{};
  a.A = x; a.lda = ld_x;
  a.B = w_tiled; a.ldb = K; a.b_group_stride = 0;
  a.C = out0; a.ldc = ld_out0;
  a.offsets = nullptr; a.G = 1;
  a.M = M; a.N = N; a.K = K;
  a.b_tiled = 1;
  int rc = validate_gemm(a, "linear_split");
  if (rc) return rc;
  if (M <= kSkinnyMaxRows) {  // one launch, the destination chosen per workgroup
    a.C2 = out1; a.ldc2 = ld_out1; a.n_split = n_split;
    return run_gemm(a, false, as_stream(stream));
  }
  // larger M: two launches over the two row-block ranges of the tiled weight
  rc = dsk_linear_ex(x, ld_x, w_tiled, DSK_LAYOUT_TILED, out0, ld_out0, M, K, n_split, stream);
  if (rc) return rc;
  const dsk_bf16* w1 = w_tiled + (int64_t)(n_split / 32) * (K / 16) * 512;
  return dsk_linear_ex(x, ld_x, w1, DSK_LAYOUT_TILED, out1, ld_out1, M, K, N - n_split, stream);
}

extern "C" int dsk_linear_batched(const dsk_bf16* x, int64_t ld_x, int64_t x_batch_stride,
                                  const dsk_bf16* w_tiled, dsk_bf16* out, int64_t ld_out,
                                  int64_t out_batch_stride, int batch, int M, int K, int N,
                                  void* stream) {
  DSK_REQUIRE(batch >= 0 && M >= 0, DSK_ERR_INVALID_ARG, "linear_batched: batch and M >= 0");
  if (batch == 0 || M == 0) return DSK_OK;
  DSK_REQUIRE(batch <= 65535 && M <= kSkinnyMaxRows, DSK_ERR_INVALID_ARG,
              "linear_batched: needs M <= 64 rows per batch entry and batch <= 65535");
  DSK_REQUIRE(x_batch_stride % 8 == 0 && out_batch_stride % 4 == 0, DSK_ERR_ALIGNMENT,
              "linear_batched: batch strides must keep rows aligned (x: 16 B, out: 8 B)");
  DSK_REQUIRE(x_batch_stride >= 0 && out_batch_stride >= 0 &&
                  (batch == 1 || (x_batch_stride > 0 && out_batch_stride > 0)),
              DSK_ERR_INVALID_ARG, "linear_batched: batch strides must be positive");
  GemmArgs a{};
  a.A = x; a.lda = ld_x; a.a_group_stride = x_batch_stride;
  a.B = w_tiled; a.ldb = K; a.b_group_stride = (int64_t)N * K;
  a.C = out; a.ldc = ld_out; a.c_group_stride = out_batch_stride;
  a.offsets = nullptr; a.G = batch;
  a.M = M; a.N = N; a.K = K;
  a.max_group_rows = M;
  a.b_tiled = 1;
  int rc = validate_gemm(a, "linear_batched");
  if (rc) return rc;
  DSK_REQUIRE(ld_out >= N, DSK_ERR_INVALID_ARG, "linear_batched: ld_out < N");
  // 32-bit byte offsets inside each entry (rows of A and C are addressed from
  // the entry's base)
  DSK_REQUIRE((int64_t)M * ld_x * 2 <= (int64_t)UINT32_MAX, DSK_ERR_INVALID_ARG,
              "linear_batched: an entry of x spans more than 4 GiB");
  return run_gemm(a, false, as_stream(stream));
}

extern "C" int dsk_kv_upproj(const dsk_bf16* normed_kv, int64_t ld_in, const dsk_bf16* weight,
                             dsk_bf16* out, int rows, int kv_lora_rank, int out_dim,
                             void* stream) {
  return dsk_linear(normed_kv, ld_in, weight, out, out_dim, rows, kv_lora_rank, out_dim,
                    stream);
}
