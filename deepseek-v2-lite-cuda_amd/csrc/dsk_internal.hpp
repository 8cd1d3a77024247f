// Internal (non-ABI) launch helpers shared between the translation units.
#pragma once

#include "dsk_common.hpp"

namespace dsk {

// Grouped GEMM problem: C[m, :] = A[row(m), :] @ B_g^T for m in group g's rows.
struct GemmArgs {
  const uint16_t* A;
  int64_t lda;
  const int32_t* a_rows;   // optional: A row of output row m is a_rows[m]
  int a_rows_limit;        // valid A rows are [0, a_rows_limit)
  const uint16_t* B;
  int64_t ldb;
  int64_t b_group_stride;  // elements between consecutive groups' weights
  uint16_t* C;
  int64_t ldc;
  const int32_t* offsets;  // [G+1] group row boundaries, or NULL: one group [0, M)
  int G;
  int M, N, K;             // N = output columns (SwiGLU: intermediate size)
  int up_row_offset;       // SwiGLU: first up row inside a group's weight
  int max_group_rows;      // upper bound on any group's row count known to the host
                           // (0: unknown, M is used); selects the small-group kernel
  int offsets_sorted;      // offsets never decrease (the fused layer's own): the small-
                           // group grid then launches min(G, M) group ordinals, else G
  int chunk_m_tiles;       // large-group kernels: M tiles of a typical group, so that
                           // tiles are dealt to the XCDs a group at a time (0: chunks
                           // of kTileChunk tiles; gemm_sched.hpp sched_chunk)
  int64_t a_group_stride;  // skinny kernel: elements between the A bases of consecutive
  int64_t c_group_stride;  // groups, and of the C bases (0: one base, rows by offsets)
  int b_tiled;             // B stored as MFMA fragments (see the fragment-tiled layout in
                           // dsk.h); ldb is then unused
  uint16_t* C2;            // skinny kernel, optional: output columns n >= n_split go to
  int64_t ldc2;            // C2[m * ldc2 + n - n_split] instead of C (n_split % 64 == 0)
  int n_split;
  // Row statistics in the epilogue of the one-wave-per-SIMD kernel (G = 1, no
  // SwiGLU, no gather), optional:
  //   rowsq_out[(n0 - rowsq_c0) / 256 * ld_rowsq + m] = sum over the 256 output
  //   columns n0.. of tile n0 (inside [rowsq_c0, rowsq_c1)) of bf16(C[m, n])^2;
  //   rowscale_ss != NULL: C[m, :] *= rsqrt(sum_p rowscale_ss[p * ld_rowscale + m]
  //   / rowscale_cols + rowscale_eps), p < rowscale_parts (an RMS norm of the A
  //   rows whose weight is folded into B).
  float* rowsq_out;
  int64_t ld_rowsq;
  int rowsq_c0, rowsq_c1;
  const float* rowscale_ss;
  int64_t ld_rowscale;
  int rowscale_parts, rowscale_cols;
  float rowscale_eps;
  // Small-group SwiGLU kernel with gathered rows, optional (decode steps of at
  // most kRouteInGemmTokens tokens): every workgroup routes the step itself in
  // its prologue from the gate's partial planes (route_token), and uses its own
  // expert offsets and row map instead of offsets / a_rows; workgroup 0 also
  // writes the routing outputs (topk idx / weights, counts, offsets with the
  // always-on groups, token_map, slot_of) for the kernels after it.
  const float* rt_parts;
  int rt_n_parts;
  int64_t rt_part_stride;
  const float* rt_bias;
  int rt_T, rt_E, rt_K, rt_nsh;
  int32_t* rt_idx;
  float* rt_w;
  int32_t* rt_counts;
  int32_t* rt_offsets;
  int32_t* rt_token_map;
  int32_t* rt_slot_of;
};

// Tokens up to which a decode step is routed in GEMM1's prologue: every launched
// workgroup routes before it knows whether its group is busy, and at T = 1 the
// grid holds only busy groups (at most T*K + always-on groups of rows).
constexpr int kRouteInGemmTokens = 1;
constexpr int kRouteInGemmSlots = 256;  // routed + always-on rows the prologue maps

int run_gemm(const GemmArgs& a, bool swiglu, hipStream_t st);


// Router logits for routing = sum over n_parts partial-sum planes
// (logits + s * part_stride, s < n_parts, fixed order) + bias[e] if given.
int launch_route(const float* logits, int64_t ld, int n_parts, int64_t part_stride,
                 const float* bias, int T, int E, int K, int32_t* idx, float* w,
                 int32_t* blk_hist, int32_t* local_rank, int32_t* counts, int32_t* offsets,
                 int32_t* token_map, int32_t* slot_of, int n_extra_groups, hipStream_t st);
// Partial gate sums: parts[s][t][e] = sum over the s-th of n_parts K slices of
// x[t, k] * wg[e, k] (fp32), for the route kernel to add up.
int gate_parts_count(int T, int E, int H);
// Full gate logits (16 waves per 32 x 32 block, K split over the waves and
// reduced in the LDS in a fixed order), + bias[e] if bias is not NULL.
int launch_gate_logits(const uint16_t* x, int64_t ld_x, const uint16_t* wg, bool tiled,
                       const float* bias, float* logits, int64_t ld_out, int T, int E, int H,
                       hipStream_t st);
int launch_gate_parts(const uint16_t* x, int64_t ld_x, const uint16_t* wg, bool tiled,
                      float* parts, int T, int E, int H, int n_parts, hipStream_t st);
int launch_scan(const int32_t* hist, int nblk, int E, int32_t* counts, int32_t* offsets,
                int32_t* blk_base, int n_extra_groups, int extra_rows, hipStream_t st);
// Scan + permutation in one launch (the fused layer's T > 64 path): offsets,
// counts, token_map and slot_of from the chunk histograms and in-chunk ranks.
int launch_scan_permute(const int32_t* hist, int nblk, const int32_t* idx, int T, int K,
                        int E, const int32_t* local_rank, int S, int32_t* counts,
                        int32_t* offsets, int32_t* token_map, int32_t* slot_of,
                        int n_extra_groups, hipStream_t st);
int launch_permute(const int32_t* idx, const float* w, int T, int K, int E,
                   const int32_t* offsets, const int32_t* blk_base, const int32_t* local_rank,
                   int S, int32_t* token_map, float* dw, int32_t* slot_of, int n_extra_groups,
                   hipStream_t st);
int launch_combine_slots(const uint16_t* y, int64_t ldy, const int32_t* slot_of,
                         const float* topk_w, int T, int K, int H, int extra_base,
                         int n_extra_groups, uint16_t* out, int64_t ldo, hipStream_t st);

}  // namespace dsk
