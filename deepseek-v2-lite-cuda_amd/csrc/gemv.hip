// Linear maps of one to four token rows with fragment-tiled weights (the
// projections of an absorbed-MLA decode step), on the vector ALU:
//
//   out[b][m][n] = sum_k x[b][m][k] * w[b][n][k]      (fp32 sums, bf16 out)
//
// At one token a projection is a stream of its weights with two flops per
// weight element, so what matters is spreading that stream over the whole
// chip. The MFMA kernels need 32 weight rows and all of K per workgroup,
// which leaves a 2048-row projection with 64 workgroups. Here a group of
// lanes owns 8 rows: exactly one 128-byte line of each fragment half of the
// tiled layout (fragment (rb, ks) holds rows 32 rb .. 32 rb + 31 and K
// 16 ks .. 16 ks + 15; its first 256 elements are the K-half 0..7 of the 32
// rows, 8 per row). With 64 lanes per group (K >= 512) a 2048-row projection
// runs as 256 single-wave workgroups; with K < 512, 16 lanes per group and four
// groups per wave. Each lane sums its K slice with v_dot2_f32_bf16 in K order,
// the lanes of a group are added by a fixed DPP tree, so results are the same
// on every run.
#include "dsk_internal.hpp"

namespace dsk {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

struct RowsArgs {
  const uint16_t* x;
  int64_t ld_x, x_bs;      // token row stride, batch-entry stride (elements)
  const uint16_t* w;       // tiled [batch][N/32][K/16][64][8]
  int64_t w_bs;
  uint16_t* out0;          // outputs n < n_split
  int64_t ld_out0, out0_bs;
  uint16_t* out1;          // outputs n >= n_split, at column n - n_split
  int64_t ld_out1, out1_bs;
  int n_split, K, N;
};

constexpr int kRowsPerGroup = 8;  // one 128-byte line of a fragment half

// 8 bf16 products of w and x added to acc in order. The elements go through
// scalars first: hipcc (ROCm 7.2) compiles bit_cast(bf16x2, vector[e]) to
// element 0 for every e.
__device__ __forceinline__ float dot8(const u32x4_t& w, const u32x4_t& x, float acc) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t wq = w[q], xq = x[q];
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wq),
                                          __builtin_bit_cast(bf16x2_t, xq), acc, false);
  }
  return acc;
}

template <int M, int LPR>
__global__ __launch_bounds__(64) void linear_rows_kernel(RowsArgs a) {
  constexpr int G = 64 / LPR;  // lane groups per wave
  // K chunks whose loads are issued together (a whole 2048-long row at 64 lanes)
  constexpr int kRowsBatch = LPR == 64 ? 4 : 1;
  const int lane = threadIdx.x;
  const int g = lane / LPR, li = lane % LPR;
  const int b = blockIdx.y;
  const int n0 = (blockIdx.x * G + g) * kRowsPerGroup;  // this group's first row
  const int nl = min(n0, a.N - kRowsPerGroup);          // rows past N: reload, unused
  const int rb = nl / 32, slab = (nl % 32) / kRowsPerGroup;
  const uint16_t* wb = a.w + b * a.w_bs + (int64_t)rb * (a.K / 16) * 512 + slab * 64;
  const uint16_t* xb = a.x + b * a.x_bs;
  const int nch = a.K / (8 * LPR);  // 8-element K chunks per lane

  float acc[M][kRowsPerGroup];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int i = 0; i < kRowsPerGroup; ++i) acc[m][i] = 0.f;

  for (int j0 = 0; j0 < nch; j0 += kRowsBatch) {
    u32x4_t wv[kRowsBatch][kRowsPerGroup], xv[kRowsBatch][M];
#pragma unroll
    for (int u = 0; u < kRowsBatch; ++u) {
      // chunk c = K elements 8c .. 8c+7: fragment c / 2, K half c % 2
      const int c = li + LPR * min(j0 + u, nch - 1);
      const uint16_t* wp = wb + (c >> 1) * 512 + (c & 1) * 256;
#pragma unroll
      for (int i = 0; i < kRowsPerGroup; ++i)
        wv[u][i] = *reinterpret_cast<const u32x4_t*>(wp + i * 8);
#pragma unroll
      for (int m = 0; m < M; ++m)
        xv[u][m] = *reinterpret_cast<const u32x4_t*>(xb + m * a.ld_x + c * 8);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch before the first use
#pragma unroll
    for (int u = 0; u < kRowsBatch; ++u) {
      if (j0 + u < nch) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int i = 0; i < kRowsPerGroup; ++i) acc[m][i] = dot8(wv[u][i], xv[u][m], acc[m][i]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // sums over the group's lanes (fixed DPP trees; every lane gets the total)
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int i = 0; i < kRowsPerGroup; ++i)
      acc[m][i] = LPR == 64 ? wave_sum(acc[m][i]) : row16_sum(acc[m][i]);

  // lane li of the group stores value idx = li + LPR * k: token idx / 8, row idx % 8
  if (n0 >= a.N) return;
#pragma unroll
  for (int k = 0; k * LPR < M * kRowsPerGroup; ++k) {
    const int idx = li + LPR * k;
    if (idx >= M * kRowsPerGroup) break;
    float v = 0.f;
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int i = 0; i < kRowsPerGroup; ++i)
        if (idx == m * kRowsPerGroup + i) v = acc[m][i];
    const int m = idx / kRowsPerGroup;
    const int n = n0 + idx % kRowsPerGroup;
    uint16_t* dst = n < a.n_split ? a.out0 + b * a.out0_bs + m * a.ld_out0 + n
                                  : a.out1 + b * a.out1_bs + m * a.ld_out1 + (n - a.n_split);
    *dst = f32_to_bf16(v);
  }
}

template <int LPR>
static void launch_rows_lpr(const RowsArgs& a, int M, int batch, hipStream_t st) {
  constexpr int G = 64 / LPR;
  const dim3 grid((unsigned)((a.N + kRowsPerGroup * G - 1) / (kRowsPerGroup * G)),
                  (unsigned)batch);
  switch (M) {
    case 1: hipLaunchKernelGGL((linear_rows_kernel<1, LPR>), grid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL((linear_rows_kernel<2, LPR>), grid, dim3(64), 0, st, a); break;
    case 3: hipLaunchKernelGGL((linear_rows_kernel<3, LPR>), grid, dim3(64), 0, st, a); break;
    default: hipLaunchKernelGGL((linear_rows_kernel<4, LPR>), grid, dim3(64), 0, st, a); break;
  }
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_linear_rows(const dsk_bf16* x, int64_t ld_x, int64_t x_batch_stride,
                               const dsk_bf16* w_tiled, int64_t w_batch_stride, dsk_bf16* out0,
                               int64_t ld_out0, int64_t out0_batch_stride, dsk_bf16* out1,
                               int64_t ld_out1, int64_t out1_batch_stride, int n_split,
                               int batch, int M, int K, int N, void* stream) {
  DSK_REQUIRE(batch >= 0 && M >= 0 && K > 0 && N > 0, DSK_ERR_INVALID_ARG,
              "linear_rows: invalid sizes");
  DSK_REQUIRE(M <= 4, DSK_ERR_INVALID_ARG, "linear_rows: at most 4 token rows");
  DSK_REQUIRE(K % 128 == 0 && N % 32 == 0, DSK_ERR_INVALID_ARG,
              "linear_rows: K must be a multiple of 128 and N of 32 (tiled weight)");
  DSK_REQUIRE(n_split >= 0 && n_split <= N, DSK_ERR_INVALID_ARG,
              "linear_rows: n_split must be in [0, N]");
  if (batch == 0 || M == 0) return DSK_OK;
  DSK_REQUIRE(x && w_tiled && (n_split == 0 || out0) && (n_split == N || out1),
              DSK_ERR_NULL_PTR, "linear_rows: NULL pointer");
  DSK_REQUIRE(aligned16(x) && aligned16(w_tiled) && ld_x % 8 == 0 && x_batch_stride % 8 == 0 &&
                  w_batch_stride % 8 == 0,
              DSK_ERR_ALIGNMENT, "linear_rows: x rows and weights must be 16-byte aligned");
  DSK_REQUIRE(ld_x >= K && (n_split == 0 || ld_out0 >= n_split) &&
                  (n_split == N || ld_out1 >= N - n_split),
              DSK_ERR_INVALID_ARG, "linear_rows: row stride smaller than the row");
  DSK_REQUIRE(batch <= 65535, DSK_ERR_INVALID_ARG, "linear_rows: batch must be at most 65535");
  RowsArgs a{reinterpret_cast<const uint16_t*>(x), ld_x, x_batch_stride,
             reinterpret_cast<const uint16_t*>(w_tiled), w_batch_stride,
             reinterpret_cast<uint16_t*>(out0), ld_out0, out0_batch_stride,
             reinterpret_cast<uint16_t*>(out1), ld_out1, out1_batch_stride, n_split, K, N};
  if (K % 512 == 0) launch_rows_lpr<64>(a, M, batch, as_stream(stream));
  else launch_rows_lpr<16>(a, M, batch, as_stream(stream));
  return check_launch("linear_rows_kernel");
}
