// Bandwidth-bound MLA helper kernels for gfx950: RMSNorm and interleaved RoPE.
//
// RMSNorm (reference module src/reference/mla.py:53-64, kernel
// src/kernels/mla/rms_norm.cu:47-120): y = w * x * rsqrt(mean(x^2) + eps) with
// fp32 math and one rounding of the output. One wave per row; the row stays in
// registers between the sum-of-squares pass and the scaling pass, so every
// element is read from HBM once. Row strides let a strided view (the 512-wide
// latent inside the 576-wide kv_a output) be normalised without a copy.
//
// RoPE (mla.py:176-206, rope.cu:61-95): input pairs (2k, 2k+1) map to outputs
// k and k + d/2. The pre-indexed cos/sin tables [B, 1, S, d] are broadcast
// over heads by index arithmetic instead of being materialised per head.
#include "dsk_common.hpp"

#include <algorithm>

namespace dsk {

template <typename T>
struct Vec8;
template <>
struct Vec8<uint16_t> {
  static __device__ __forceinline__ void load(const uint16_t* p, float (&x)[8]) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = bf16lo(v[j]);
      x[2 * j + 1] = bf16hi(v[j]);
    }
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float (&x)[8]) {
    u32x4_t v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = pack_bf16x2(x[2 * j], x[2 * j + 1]);
    *reinterpret_cast<u32x4_t*>(p) = v;
  }
};
template <>
struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&x)[8]) {
    const floatx4_t a = *reinterpret_cast<const floatx4_t*>(p);
    const floatx4_t b = *reinterpret_cast<const floatx4_t*>(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = a[j];
      x[4 + j] = b[j];
    }
  }
  static __device__ __forceinline__ void store(float* p, const float (&x)[8]) {
    floatx4_t a, b;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[j] = x[j];
      b[j] = x[4 + j];
    }
    *reinterpret_cast<floatx4_t*>(p) = a;
    *reinterpret_cast<floatx4_t*>(p + 4) = b;
  }
};

__device__ __forceinline__ float to_f(uint16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ float to_f(float v) { return v; }
__device__ __forceinline__ void from_f(float v, uint16_t* p) { *p = f32_to_bf16(v); }
__device__ __forceinline__ void from_f(float v, float* p) { *p = v; }

constexpr int kNormThreads = 256;  // 4 waves per workgroup

// NV = 8-element chunks held per lane in registers (H <= 512 * NV, H % 8 == 0).
// One row per wave, the row and the weight vector loaded before the reduction.
// At 16384 rows of 512 this measured fastest: 6.5 us against 7.9 us with 4 rows
// per wave and 9.1 us with 8 (more rows per wave meant fewer, longer waves that
// started their stores later), and 256-thread workgroups beat 64, 128 and 512.
template <typename Tin, typename Tout, int NV>
__global__ __launch_bounds__(kNormThreads) void rms_norm_vec_kernel(
    const Tin* __restrict__ in, int64_t ld_in, const float* __restrict__ w,
    Tout* __restrict__ out, int64_t ld_out, int rows, int H, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  floatx4_t w0[NV], w1[NV];
  float x[NV][8];
  const Tin* src = in + row * ld_in;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = lane + 64 * j;
    if (c * 8 < H) {
      Vec8<Tin>::load(src + c * 8, x[j]);
      w0[j] = *reinterpret_cast<const floatx4_t*>(w + c * 8);
      w1[j] = *reinterpret_cast<const floatx4_t*>(w + c * 8 + 4);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = lane + 64 * j;
    if (c * 8 < H) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(x[j][e], x[j][e], ss);
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)H + eps);
  Tout* dst = out + row * ld_out;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = lane + 64 * j;
    if (c * 8 < H) {
      float y[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y[e] = (x[j][e] * r) * w0[j][e];
        y[4 + e] = (x[j][4 + e] * r) * w1[j][e];
      }
      Vec8<Tout>::store(dst + c * 8, y);
    }
  }
}

// Any even H: scalar two-pass variant (the row is re-read, typically from L2).
template <typename Tin, typename Tout>
__global__ __launch_bounds__(kNormThreads) void rms_norm_scalar_kernel(
    const Tin* __restrict__ in, int64_t ld_in, const float* __restrict__ w,
    Tout* __restrict__ out, int64_t ld_out, int rows, int H, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const Tin* src = in + row * ld_in;
  float ss = 0.f;
  for (int c = lane; c < H; c += 64) {
    const float v = to_f(src[c]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)H + eps);
  Tout* dst = out + row * ld_out;
  for (int c = lane; c < H; c += 64) from_f((to_f(src[c]) * r) * w[c], dst + c);
}

template <typename Tin, typename Tout, int NV>
static void launch_rms_norm_nv(const Tin* in, int64_t ld_in, const float* w, Tout* out,
                               int64_t ld_out, int rows, int H, float eps, hipStream_t st) {
  const int per_wg = kNormThreads / 64;
  const unsigned grid = (unsigned)(((int64_t)rows + per_wg - 1) / per_wg);
  hipLaunchKernelGGL((rms_norm_vec_kernel<Tin, Tout, NV>), dim3(grid), dim3(kNormThreads), 0, st,
                     in, ld_in, w, out, ld_out, rows, H, eps);
}

template <typename Tin, typename Tout>
static int launch_rms_norm(const Tin* in, int64_t ld_in, const float* w, Tout* out,
                           int64_t ld_out, int rows, int H, float eps, hipStream_t st) {
  const unsigned grid = (unsigned)(((int64_t)rows + 3) / 4);
  const bool vec = H % 8 == 0 && H <= 4096 && aligned16(in) && aligned16(out) &&
                   aligned16(w) && (ld_in * (int64_t)sizeof(Tin)) % 16 == 0 &&
                   (ld_out * (int64_t)sizeof(Tout)) % 16 == 0;
  if (vec) {
    const int nv = (H + 511) / 512;
    if (nv <= 1) launch_rms_norm_nv<Tin, Tout, 1>(in, ld_in, w, out, ld_out, rows, H, eps, st);
    else if (nv <= 2) launch_rms_norm_nv<Tin, Tout, 2>(in, ld_in, w, out, ld_out, rows, H, eps, st);
    else if (nv <= 4) launch_rms_norm_nv<Tin, Tout, 4>(in, ld_in, w, out, ld_out, rows, H, eps, st);
    else launch_rms_norm_nv<Tin, Tout, 8>(in, ld_in, w, out, ld_out, rows, H, eps, st);
  } else {
    hipLaunchKernelGGL((rms_norm_scalar_kernel<Tin, Tout>), dim3(grid), dim3(kNormThreads), 0,
                       st, in, ld_in, w, out, ld_out, rows, H, eps);
  }
  return check_launch("rms_norm_kernel");
}

// ------------------------------------------------------------------- rope ---
// A thread owns NP input pairs (16 or 8 bytes of a row) of kRopeHeadsPerThread
// heads at one position: it loads the position's cos/sin at k and k + d/2 once
// and rotates each head's chunk with them (two stores per head, outputs k and
// k + d/2). At b=8, s=2048, 16 q heads + 1 k head of 64 dims this took the op
// from 14.0 to 13.0 us; 16 heads per thread measured 13.7 us.
constexpr int kRopeHeadsPerThread = 8;

struct RopeTensor {
  const uint16_t* x;
  int64_t sb, sh, ss;
  uint16_t* out;
  int heads;
};

// Division by a divisor fixed for the launch, for indices below 2^31, as a
// high multiply and a shift (Granlund and Montgomery, "Division by invariant
// integers using multiplication", 1994): with l = ceil(log2 d),
// m = ceil(2^(31+l) / d), q = umulhi(x, m) >> (l - 1); d = 1 is m = 0.
struct FastDiv {
  uint32_t m, s;
  int d;
};
static FastDiv make_fastdiv(int d) {
  FastDiv f{0u, 0u, d};
  if (d <= 1) return f;
  uint32_t l = 0;
  while ((1ull << l) < (uint64_t)d) ++l;
  f.m = (uint32_t)(((1ull << (31 + l)) + (uint64_t)d - 1) / (uint64_t)d);
  f.s = l - 1;
  return f;
}
__device__ __forceinline__ int fdiv(int x, const FastDiv& f) {
  return f.m == 0 ? x : (int)(__umulhi((uint32_t)x, f.m) >> f.s);
}

// NP consecutive bf16 values (NP = 4: 8 bytes, NP = 8: 16 bytes) as packed pairs
template <int NP>
__device__ __forceinline__ void load_bf16(const uint16_t* p, uint32_t (&v)[NP / 2]) {
  if constexpr (NP == 8) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = w[k];
  } else {
    const u32x2_t w = *reinterpret_cast<const u32x2_t*>(p);
    v[0] = w[0];
    v[1] = w[1];
  }
}
template <int NP>
__device__ __forceinline__ void store_bf16(uint16_t* p, const uint32_t (&v)[NP / 2]) {
  if constexpr (NP == 8) {
    *reinterpret_cast<u32x4_t*>(p) = u32x4_t{v[0], v[1], v[2], v[3]};
  } else {
    *reinterpret_cast<u32x2_t*>(p) = u32x2_t{v[0], v[1]};
  }
}

// NP = 8 pairs per thread when the rope dim is a multiple of 16, else 4; 32-bit
// index arithmetic, the item index split by multiply-shift division (the
// divisors are fixed per launch).
template <int NP>
__global__ __launch_bounds__(256) void rope_kernel(RopeTensor a, RopeTensor b, int items_a,
                                                   int items_b,
                                                   const uint16_t* __restrict__ cos_t,
                                                   const uint16_t* __restrict__ sin_t,
                                                   int64_t cb, int64_t cs, int d, FastDiv div_cpr,
                                                   FastDiv div_s, FastDiv div_ha,
                                                   FastDiv div_hb) {
  int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= items_a + items_b) return;
  const bool is_a = i < items_a;
  const RopeTensor& r = is_a ? a : b;
  if (!is_a) i -= items_a;
  const int half = d >> 1;
  // items run (batch, position, head group, chunk) with the chunk fastest, so
  // the lanes of a wave share a position's cos/sin row
  constexpr int HPT = kRopeHeadsPerThread;
  const int bsh = fdiv(i, div_cpr);
  const int c = i - bsh * div_cpr.d;
  const int hg = (r.heads + HPT - 1) / HPT;
  const int bs = fdiv(bsh, is_a ? div_ha : div_hb);
  const int h0 = (bsh - bs * hg) * HPT;
  const int bb = fdiv(bs, div_s);
  const int s = bs - bb * div_s.d;
  const int64_t toff = bb * cb + (int64_t)s * cs;
  uint32_t cl[NP / 2], ch[NP / 2], sl[NP / 2], sh[NP / 2];
  load_bf16<NP>(cos_t + toff + NP * c, cl);
  load_bf16<NP>(cos_t + toff + half + NP * c, ch);
  load_bf16<NP>(sin_t + toff + NP * c, sl);
  load_bf16<NP>(sin_t + toff + half + NP * c, sh);
  uint32_t xv[HPT][NP];
#pragma unroll
  for (int u = 0; u < HPT; ++u) {
    const int h = min(h0 + u, r.heads - 1);
    const uint16_t* xp = r.x + bb * r.sb + h * r.sh + (int64_t)s * r.ss + c * 2 * NP;
    load_bf16<NP>(xp, *reinterpret_cast<uint32_t(*)[NP / 2]>(&xv[u][0]));
    load_bf16<NP>(xp + NP, *reinterpret_cast<uint32_t(*)[NP / 2]>(&xv[u][NP / 2]));
  }
#pragma unroll
  for (int hh = 0; hh < HPT; ++hh) {
    const int h = h0 + hh;
    if (h >= r.heads) break;
    uint32_t olo[NP / 2], ohi[NP / 2];
#pragma unroll
    for (int j = 0; j < NP; j += 2) {
      float lo[2], hi[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int k = j + u;
        const float x0 = bf16lo(xv[hh][k]);  // x[2k]
        const float x1 = bf16hi(xv[hh][k]);  // x[2k+1]
        const float c_lo = u ? bf16hi(cl[k >> 1]) : bf16lo(cl[k >> 1]);
        const float c_hi = u ? bf16hi(ch[k >> 1]) : bf16lo(ch[k >> 1]);
        const float s_lo = u ? bf16hi(sl[k >> 1]) : bf16lo(sl[k >> 1]);
        const float s_hi = u ? bf16hi(sh[k >> 1]) : bf16lo(sh[k >> 1]);
        rope_pair(x0, x1, c_lo, c_hi, s_lo, s_hi, lo[u], hi[u]);
      }
      olo[j >> 1] = pack_bf16x2(lo[0], lo[1]);
      ohi[j >> 1] = pack_bf16x2(hi[0], hi[1]);
    }
    // output row (batch, head, position)
    uint16_t* op = r.out + (int64_t)((bb * r.heads + h) * div_s.d + s) * d;
    store_bf16<NP>(op + NP * c, olo);
    store_bf16<NP>(op + half + NP * c, ohi);
  }
}

static int check_rope(const void* x, int64_t sb, int64_t sh, int64_t ss, const void* out,
                      int d) {
  if (!x || !out) return fail(DSK_ERR_NULL_PTR, "rope: NULL pointer");
  if (!aligned16(x) || !aligned16(out) || sb % 8 || sh % 8 || ss % 8)
    return fail(DSK_ERR_ALIGNMENT, "rope: rows must be 16-byte aligned");
  (void)d;
  return DSK_OK;
}


// ------------------------------------------------------- attention softmax --
// In place over bf16 attention scores, rows of kv_len keys: the reference's
// eager sequence (mla.py:366-381) in one pass, p = softmax over keys of
// bf16(score * scale) + mask, in fp32, rounded once to bf16. The scaled score
// is rounded to bf16 first because the reference multiplies the bf16 matmul
// output by the scale in the model dtype.
// * Causal: key j of query i (query positions are the last q_len of the kv_len
//   keys) is masked for j > i + kv_len - q_len: its probability is 0 and its
//   score is never read.
// * Additive mask (mla.py:374, `attn_weights + attention_mask`): element j of the
//   row's mask row is added to the scaled score. The sum takes the dtype torch
//   promotes to: a bf16 mask gives a bf16 sum (rounded), an fp32 mask an fp32
//   sum. Mask rows are addressed by (batch, head, query) strides, so a
//   [b, 1, q, kv] mask broadcasts over the heads with a head stride of 0.
// * Keys from kv_len up to the row's next multiple of 8 are written as 0, so a
//   score buffer padded to 16-byte rows feeds the P.V product with exact zeros.
struct SoftmaxMask {
  const void* ptr;  // nullptr: no additive mask
  int f32;          // 1: fp32 elements, 0: bf16
  int heads;        // rows are (batch, head, query) with query fastest
  int64_t sb, sh, sq;  // element strides; key stride 1
};

__device__ __forceinline__ float mask_at(const SoftmaxMask& m, int64_t off) {
  return m.f32 ? reinterpret_cast<const float*>(m.ptr)[off]
               : bf16_to_f32(reinterpret_cast<const uint16_t*>(m.ptr)[off]);
}

// The scaled (and masked) score of key `col + e` from the loaded chunk w.
__device__ __forceinline__ float softmax_logit(uint32_t word, int e, float scale, const SoftmaxMask& m,
                                               int64_t moff, int col, int kv_len) {
  const float x = (e & 1) ? bf16hi(word) : bf16lo(word);
  float xs = bf16_to_f32(f32_to_bf16(x * scale));
  if (m.ptr != nullptr && col + e < kv_len) {
    const float mv = mask_at(m, moff + col + e);
    xs = m.f32 ? xs + mv : bf16_to_f32(f32_to_bf16(xs + mv));
  }
  return xs;
}

__device__ __forceinline__ int64_t softmax_mask_row(const SoftmaxMask& m, int64_t row, int q_len) {
  if (m.ptr == nullptr) return 0;
  const int64_t qi = row % q_len, bh = row / q_len;
  return (bh / m.heads) * m.sb + (bh % m.heads) * m.sh + qi * m.sq;
}

// One wave per row; a lane holds 8 consecutive keys of each 512-key chunk in
// registers (kv_len <= 512 * NC).
template <int NC>
__global__ __launch_bounds__(256) void attn_softmax_kernel(uint16_t* __restrict__ sc, int64_t ld,
                                                           int64_t rows, int kv_len, int q_len,
                                                           float scale, int causal,
                                                           SoftmaxMask mask) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // uniform over the wave
  uint16_t* p = sc + row * ld;
  const int qi = (int)(row % q_len);
  const int limit = causal ? min(kv_len, qi + 1 + (kv_len - q_len)) : kv_len;
  const int64_t moff = softmax_mask_row(mask, row, q_len);
  float v[NC][8];
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = c * 512 + lane * 8;
    u32x4_t w = u32x4_t{0u, 0u, 0u, 0u};
    if (col < limit) w = *reinterpret_cast<const u32x4_t*>(p + col);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[c][e] = col + e < limit ? softmax_logit(w[e / 2], e, scale, mask, moff, col, kv_len)
                                : -INFINITY;
      mx = fmaxf(mx, v[c][e]);
    }
  }
  mx = wave_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[c][e] = v[c][e] == -INFINITY ? 0.f : __expf(v[c][e] - mx);
      sum += v[c][e];
    }
  sum = wave_sum(sum);
  // one division per row, then products: within an fp32 ulp of p / sum, far
  // below the bf16 rounding of the result, and a fraction of the ALU work
  const float inv = 1.f / sum;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = c * 512 + lane * 8;
    if (col < kv_len) {
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(v[c][2 * e] * inv, v[c][2 * e + 1] * inv);
      *reinterpret_cast<u32x4_t*>(p + col) = o;
    }
  }
}

// Rows longer than the register-resident kernel holds (kv_len > 4096): one wave
// per row in two passes over 512-key chunks. The first keeps a running max and
// sum per lane (each lane's sum rescaled when its max grows), combined over the
// wave; the second recomputes the logits and writes exp(x - max) / sum. The
// probabilities are the single-pass kernel's formula with the sum accumulated
// in a different order.
__global__ __launch_bounds__(256) void attn_softmax_long_kernel(uint16_t* __restrict__ sc,
                                                                int64_t ld, int64_t rows,
                                                                int kv_len, int q_len, float scale,
                                                                int causal, SoftmaxMask mask) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // uniform over the wave
  uint16_t* p = sc + row * ld;
  const int qi = (int)(row % q_len);
  const int limit = causal ? min(kv_len, qi + 1 + (kv_len - q_len)) : kv_len;
  const int64_t moff = softmax_mask_row(mask, row, q_len);
  float m = -INFINITY, s = 0.f;
  for (int col = lane * 8; col < limit; col += 512) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(p + col);
    float x[8];
    float cm = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = col + e < limit ? softmax_logit(w[e / 2], e, scale, mask, moff, col, kv_len)
                             : -INFINITY;
      cm = fmaxf(cm, x[e]);
    }
    if (cm == -INFINITY) continue;
    if (cm > m) {
      s = m == -INFINITY ? 0.f : s * __expf(m - cm);
      m = cm;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) s += x[e] == -INFINITY ? 0.f : __expf(x[e] - m);
  }
  const float mx = wave_max(m);
  const float sum = wave_sum(m == -INFINITY ? 0.f : s * __expf(m - mx));
  const float inv = 1.f / sum;
  for (int col = lane * 8; col < kv_len; col += 512) {
    u32x4_t w = u32x4_t{0u, 0u, 0u, 0u};
    if (col < limit) w = *reinterpret_cast<const u32x4_t*>(p + col);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = col + e < limit ? softmax_logit(w[e / 2], e, scale, mask, moff, col, kv_len)
                                      : -INFINITY;
      y[e] = (x == -INFINITY ? 0.f : __expf(x - mx)) * inv;  // a fully masked row gives NaN, as torch
    }
    u32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(y[2 * e], y[2 * e + 1]);
    *reinterpret_cast<u32x4_t*>(p + col) = o;
  }
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_rms_norm(const dsk_bf16* in, int64_t ld_in, const float* weight,
                            dsk_bf16* out, int64_t ld_out, int rows, int hidden, float eps,
                            void* stream) {
  DSK_REQUIRE(hidden > 0 && hidden % 2 == 0, DSK_ERR_INVALID_ARG,
              "rms_norm: hidden_size must be even for bfloat162 vectorisation.");
  DSK_REQUIRE(rows >= 0, DSK_ERR_INVALID_ARG, "rms_norm: rows < 0");
  if (rows == 0) return DSK_OK;
  DSK_REQUIRE(in && weight && out, DSK_ERR_NULL_PTR, "rms_norm: NULL pointer");
  DSK_REQUIRE(ld_in >= hidden && ld_out >= hidden, DSK_ERR_INVALID_ARG,
              "rms_norm: row stride < hidden_size");
  return launch_rms_norm<uint16_t, uint16_t>(in, ld_in, weight, out, ld_out, rows, hidden, eps,
                                             as_stream(stream));
}

extern "C" int dsk_rms_norm_f32(const float* in, int64_t ld_in, const float* weight,
                                float* out, int64_t ld_out, int rows, int hidden, float eps,
                                void* stream) {
  DSK_REQUIRE(hidden > 0, DSK_ERR_INVALID_ARG, "rms_norm_f32: hidden_size must be positive");
  DSK_REQUIRE(rows >= 0, DSK_ERR_INVALID_ARG, "rms_norm_f32: rows < 0");
  if (rows == 0) return DSK_OK;
  DSK_REQUIRE(in && weight && out, DSK_ERR_NULL_PTR, "rms_norm_f32: NULL pointer");
  DSK_REQUIRE(ld_in >= hidden && ld_out >= hidden, DSK_ERR_INVALID_ARG,
              "rms_norm_f32: row stride < hidden_size");
  return launch_rms_norm<float, float>(in, ld_in, weight, out, ld_out, rows, hidden, eps,
                                       as_stream(stream));
}

extern "C" int dsk_rope_qk(const dsk_bf16* q, int64_t qsb, int64_t qsh, int64_t qss,
                           const dsk_bf16* k, int64_t ksb, int64_t ksh, int64_t kss,
                           const dsk_bf16* cos_t, const dsk_bf16* sin_t, int64_t cb,
                           int64_t cs, dsk_bf16* q_out, dsk_bf16* k_out, int B, int Hq,
                           int Hk, int S, int d, void* stream) {
  DSK_REQUIRE(d > 0 && d % 8 == 0 && d <= 256, DSK_ERR_INVALID_ARG,
              "rope: rope_dim must be a multiple of 8 in [8, 256]");
  DSK_REQUIRE(B >= 0 && Hq >= 0 && Hk >= 0 && S >= 0, DSK_ERR_INVALID_ARG,
              "rope: negative size");
  const int64_t rows_q = (int64_t)B * Hq * S;
  const int64_t rows_k = (int64_t)B * Hk * S;
  if (rows_q + rows_k == 0) return DSK_OK;
  DSK_REQUIRE(cos_t && sin_t, DSK_ERR_NULL_PTR, "rope: cos/sin is NULL");
  DSK_REQUIRE(aligned16(cos_t) && aligned16(sin_t) && cb % 8 == 0 && cs % 8 == 0,
              DSK_ERR_ALIGNMENT, "rope: cos/sin rows must be 16-byte aligned");
  int rc;
  if (rows_q && (rc = check_rope(q, qsb, qsh, qss, q_out, d))) return rc;
  if (rows_k && (rc = check_rope(k, ksb, ksh, kss, k_out, d))) return rc;
  DSK_REQUIRE((rows_q + rows_k) * (d / 8) < (int64_t)INT32_MAX, DSK_ERR_INVALID_ARG,
              "rope: more than 2^31 8-element chunks");
  RopeTensor a{q, qsb, qsh, qss, q_out, Hq > 0 ? Hq : 1};
  RopeTensor b{k, ksb, ksh, kss, k_out, Hk > 0 ? Hk : 1};
  const int np = d % 16 == 0 ? 8 : 4;  // pairs per thread
  const int cpr = d / (2 * np);          // threads per row
  const int64_t hpt = kRopeHeadsPerThread;
  const int items_q = (int)((int64_t)B * S * ((Hq + hpt - 1) / hpt) * cpr);
  const int items_k = (int)((int64_t)B * S * ((Hk + hpt - 1) / hpt) * cpr);
  const unsigned grid = (unsigned)(((int64_t)items_q + items_k + 255) / 256);
  const FastDiv dc = make_fastdiv(cpr), ds = make_fastdiv(S > 0 ? S : 1);
  // head groups of kRopeHeadsPerThread per (batch, position)
  const FastDiv dha = make_fastdiv((a.heads + kRopeHeadsPerThread - 1) / kRopeHeadsPerThread);
  const FastDiv dhb = make_fastdiv((b.heads + kRopeHeadsPerThread - 1) / kRopeHeadsPerThread);
  if (np == 8)
    hipLaunchKernelGGL(rope_kernel<8>, dim3(grid), dim3(256), 0, as_stream(stream), a, b, items_q,
                       items_k, cos_t, sin_t, cb, cs, d, dc, ds, dha, dhb);
  else
    hipLaunchKernelGGL(rope_kernel<4>, dim3(grid), dim3(256), 0, as_stream(stream), a, b, items_q,
                       items_k, cos_t, sin_t, cb, cs, d, dc, ds, dha, dhb);
  return check_launch("rope_kernel");
}

extern "C" int dsk_rope(const dsk_bf16* x, int64_t sb, int64_t sh, int64_t ss,
                        const dsk_bf16* cos_t, const dsk_bf16* sin_t, int64_t cb, int64_t cs,
                        dsk_bf16* out, int B, int Hh, int S, int d, void* stream) {
  return dsk_rope_qk(x, sb, sh, ss, nullptr, 0, 0, 0, cos_t, sin_t, cb, cs, out, nullptr, B, Hh,
                     0, S, d, stream);
}

// ----------------------------------------------- attention operand pack ---
// The full-sequence attention of DeepSeekMLA.forward (mla.py:354-366) multiplies
// query_states [b, h, s, 192] = (q_nope | rotated q_pe) by key_states^T, with
// key_states = (k_nope | rotated k_pe, broadcast over the heads), and the
// probabilities by value_states [b, h, s, 128]. The projections leave q, k_nope,
// v and k_pe as slices of token rows, so the batched products need them packed
// head-major first. One pass does it: Q (the nope part copied, the rope part
// rotated), K^T (k_nope and the rotated k_pe transposed through the LDS, 64
// positions per workgroup) and V. The rotation is the RoPE kernel's expression
// (rope_pair on bf16 table values), so Q and K^T are bitwise those of the RoPE
// kernel followed by the copies.
constexpr int kPackPos = 64;  // positions per workgroup
constexpr int kPackNope = 128, kPackRope = 64, kPackV = 128;
constexpr int kPackQK = kPackNope + kPackRope;  // 192: one Q row, one K column
constexpr int kPackChunks = kPackQK / 8;        // 16-byte chunks per K row in the tile
constexpr int kPackThreads = 256;

// 16-byte slot of chunk c of position p in the K tile. The chunk index is XORed
// with the position's octet (it stays inside its aligned block of 8 chunks), so
// the transposing reads, 8 octets x 8 dimension pairs per wave instruction,
// touch each LDS bank at most twice.
__device__ __forceinline__ int pack_slot(int p, int c) {
  return p * kPackChunks + (c ^ ((p >> 3) & 7));
}

__global__ __launch_bounds__(kPackThreads) void attn_pack_kernel(
    const uint16_t* __restrict__ q, int64_t ld_q, const uint16_t* __restrict__ kv,
    int64_t ld_kv, const uint16_t* __restrict__ kpe, int64_t ld_kpe,
    const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t, int64_t ld_cs,
    int64_t cs_bs, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_t,
    uint16_t* __restrict__ v_out, int S, int SP, int heads) {
  __shared__ u32x4_t tile[kPackPos * kPackChunks];  // K rows of the block, 24 KB
  const int tid = threadIdx.x;
  const int pos0 = blockIdx.x * kPackPos;
  const int hh = blockIdx.y;
  const int bi = blockIdx.z;
  const int npos = min(kPackPos, S - pos0);   // real positions of the block
  const int nall = min(kPackPos, SP - pos0);  // with the zero padding up to SP
  const int64_t bh = (int64_t)bi * heads + hh;
  const int64_t row0 = (int64_t)bi * S + pos0;  // token row of the block's first position
  cos_t += bi * cs_bs;
  sin_t += bi * cs_bs;

  // q nope -> Q, v -> V, k nope -> tile: 16 chunks per position each
#pragma unroll
  for (int r = 0; r < kPackPos * 16 / kPackThreads; ++r) {
    const int it = tid + kPackThreads * r;
    const int p = it >> 4, c = it & 15;
    if (p < npos) {
      const uint16_t* kvr = kv + (row0 + p) * ld_kv + hh * (kPackNope + kPackV);
      const u32x4_t qn =
          *reinterpret_cast<const u32x4_t*>(q + (row0 + p) * ld_q + hh * kPackQK + 8 * c);
      const u32x4_t kn = *reinterpret_cast<const u32x4_t*>(kvr + 8 * c);
      const u32x4_t vv = *reinterpret_cast<const u32x4_t*>(kvr + kPackNope + 8 * c);
      *reinterpret_cast<u32x4_t*>(q_out + (bh * S + pos0 + p) * kPackQK + 8 * c) = qn;
      *reinterpret_cast<u32x4_t*>(v_out + (bh * SP + pos0 + p) * kPackV + 8 * c) = vv;
      tile[pack_slot(p, c)] = kn;
    } else if (p < nall) {  // padding position: zero V row and K column
      const u32x4_t z = u32x4_t{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4_t*>(v_out + (bh * SP + pos0 + p) * kPackV + 8 * c) = z;
      tile[pack_slot(p, c)] = z;
      if (c < kPackChunks - 16) tile[pack_slot(p, 16 + c)] = z;
    }
  }
  // rotation, 8 pairs per item: q_pe into Q, k_pe into the tile
#pragma unroll
  for (int r = 0; r < 2 * kPackPos * 4 / kPackThreads; ++r) {
    const int it = tid + kPackThreads * r;
    const bool is_k = it >= kPackPos * 4;
    const int i2 = is_k ? it - kPackPos * 4 : it;
    const int p = i2 >> 2, c = i2 & 3;
    if (p < npos) {
      const uint16_t* x = is_k ? kpe + (row0 + p) * ld_kpe + 16 * c
                               : q + (row0 + p) * ld_q + hh * kPackQK + kPackNope + 16 * c;
      const uint16_t* ct = cos_t + (int64_t)(pos0 + p) * ld_cs + 8 * c;
      const uint16_t* st = sin_t + (int64_t)(pos0 + p) * ld_cs + 8 * c;
      const u32x4_t x0 = *reinterpret_cast<const u32x4_t*>(x);
      const u32x4_t x1 = *reinterpret_cast<const u32x4_t*>(x + 8);
      const u32x4_t cl = *reinterpret_cast<const u32x4_t*>(ct);
      const u32x4_t ch = *reinterpret_cast<const u32x4_t*>(ct + kPackRope / 2);
      const u32x4_t sl = *reinterpret_cast<const u32x4_t*>(st);
      const u32x4_t sh = *reinterpret_cast<const u32x4_t*>(st + kPackRope / 2);
      u32x4_t olo, ohi;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float lo[2], hi[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint32_t xw = (2 * j + u) < 4 ? x0[2 * j + u] : x1[2 * j + u - 4];
          const float c_lo = u ? bf16hi(cl[j]) : bf16lo(cl[j]);
          const float c_hi = u ? bf16hi(ch[j]) : bf16lo(ch[j]);
          const float s_lo = u ? bf16hi(sl[j]) : bf16lo(sl[j]);
          const float s_hi = u ? bf16hi(sh[j]) : bf16lo(sh[j]);
          rope_pair(bf16lo(xw), bf16hi(xw), c_lo, c_hi, s_lo, s_hi, lo[u], hi[u]);
        }
        olo[j] = pack_bf16x2(lo[0], lo[1]);
        ohi[j] = pack_bf16x2(hi[0], hi[1]);
      }
      if (is_k) {
        tile[pack_slot(p, 16 + c)] = olo;  // dims 128 + 8c .. : outputs k = 8c ..
        tile[pack_slot(p, 20 + c)] = ohi;  // dims 160 + 8c .. : outputs k + 32
      } else {
        uint16_t* qo = q_out + (bh * S + pos0 + p) * kPackQK + kPackNope + 8 * c;
        *reinterpret_cast<u32x4_t*>(qo) = olo;
        *reinterpret_cast<u32x4_t*>(qo + kPackRope / 2) = ohi;
      }
    }
  }
  __syncthreads();
  // K^T: rows 2dp and 2dp + 1, 8 positions (octet po) per item; 8 consecutive
  // lanes cover one 128-byte row segment of each
  const uint32_t* tw = reinterpret_cast<const uint32_t*>(tile);
  uint16_t* kt_bh = k_t + bh * kPackQK * SP + pos0;
#pragma unroll
  for (int r = 0; r < (kPackQK / 2) * 8 / kPackThreads; ++r) {
    const int it = tid + kPackThreads * r;
    const int po = it & 7, dp = it >> 3;
    if (8 * po < nall) {
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = tw[pack_slot(8 * po + i, dp >> 2) * 4 + (dp & 3)];
      u32x4_t lo, hi;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        lo[k] = __builtin_amdgcn_perm(w[2 * k + 1], w[2 * k], 0x05040100u);
        hi[k] = __builtin_amdgcn_perm(w[2 * k + 1], w[2 * k], 0x07060302u);
      }
      *reinterpret_cast<u32x4_t*>(kt_bh + (int64_t)(2 * dp) * SP + 8 * po) = lo;
      *reinterpret_cast<u32x4_t*>(kt_bh + (int64_t)(2 * dp + 1) * SP + 8 * po) = hi;
    }
  }
}

extern "C" int dsk_mla_attn_pack_ex(const dsk_bf16* q, int64_t ld_q, const dsk_bf16* kv,
                                    int64_t ld_kv, const dsk_bf16* k_pe, int64_t ld_kpe,
                                    const dsk_bf16* cos_t, const dsk_bf16* sin_t, int64_t ld_cs,
                                    int64_t cs_batch_stride, dsk_bf16* q_out, dsk_bf16* k_t,
                                    dsk_bf16* v_out, int batch, int seq, int seq_pad, int heads,
                                    int nope, int rope, int v_dim, void* stream) {
  DSK_REQUIRE(nope == kPackNope && rope == kPackRope && v_dim == kPackV, DSK_ERR_INVALID_ARG,
              "attn_pack: head dims must be nope 128, rope 64, v 128");
  DSK_REQUIRE(batch >= 0 && seq >= 0 && heads >= 0, DSK_ERR_INVALID_ARG,
              "attn_pack: negative size");
  if ((int64_t)batch * seq * heads == 0) return DSK_OK;
  DSK_REQUIRE(seq_pad % 8 == 0 && seq_pad >= seq && seq_pad - seq < 8, DSK_ERR_INVALID_ARG,
              "attn_pack: seq_pad must be seq rounded up to a multiple of 8");
  DSK_REQUIRE(batch <= 65535 && heads <= 65535, DSK_ERR_INVALID_ARG,
              "attn_pack: batch and heads must be at most 65535");
  DSK_REQUIRE(q && kv && k_pe && cos_t && sin_t && q_out && k_t && v_out, DSK_ERR_NULL_PTR,
              "attn_pack: NULL pointer");
  DSK_REQUIRE(aligned16(q) && aligned16(kv) && aligned16(k_pe) && aligned16(cos_t) &&
                  aligned16(sin_t) && aligned16(q_out) && aligned16(k_t) && aligned16(v_out) &&
                  ld_q % 8 == 0 && ld_kv % 8 == 0 && ld_kpe % 8 == 0 && ld_cs % 8 == 0 &&
                  cs_batch_stride % 8 == 0,
              DSK_ERR_ALIGNMENT, "attn_pack: rows must be 16-byte aligned");
  DSK_REQUIRE(ld_q >= (int64_t)heads * kPackQK && ld_kv >= (int64_t)heads * (kPackNope + kPackV) &&
                  ld_kpe >= kPackRope && ld_cs >= kPackRope && cs_batch_stride >= 0,
              DSK_ERR_INVALID_ARG, "attn_pack: row stride smaller than the row");
  const dim3 grid((unsigned)((seq + kPackPos - 1) / kPackPos), (unsigned)heads, (unsigned)batch);
  hipLaunchKernelGGL(attn_pack_kernel, grid, dim3(kPackThreads), 0, as_stream(stream),
                     reinterpret_cast<const uint16_t*>(q), ld_q,
                     reinterpret_cast<const uint16_t*>(kv), ld_kv,
                     reinterpret_cast<const uint16_t*>(k_pe), ld_kpe,
                     reinterpret_cast<const uint16_t*>(cos_t),
                     reinterpret_cast<const uint16_t*>(sin_t), ld_cs, cs_batch_stride,
                     reinterpret_cast<uint16_t*>(q_out), reinterpret_cast<uint16_t*>(k_t),
                     reinterpret_cast<uint16_t*>(v_out), seq, seq_pad, heads);
  return check_launch("attn_pack_kernel");
}

extern "C" int dsk_mla_attn_pack(const dsk_bf16* q, int64_t ld_q, const dsk_bf16* kv,
                                 int64_t ld_kv, const dsk_bf16* k_pe, int64_t ld_kpe,
                                 const dsk_bf16* cos_t, const dsk_bf16* sin_t, int64_t ld_cs,
                                 dsk_bf16* q_out, dsk_bf16* k_t, dsk_bf16* v_out, int batch,
                                 int seq, int heads, int nope, int rope, int v_dim,
                                 void* stream) {
  DSK_REQUIRE(seq % 8 == 0, DSK_ERR_INVALID_ARG,
              "attn_pack: seq must be a multiple of 8 (dsk_mla_attn_pack_ex pads other lengths)");
  return dsk_mla_attn_pack_ex(q, ld_q, kv, ld_kv, k_pe, ld_kpe, cos_t, sin_t, ld_cs, 0, q_out,
                              k_t, v_out, batch, seq, seq, heads, nope, rope, v_dim, stream);
}

namespace {
int attn_softmax_launch(dsk_bf16* scores, int64_t ld, int64_t rows, int kv_len, int q_len,
                        float scale, int causal, const SoftmaxMask& mask, void* stream) {
  DSK_REQUIRE(rows >= 0 && kv_len > 0 && q_len > 0, DSK_ERR_INVALID_ARG,
              "attn_softmax: rows >= 0, kv_len > 0 and q_len > 0 required");
  DSK_REQUIRE(rows % q_len == 0 && (!causal || q_len <= kv_len), DSK_ERR_INVALID_ARG,
              "attn_softmax: rows must be a multiple of q_len, and q_len <= kv_len when causal");
  if (rows == 0) return DSK_OK;
  DSK_REQUIRE(scores != nullptr, DSK_ERR_NULL_PTR, "attn_softmax: NULL pointer");
  DSK_REQUIRE(aligned16(scores) && ld % 8 == 0 && ld >= (int64_t)align_up((size_t)kv_len, 8),
              DSK_ERR_ALIGNMENT,
              "attn_softmax: rows must be 16-byte aligned with ld >= kv_len rounded up to 8");
  const unsigned grid = (unsigned)((rows + 3) / 4);
  uint16_t* s = reinterpret_cast<uint16_t*>(scores);
  hipStream_t st = as_stream(stream);
  if (kv_len <= 512)
    hipLaunchKernelGGL(attn_softmax_kernel<1>, dim3(grid), dim3(256), 0, st, s, ld, rows, kv_len,
                       q_len, scale, causal, mask);
  else if (kv_len <= 1024)
    hipLaunchKernelGGL(attn_softmax_kernel<2>, dim3(grid), dim3(256), 0, st, s, ld, rows, kv_len,
                       q_len, scale, causal, mask);
  else if (kv_len <= 2048)
    hipLaunchKernelGGL(attn_softmax_kernel<4>, dim3(grid), dim3(256), 0, st, s, ld, rows, kv_len,
                       q_len, scale, causal, mask);
  else if (kv_len <= 4096)
    hipLaunchKernelGGL(attn_softmax_kernel<8>, dim3(grid), dim3(256), 0, st, s, ld, rows, kv_len,
                       q_len, scale, causal, mask);
  else
    hipLaunchKernelGGL(attn_softmax_long_kernel, dim3(grid), dim3(256), 0, st, s, ld, rows,
                       kv_len, q_len, scale, causal, mask);
  return check_launch("attn_softmax_kernel");
}
}  // namespace

extern "C" int dsk_attn_softmax(dsk_bf16* scores, int64_t ld, int64_t rows, int kv_len,
                                int q_len, float scale, int causal, void* stream) {
  return attn_softmax_launch(scores, ld, rows, kv_len, q_len, scale, causal,
                             SoftmaxMask{nullptr, 0, 1, 0, 0, 0}, stream);
}

extern "C" int dsk_attn_softmax_masked(dsk_bf16* scores, int64_t ld, int64_t rows, int kv_len,
                                       int q_len, int heads, float scale, int causal,
                                       const void* mask, int mask_dtype, int64_t mask_sb,
                                       int64_t mask_sh, int64_t mask_sq, void* stream) {
  DSK_REQUIRE(mask_dtype == DSK_DTYPE_BF16 || mask_dtype == DSK_DTYPE_F32, DSK_ERR_INVALID_ARG,
              "attn_softmax: mask dtype must be DSK_DTYPE_BF16 or DSK_DTYPE_F32");
  DSK_REQUIRE(heads > 0 && (rows / (q_len > 0 ? q_len : 1)) % heads == 0, DSK_ERR_INVALID_ARG,
              "attn_softmax: rows / q_len must be a multiple of heads");
  DSK_REQUIRE(mask != nullptr || rows == 0, DSK_ERR_NULL_PTR, "attn_softmax: NULL mask");
  return attn_softmax_launch(scores, ld, rows, kv_len, q_len, scale, causal,
                             SoftmaxMask{mask, mask_dtype == DSK_DTYPE_F32 ? 1 : 0, heads,
                                         mask_sb, mask_sh, mask_sq},
                             stream);
}
