// Absorbed-MLA decode attention over the latent KV cache (gfx950).
//
// The reference keeps, per token, the raw compressed latent (512, before the
// RMSNorm) and the raw shared RoPE key (64, before RoPE) in its latent cache
// (src/kernels/mla_cache.py:29-219); its attention (mla.py:356-384) works on
// the up-projected K = kv_b(norm(latent)) and V. With the up-projection folded
// into the query (absorbed form), for query token i and head h:
//
//   score(h, j) = scale * ( q_abs[h] . (r_j x_j) + rope_i(q_pe[h]) . rope_j(k_pe_j) )
//   o_lat(h)    = sum_j softmax_j(score(h, .)) * r_j x_j
//
// where x_j is the raw latent of key j, r_j = rsqrt(mean(x_j^2) + eps) its RMS
// scale and q_abs[h] = (W_UK[h] * w)^T q_nope[h] with the norm weight w folded
// into the up-projection rows; the caller applies (W_UV[h] * w) to o_lat(h) and
// o_proj after it.
//
// RoPE without a permutation: the reference's RoPE (mla.py:196-205) maps the
// raw pair (x[2k], x[2k+1]) to output elements k and k + 32. Dot products do
// not care where an element sits as long as both operands agree, so query and
// key are both rotated pair-in-place (element k at 2k, element k + 32 at
// 2k + 1) and the raw k_pe is rotated in registers as it is loaded.
//
// attn_split_kernel: one workgroup per (batch, query token, key split); a split
// is one or more blocks of 64 keys, 16 per wave, walked with an online softmax.
// Scores: v_mfma_f32_16x16x32_bf16 with the keys as operand A in the cache's
// natural row layout (a lane holds 8 consecutive dims of one key) and the 16
// heads as operand B; the same fragments give each key's sum of squares. P.X:
// the block's latent rows are staged in LDS and the output is built
// transposed, O^T[dims][heads] += X^T (p r)^T, on the same MFMA: a lane reads 8
// dims of 8 keys with 16-byte LDS reads and regroups them in registers into the
// dim-major operand of 8 output tiles. Each split leaves its running max, sum
// and unnormalised output in a workspace; attn_merge_kernel rescales and sums
// the splits of a query token in a fixed order (no atomics) and writes bf16.
#include "dsk_common.hpp"

#include <math.h>

#include <algorithm>

namespace dsk {

constexpr int kLat = 512;     // latent width
constexpr int kRope = 64;     // RoPE key width
constexpr int kHeads = 16;
constexpr int kBlock = 64;      // keys per block: 4 waves x 16
constexpr int kMaxSplits = 256; // key splits per query token
constexpr int kLatPad = kLat + 8;  // LDS row pitch: 16 B of padding spreads rows over banks

// Rotate the 4 raw pairs (x[2k], x[2k+1]), k = k0..k0+3, held in xv by the
// angles of one position: returns (rot[k], rot[k + 32]) per pair, where
// rot[k] = x[2k] cos[k] - x[2k+1] sin[k] and
// rot[k + 32] = x[2k+1] cos[k + 32] + x[2k] sin[k + 32] (mla.py:196-205).
__device__ __forceinline__ u32x4_t rope_pairs(u32x4_t xv, u32x2_t clo, u32x2_t chi, u32x2_t slo,
                                              u32x2_t shi) {
  u32x4_t rv;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x0 = bf16lo(xv[e]), x1 = bf16hi(xv[e]);
    const uint32_t cl = clo[e >> 1], ch = chi[e >> 1], sl = slo[e >> 1], sh = shi[e >> 1];
    const float c_lo = (e & 1) ? bf16hi(cl) : bf16lo(cl);
    const float c_hi = (e & 1) ? bf16hi(ch) : bf16lo(ch);
    const float s_lo = (e & 1) ? bf16hi(sl) : bf16lo(sl);
    const float s_hi = (e & 1) ? bf16hi(sh) : bf16lo(sh);
    rv[e] = pack_bf16x2(x0 * c_lo - x1 * s_lo, x1 * c_hi + x0 * s_hi);
  }
  return rv;
}

// The angles of pairs k0..k0+3 of one position: cos[k0..], cos[k0+32..], sin[k0..], sin[k0+32..].
struct RopeAngles {
  u32x2_t clo, chi, slo, shi;
};
__device__ __forceinline__ RopeAngles load_angles(const uint16_t* crow, const uint16_t* srow,
                                                  int k0) {
  RopeAngles r;
  r.clo = *reinterpret_cast<const u32x2_t*>(crow + k0);
  r.chi = *reinterpret_cast<const u32x2_t*>(crow + kRope / 2 + k0);
  r.slo = *reinterpret_cast<const u32x2_t*>(srow + k0);
  r.shi = *reinterpret_cast<const u32x2_t*>(srow + kRope / 2 + k0);
  return r;
}
__device__ __forceinline__ u32x4_t rope_pairs(u32x4_t xv, const RopeAngles& r) {
  return rope_pairs(xv, r.clo, r.chi, r.slo, r.shi);
}

struct DecodeArgs {
  const uint16_t* q_abs;   // token t, head h at t * qa_tok + h * qa_head (512 wide)
  int64_t qa_tok, qa_head;
  const uint16_t* q_pe;    // raw query RoPE part, t * qp_tok + h * qp_head (64 wide)
  int64_t qp_tok, qp_head;
  const uint16_t* latent;  // cache token j of sequence b at b * ld_batch + j * ld_tok
  const uint16_t* kpe;     // same strides
  int64_t ld_tok, ld_batch;
  const uint16_t* cos_t;   // [positions, 64], row = position
  const uint16_t* sin_t;
  float eps, scale;
  int L, Q;
  int n_splits;            // key splits per query token
  int split_blocks;        // 64-key blocks per split
  float* part_o;           // [B * Q, n_splits, 8192] in MFMA fragment order (see below)
  float* part_ml;          // [B * Q, n_splits, 2, 16] (running max, sum) per head
  uint16_t* out;           // token t, head h at t * o_tok + h * o_head (512 wide)
  int64_t o_tok, o_head;
};

// Key of slot s (0..31) inside one 32-key MFMA step. Lane group g feeds slots
// 8g..8g+7 of operand B; slot 8g + e holds key (e >> 1) * 8 + 2g + (e & 1), so
// that at a fixed e the 4 lane groups read LDS rows two apart (rows 8 apart
// would hit the same banks at this row pitch).
__device__ __forceinline__ int slot_of_key(int k) {  // k < 32
  return 8 * ((k >> 1) & 3) + (((k >> 3) << 1) | (k & 1));
}
__device__ __forceinline__ int key_of_slot(int g, int e) { return (e >> 1) * 8 + 2 * g + (e & 1); }

// Partial output of a split, per wave w (dims w*128 .. w*128+127), tile t < 8 and
// lane: 4 floats, element i = head (lane & 15), dim w*128 + 8*(4*(lane>>4) + i) + t.
__device__ __forceinline__ int frag_dim(int w, int t, int lane, int i) {
  return w * 128 + 8 * (4 * (lane >> 4) + i) + t;
}

__global__ __launch_bounds__(256, 2) void attn_split_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t s_x[kBlock][kLatPad];       // 65 KB
  __shared__ __attribute__((aligned(16))) uint16_t s_p[kHeads][kBlock + 8];    // P'^T by slot
  __shared__ float s_max[4][kHeads], s_l[4][kHeads];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int split = blockIdx.x, qi = blockIdx.y, b = blockIdx.z;
  const int L = a.L;
  const int pos_q = L - a.Q + qi;  // cache position of this query token
  const int64_t tok = (int64_t)b * a.Q + qi;
  const int r16 = lane & 15, g = lane >> 4;
  const int k_begin = split * a.split_blocks * kBlock;
  const int k_end = min(min(L, pos_q + 1), k_begin + a.split_blocks * kBlock);  // visible keys

  const uint16_t* xbase = a.latent + (int64_t)b * a.ld_batch;
  const uint16_t* pbase = a.kpe + (int64_t)b * a.ld_batch;
  // cache fragments of a block: lane holds key r16 of the wave's 16, dims
  // 8g..8g+7 of each 32-dim step, and that key's RoPE angles
  u32x4_t xv[kLat / 32], pv[kRope / 32];
  RopeAngles ka[kRope / 32];
  auto load_block = [&](int kb) {
    const int key = kb + wave * 16 + r16;
    const int keyc = key < L ? key : L - 1;  // clamped for loads; masked below
    const uint16_t* xrow = xbase + (int64_t)keyc * a.ld_tok;
    const uint16_t* prow = pbase + (int64_t)keyc * a.ld_tok;
#pragma unroll
    for (int ks = 0; ks < kLat / 32; ++ks)
      xv[ks] = *reinterpret_cast<const u32x4_t*>(xrow + ks * 32 + 8 * g);
#pragma unroll
    for (int ks = 0; ks < kRope / 32; ++ks) {
      pv[ks] = *reinterpret_cast<const u32x4_t*>(prow + ks * 32 + 8 * g);
      ka[ks] = load_angles(a.cos_t + (int64_t)keyc * kRope, a.sin_t + (int64_t)keyc * kRope,
                           (ks * 32 + 8 * g) / 2);
    }
  };
  // query fragments (operand B of the scores, head r16): loop invariant. The
  // 16 KB of q_abs rows are fetched once per workgroup and handed to the waves
  // through LDS rows 0..15 of s_x (free until the first block is staged); the
  // first block's loads are issued in between, so both latencies overlap.
  u32x4_t qv[kLat / 32], qr[kRope / 32];
  {
    u32x4_t qst[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = threadIdx.x + 256 * j;  // 16 heads x 64 pieces of 16 B
      qst[j] = *reinterpret_cast<const u32x4_t*>(a.q_abs + tok * a.qa_tok +
                                                 (c >> 6) * a.qa_head + (c & 63) * 8);
    }
    const uint16_t* qp = a.q_pe + tok * a.qp_tok + r16 * a.qp_head;
    u32x4_t qpv[kRope / 32];
#pragma unroll
    for (int ks = 0; ks < kRope / 32; ++ks)
      qpv[ks] = *reinterpret_cast<const u32x4_t*>(qp + ks * 32 + 8 * g);
    if (k_begin < k_end) load_block(k_begin);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = threadIdx.x + 256 * j;
      *reinterpret_cast<u32x4_t*>(&s_x[c >> 6][(c & 63) * 8]) = qst[j];
    }
#pragma unroll
    for (int ks = 0; ks < kRope / 32; ++ks) {
      const int d0 = ks * 32 + 8 * g;
      qr[ks] = rope_pairs(qpv[ks], load_angles(a.cos_t + (int64_t)pos_q * kRope,
                                               a.sin_t + (int64_t)pos_q * kRope, d0 / 2));
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kLat / 32; ++ks)
      qv[ks] = *reinterpret_cast<const u32x4_t*>(&s_x[r16][ks * 32 + 8 * g]);
    __syncthreads();  // every wave holds its copy before s_x is overwritten
  }

  float m_run = -INFINITY;  // running max of head r16 (same in every wave)
  float l_lane = 0.f;       // this lane's share of the running sum of head r16
  floatx4_t acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  for (int kb = k_begin; kb < k_end; kb += kBlock) {
    // ---- scores of the wave's 16 keys: latent part, RMS statistics, RoPE part
    floatx4_t acc_n = {0.f, 0.f, 0.f, 0.f}, acc_r = {0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < kLat / 32; ++ks) {
      *reinterpret_cast<u32x4_t*>(&s_x[wave * 16 + r16][ks * 32 + 8 * g]) = xv[ks];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = bf16lo(xv[ks][e]), x1 = bf16hi(xv[ks][e]);
        ss = fmaf(x0, x0, ss);
        ss = fmaf(x1, x1, ss);
      }
      acc_n = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xv[ks]),
                                                      __builtin_bit_cast(bf16x8_t, qv[ks]),
                                                      acc_n, 0, 0, 0);
    }
#pragma unroll
    for (int ks = 0; ks < kRope / 32; ++ks) {
      const u32x4_t kv = rope_pairs(pv[ks], ka[ks]);
      acc_r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kv),
                                                      __builtin_bit_cast(bf16x8_t, qr[ks]),
                                                      acc_r, 0, 0, 0);
    }
    // RMS scale of this lane's key: lanes r16 + 16 g (g < 4) hold its 4 dim groups
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    const float r_key = rsqrtf(ss * (1.f / kLat) + a.eps);

    // ---- scores in the MFMA output layout: lane holds keys 4g + i of head r16
    float sc[4], rk[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kr = 4 * g + i;
      rk[i] = __shfl(r_key, kr, 64);  // lane kr holds key kr's scale
      const bool ok = kb + wave * 16 + kr < k_end;
      sc[i] = ok ? a.scale * (rk[i] * acc_n[i] + acc_r[i]) : -INFINITY;
      mx = fmaxf(mx, sc[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (lane < 16) s_max[wave][lane] = mx;
    __syncthreads();  // s_max, s_x complete
    // key kb is visible, so the block max is finite
    const float m_new = fmaxf(m_run, fmaxf(fmaxf(s_max[0][r16], s_max[1][r16]),
                                           fmaxf(s_max[2][r16], s_max[3][r16])));
    const float alpha = __expf(m_run - m_new);  // 0 on the first block
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = sc[i] == -INFINITY ? 0.f : __expf(sc[i] - m_new);
      psum += p;
      const int kr = wave * 16 + 4 * g + i;  // key within the block
      s_p[r16][(kr & 32) + slot_of_key(kr & 31)] = f32_to_bf16(p * rk[i]);
    }
    l_lane = fmaf(l_lane, alpha, psum);
    __syncthreads();  // s_p complete

    // ---- O^T[dims][heads] += X^T P'^T over the block's 64 keys (2 MFMA steps)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] *= alpha;  // output lane holds head r16
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4_t bp = *reinterpret_cast<const u32x4_t*>(&s_p[r16][ks * 32 + 8 * g]);
      u32x4_t w[8];  // 8 keys x dims wave*128 + 8 r16 .. +7
#pragma unroll
      for (int e = 0; e < 8; ++e)
        w[e] = *reinterpret_cast<const u32x4_t*>(
            &s_x[ks * 32 + key_of_slot(g, e)][wave * 128 + 8 * r16]);
#pragma unroll
      for (int t = 0; t < 8; ++t) {  // tile t: dim wave*128 + 8 r16 + t of each key
        u32x4_t fa;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = w[2 * j][t >> 1], hi = w[2 * j + 1][t >> 1];
          fa[j] = (t & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, fa),
                                                         __builtin_bit_cast(bf16x8_t, bp),
                                                         acc[t], 0, 0, 0);
      }
    }
    if (kb + kBlock < k_end) {
      load_block(kb + kBlock);  // in flight while the waves meet at the barrier
      __syncthreads();          // this block's P.X reads of s_x / s_p done
    }
  }

  // ---- split statistics and partial output
  l_lane += __shfl_xor(l_lane, 16, 64);
  l_lane += __shfl_xor(l_lane, 32, 64);
  if (lane < 16) s_l[wave][lane] = l_lane;
  __syncthreads();  // also: every wave is past its last read of s_x
  if (a.n_splits == 1) {
    // The only split holds every visible key (key 0 among them, so the sum is
    // >= 1): normalise here and write bf16, staged through s_x for whole-row
    // stores; no merge pass follows.
    const float inv = 1.f / ((s_l[0][r16] + s_l[1][r16]) + (s_l[2][r16] + s_l[3][r16]));
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_x[r16][frag_dim(wave, t, lane, i)] = f32_to_bf16(acc[t][i] * inv);
    __syncthreads();
    uint16_t* o = a.out + tok * a.o_tok;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int c = threadIdx.x + 256 * j;  // 16 heads x 256 bf16 pairs
      const int h = c >> 8, d = (c & 255) * 2;
      *reinterpret_cast<uint32_t*>(o + h * a.o_head + d) =
          *reinterpret_cast<const uint32_t*>(&s_x[h][d]);
    }
    return;
  }
  const int64_t part = tok * a.n_splits + split;
  if (threadIdx.x < kHeads) {  // thread t < 16 is lane t of wave 0: head t
    const int h = threadIdx.x;
    float* ml = a.part_ml + part * 2 * kHeads;
    ml[h] = m_run;
    ml[kHeads + h] = (s_l[0][h] + s_l[1][h]) + (s_l[2][h] + s_l[3][h]);
  }
  if (k_begin < k_end) {  // a split with no visible key leaves its partial unwritten
    float* po = a.part_o + part * (kHeads * kLat) + wave * 8 * 256;
#pragma unroll
    for (int t = 0; t < 8; ++t)
      *reinterpret_cast<floatx4_t*>(po + t * 256 + lane * 4) = acc[t];
  }
}

// Merge of a query token's splits: out = sum_s exp(m_s - m) O_s / sum_s exp(m_s - m) l_s
// per head. Workgroup (slice, token) owns 16 fragment-order float4s (256 B of
// each split's partial, one per head); its 16 split lanes sum consecutive
// sixteenths of the splits, 4 loads in flight, and the sixteenths are added in
// a fixed order (no atomics). Splits with no visible key (m_s = -inf)
// contribute nothing.
__global__ __launch_bounds__(256) void attn_merge_kernel(DecodeArgs a) {
  __shared__ float s_f[kMaxSplits][kHeads];  // exp(m_s - m) per split and head
  __shared__ float s_red[16][kHeads];
  __shared__ floatx4_t s_acc[16][16];
  const int S = a.n_splits;
  const int64_t tok = blockIdx.y;
  const float* ml = a.part_ml + tok * S * 2 * kHeads;
  const int h16 = threadIdx.x & 15, sl = threadIdx.x >> 4;  // head, split lane (16)
  float m = -INFINITY;
  for (int s = sl; s < S; s += 16) m = fmaxf(m, ml[s * 2 * kHeads + h16]);
  s_red[sl][h16] = m;
  __syncthreads();
  m = -INFINITY;
#pragma unroll
  for (int i = 0; i < 16; ++i) m = fmaxf(m, s_red[i][h16]);
  __syncthreads();
  float den = 0.f;
  for (int s = sl; s < S; s += 16) {
    const float ms = ml[s * 2 * kHeads + h16];
    const float f = ms == -INFINITY ? 0.f : __expf(ms - m);
    s_f[s][h16] = f;
    den = fmaf(f, ml[s * 2 * kHeads + kHeads + h16], den);
  }
  s_red[sl][h16] = den;
  __syncthreads();
  den = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) den += s_red[i][h16];  // fixed order
  const float inv = 1.f / den;  // split 0 holds key 0, so den >= 1

  const int e4 = blockIdx.x * 16 + h16;  // fragment-order float4 index
  const int ln = e4 & 63;
  const int head = ln & 15;              // == h16
  const float* po = a.part_o + tok * S * (kHeads * kLat) + (int64_t)e4 * 4;
  const int s0 = (S * sl) >> 4, s1 = (S * (sl + 1)) >> 4;
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
  int s = s0;
  for (; s + 4 <= s1; s += 4) {
    floatx4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      v[u] = *reinterpret_cast<const floatx4_t*>(po + (int64_t)(s + u) * (kHeads * kLat));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float f = s_f[s + u][head];
      if (f != 0.f) acc += f * v[u];
    }
  }
  for (; s < s1; ++s) {
    const float f = s_f[s][head];
    if (f != 0.f) acc += f * *reinterpret_cast<const floatx4_t*>(po + (int64_t)s * (kHeads * kLat));
  }
  s_acc[sl][h16] = acc;
  __syncthreads();
  if (sl == 0) {
    acc = s_acc[0][h16];
#pragma unroll
    for (int i = 1; i < 16; ++i) acc += s_acc[i][h16];  // fixed order
    const int wv = e4 >> 9, t = (e4 >> 6) & 7;
    uint16_t* o = a.out + tok * a.o_tok + head * a.o_head;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[frag_dim(wv, t, ln, i)] = f32_to_bf16(acc[i] * inv);
  }
}

}  // namespace dsk

using namespace dsk;

namespace {

#ifndef DSK_DECODE_WGS
#define DSK_DECODE_WGS 512
#endif

// Key splits per query token: enough workgroups to cover the chip about twice
// (DSK_DECODE_WGS), at most kMaxSplits, at least one 64-key block each.
void split_plan(int batch, int q_len, int kv_len, int* n_splits, int* split_blocks) {
  const int blocks = (kv_len + kBlock - 1) / kBlock;
  const int64_t tokens = (int64_t)batch * q_len;
  int want = (int)std::min<int64_t>(blocks, std::max<int64_t>(1, (DSK_DECODE_WGS + tokens - 1) / tokens));
  want = std::min(want, kMaxSplits);
  int per = (blocks + want - 1) / want;
  *split_blocks = per;
  *n_splits = (blocks + per - 1) / per;
}

}  // namespace

extern "C" size_t dsk_mla_decode_workspace_size(int batch, int q_len, int kv_len) {
  if (batch <= 0 || q_len <= 0 || kv_len <= 0) return 256;
  int S, per;
  split_plan(batch, q_len, kv_len, &S, &per);
  if (S == 1) return 256;  // one split per token writes the output itself
  const size_t per_token = (size_t)S * (kHeads * kLat + 2 * kHeads) * sizeof(float);
  return align_up((size_t)batch * q_len * per_token, 256);
}

extern "C" int dsk_mla_decode_attention(const dsk_bf16* q_abs, int64_t qa_tok, int64_t qa_head,
                                        const dsk_bf16* q_pe, int64_t qp_tok, int64_t qp_head,
                                        const dsk_bf16* latent, const dsk_bf16* k_pe,
                                        int64_t ld_tok, int64_t ld_batch,
                                        const dsk_bf16* cos_tab, const dsk_bf16* sin_tab,
                                        float eps, float scale, int batch, int q_len, int kv_len,
                                        dsk_bf16* o_latent, int64_t o_tok, int64_t o_head,
                                        void* workspace, size_t bytes, void* stream) {
  DSK_REQUIRE(batch >= 0 && q_len >= 0, DSK_ERR_INVALID_ARG,
              "mla_decode_attention: batch and q_len must be >= 0");
  if (batch == 0 || q_len == 0) return DSK_OK;
  DSK_REQUIRE(kv_len >= q_len, DSK_ERR_INVALID_ARG,
              "mla_decode_attention: need q_len <= kv_len (the new tokens are in the cache)");
  DSK_REQUIRE(ld_tok >= kRope && ld_tok % 8 == 0 && ld_batch % 8 == 0 &&
                  (batch == 1 || ld_batch >= (int64_t)kv_len * ld_tok),
              DSK_ERR_INVALID_ARG,
              "mla_decode_attention: token stride must be a multiple of 8 (>= 64) and the batch "
              "stride a multiple of 8 covering kv_len tokens");
  DSK_REQUIRE(qa_tok % 8 == 0 && qa_head % 8 == 0 && qp_tok % 8 == 0 && qp_head % 8 == 0 &&
                  o_tok % 2 == 0 && o_head % 2 == 0,
              DSK_ERR_ALIGNMENT,
              "mla_decode_attention: query strides must be multiples of 8, output strides of 2");
  DSK_REQUIRE(q_abs && q_pe && latent && k_pe && cos_tab && sin_tab && o_latent && workspace,
              DSK_ERR_NULL_PTR, "mla_decode_attention: NULL pointer");
  DSK_REQUIRE(aligned16(q_abs) && aligned16(q_pe) && aligned16(latent) && aligned16(k_pe) &&
                  aligned16(cos_tab) && aligned16(sin_tab) &&
                  (reinterpret_cast<uintptr_t>(o_latent) & 3u) == 0,
              DSK_ERR_ALIGNMENT,
              "mla_decode_attention: inputs must be 16-byte aligned, the output 4-byte aligned");
  DSK_REQUIRE((int64_t)batch * q_len <= 65535, DSK_ERR_INVALID_ARG,
              "mla_decode_attention: batch * q_len must be <= 65535");
  DSK_REQUIRE(bytes >= dsk_mla_decode_workspace_size(batch, q_len, kv_len), DSK_ERR_WORKSPACE,
              "mla_decode_attention: workspace too small");
  int S, per;
  split_plan(batch, q_len, kv_len, &S, &per);
  DecodeArgs a;
  a.q_abs = reinterpret_cast<const uint16_t*>(q_abs);
  a.qa_tok = qa_tok;
  a.qa_head = qa_head;
  a.q_pe = reinterpret_cast<const uint16_t*>(q_pe);
  a.qp_tok = qp_tok;
  a.qp_head = qp_head;
  a.latent = reinterpret_cast<const uint16_t*>(latent);
  a.kpe = reinterpret_cast<const uint16_t*>(k_pe);
  a.ld_tok = ld_tok;
  a.ld_batch = ld_batch;
  a.cos_t = reinterpret_cast<const uint16_t*>(cos_tab);
  a.sin_t = reinterpret_cast<const uint16_t*>(sin_tab);
  a.eps = eps;
  a.scale = scale;
  a.L = kv_len;
  a.Q = q_len;
  a.n_splits = S;
  a.split_blocks = per;
  a.part_ml = reinterpret_cast<float*>(workspace);
  a.part_o = a.part_ml + (size_t)batch * q_len * S * 2 * kHeads;  // 128-byte multiple
  a.out = reinterpret_cast<uint16_t*>(o_latent);
  a.o_tok = o_tok;
  a.o_head = o_head;
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(attn_split_kernel, dim3(S, q_len, batch), dim3(256), 0, st, a);
  int rc = check_launch("attn_split_kernel");
  if (rc || S == 1) return rc;
  hipLaunchKernelGGL(attn_merge_kernel, dim3(kHeads * kLat / 4 / 16, batch * q_len), dim3(256),
                     0, st, a);
  return check_launch("attn_merge_kernel");
}
