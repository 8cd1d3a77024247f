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
// Rotated keys are cached: beside the raw k_pe, each cache row holds
// rope_j(k_pe_j) in the reference's output layout (mla.py:196-205: raw pair
// (2k, 2k+1) -> outputs k and k + 32). Keys at positions below `rope_len` are
// read rotated; the ones from rope_len on (the tokens appended since the last
// call) are rotated here from the raw k_pe and the cos/sin tables and written
// back, so every key is rotated once. The query is rotated here the same way.
//
// attn_split_kernel: one workgroup per (batch, query token, key split); a
// split is one or more blocks of 64 keys, 16 per wave, walked with an online
// softmax. The blocks stream through a two-stage LDS ring filled by
// global->LDS DMA (raw latent rows and rotated keys): block i + 1's DMA is
// issued while block i is scored, one instruction after each score MFMA, so
// the wave never stalls long on a full memory queue and the loads of the next
// block overlap the math of this one.
//   Scores: v_mfma_f32_16x16x32_bf16 with the wave's 16 keys as operand A
//   (row layout, 16-byte LDS reads) and the 16 heads as operand B; the same
//   operand reads give each key's sum of squares (v_dot2 on the bf16 pairs),
//   so the RMS scale costs no extra read.
//   P.X: the output is built transposed, O^T[dims][heads] += X^T (p r)^T, on
//   the same MFMA: a lane reads 8 dims of 8 keys with 16-byte LDS reads and
//   regroups them with byte permutes into the dim-major operand of 8 output
//   tiles; wave w owns dims 128w..128w+127.
// Each split leaves its running max, sum and unnormalised output in a
// workspace; attn_merge_kernel rescales and sums the splits of a query token in
// a fixed order (no atomics) and writes bf16.
#include "dsk_common.hpp"

#include <math.h>

#include <algorithm>

namespace dsk {

constexpr int kLat = 512;     // latent width
constexpr int kRope = 64;     // RoPE key width
constexpr int kHeads = 16;
constexpr int kWaves = 4;  // compute waves (16 keys each per block)
// Waves that only issue the ring's DMA, beside the compute waves: a wave moves
// about 10 GB/s through the memory pipeline however many loads it keeps in
// flight, so 4 waves that also score and accumulate fetch a 75 KB block at
// ~22 GB/s per CU; with the loads on 4 more waves (2 per SIMD) the compute
// waves never stall on a full memory queue.
#ifndef DSK_ATTN_PRODUCERS
#define DSK_ATTN_PRODUCERS 4
#endif
constexpr int kProducers = DSK_ATTN_PRODUCERS;
constexpr int kSplitThreads = 64 * (kWaves + kProducers);
constexpr int kBlock = 64;                   // keys per block: 4 waves x 16
constexpr int kMaxSplits = 256;              // key splits per query token
// A stage of the ring, in 16-byte pieces: the block's 64 latent rows at a
// pitch of 65 pieces (1040 B), then its 64 rotated keys at a pitch of 9 pieces
// (144 B; slot 9k + 8 is padding). The odd pitches spread both the row reads
// of the scores (16 keys, one piece each) and the column reads of P.X (one key,
// 16 consecutive pieces) over the banks, and every read of a lane is a
// constant offset from one base address.
constexpr int kLatPitch = 1040;                               // bytes per latent row
constexpr int kRopePitch = 144;                               // bytes per rotated key
constexpr int kRopeOff = kBlock * kLatPitch;                  // 66,560
constexpr int kRopeDma = kBlock * 9 / 64;                     // 9 instructions of 64 slots
constexpr int kStageBytes = kRopeOff + kRopeDma * 1024;       // 75,776
constexpr int kStages = 2;
constexpr int kRingBytes = kStages * kStageBytes;             // 151,552
constexpr int kPPitch = kBlock + 8;                           // s_p row, bf16
static_assert(kRingBytes + kHeads * kPPitch * 2 + 2 * kWaves * kHeads * 4 <= 160 * 1024,
              "LDS budget");
static_assert(kHeads * kLatPitch + kHeads * kRope * 2 + 2048 <= kStageBytes, "query staging");

struct DecodeArgs {
  const uint16_t* q_abs;   // token t, head h at t * qa_tok + h * qa_head (512 wide)
  int64_t qa_tok, qa_head;
  const uint16_t* q_pe;    // raw query RoPE part, t * qp_tok + h * qp_head (64 wide)
  int64_t qp_tok, qp_head;
  const uint16_t* latent;  // cache token j of sequence b at b * ld_batch + j * ld_tok
  const uint16_t* kpe;     // raw RoPE key, same strides
  uint16_t* krope;         // rotated RoPE key, same strides
  int64_t ld_tok, ld_batch;
  const uint16_t* cos_t;   // [positions, 64], row = position
  const uint16_t* sin_t;
  float eps, scale;
  int L, Q, rope_len;
  int n_splits;            // key splits per query token
  int split_blocks;        // 64-key blocks per split
  float* part_o;           // [B * Q, n_splits, 8192] in MFMA fragment order (see below)
  float* part_ml;          // [B * Q, n_splits, 2, 16] (running max, sum) per head
  uint16_t* out;           // token t, head h at t * o_tok + h * o_head (512 wide)
  int64_t o_tok, o_head;
};

// Partial output of a split, per wave c (dims c*128 .. c*128+127), tile t < 8
// and lane: 4 floats, element i = head (lane & 15), dim c*128 + 8*(4*(lane>>4) + i) + t.
__device__ __forceinline__ int frag_dim(int c, int t, int lane, int i) {
  return c * 128 + 8 * (4 * (lane >> 4) + i) + t;
}

// Pieces g and 4 + g (elements 8g..8g+7 and 32+8g..32+8g+7) of the rotated
// 64-wide RoPE vector, from the raw elements 16g..16g+15 (x, two 16-byte
// pieces) and the angles cos/sin[8g..8g+7] and [32+8g..32+8g+7] of its position.
__device__ __forceinline__ void rope_pieces(const u32x4_t (&x)[2], u32x4_t clo, u32x4_t chi,
                                            u32x4_t slo, u32x4_t shi, u32x4_t& lo_piece,
                                            u32x4_t& hi_piece) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {  // output pair (2e, 2e+1) of each piece
    float lo[2], hi[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = 2 * e + u;                 // element 8g + j: raw pair j
      const uint32_t xr = x[j >> 2][j & 3];    // (x[2k], x[2k+1]) with k = 8g + j
      const float cl = u ? bf16hi(clo[e]) : bf16lo(clo[e]);
      const float ch = u ? bf16hi(chi[e]) : bf16lo(chi[e]);
      const float sl = u ? bf16hi(slo[e]) : bf16lo(slo[e]);
      const float sh = u ? bf16hi(shi[e]) : bf16lo(shi[e]);
      rope_pair(bf16lo(xr), bf16hi(xr), cl, ch, sl, sh, lo[u], hi[u]);
    }
    lo_piece[e] = pack_bf16x2(lo[0], lo[1]);
    hi_piece[e] = pack_bf16x2(hi[0], hi[1]);
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4_t lds_read16(uint32_t byte_addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
      (uintptr_t)byte_addr);
}

// Key of slot s (0..31) inside one 32-key MFMA step of P.X. Lane group g feeds
// slots 8g..8g+7 of operand B; slot 8g + e holds key (e >> 1) * 8 + 2g + (e & 1),
// so that at a fixed e the 4 lane groups read LDS rows two apart (rows 8 apart
// would hit the same banks at this row pitch).
__device__ __forceinline__ int slot_of_key(int k) {  // k < 32
  return 8 * ((k >> 1) & 3) + (((k >> 3) << 1) | (k & 1));
}
__device__ __forceinline__ int key_of_slot(int g, int e) { return (e >> 1) * 8 + 2 * g + (e & 1); }

// Global->LDS DMA of 1 KB (16 bytes per lane) like dma_1kb, without a memory
// clobber: the ring stage it fills is not read until a later barrier (an asm
// with a memory clobber), so the compiler may move the current stage's LDS
// reads across it.
__device__ __forceinline__ void dma_ring(const char* base, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(base), "s"(lds_addr) : "m0");
}

// Workgroup barrier after this wave's LDS accesses are done (lgkmcnt(0)),
// without __syncthreads()'s wait for the in-flight DMA of the next block.
__device__ __forceinline__ void lds_barrier_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__global__ __launch_bounds__(kSplitThreads, 1) void attn_split_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(1024))) char s_ring[kRingBytes];
  __shared__ __attribute__((aligned(16))) uint16_t s_p[kHeads][kPPitch];  // P'^T by slot
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
  const int n_blk = k_begin < k_end ? (k_end - k_begin + kBlock - 1) / kBlock : 0;

  const uint32_t ring0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_ring));
  const uint32_t ld_bytes = (uint32_t)a.ld_tok * 2;
  const char* lat_b = reinterpret_cast<const char*>(a.latent + (int64_t)b * a.ld_batch);
  const char* rope_b = reinterpret_cast<const char*>(a.krope + (int64_t)b * a.ld_batch);

  // This wave's share of the DMA of block kb into a stage: latent rows
  // 16 wave + j (one instruction each, lane l -> piece l) and rotated-key
  // instructions wave, wave + 4, wave + 8 (slot s = 64 r + l holds piece s % 9
  // of key s / 9; padding slots fetch piece 7). Rows past the cache are clamped
  // to its last row; their scores are masked.
  // dw: the issuing wave's slot 0..3 (a compute wave, or a producer wave - 4)
  const int dw = wave < kWaves ? wave : wave - kWaves;
  auto dma_lat = [&](int kb, uint32_t st, int j) __attribute__((always_inline)) {
    const int row = 16 * dw + j;
    dma_ring(lat_b, (uint32_t)min(kb + row, L - 1) * ld_bytes + (uint32_t)(lane << 4),
             st + row * kLatPitch);
  };
  auto dma_rope = [&](int kb, uint32_t st, int r) __attribute__((always_inline)) {
    const int sl = 64 * r + lane;
    const int k = sl / 9, p = min(sl - 9 * k, 7);
    dma_ring(rope_b, (uint32_t)min(kb + k, L - 1) * ld_bytes + (uint32_t)(p << 4),
             st + kRopeOff + r * 1024);
  };
  auto dma_block = [&](int kb, uint32_t st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 16; ++j) dma_lat(kb, st, j);
    for (int r = dw; r < kRopeDma; r += 4) dma_rope(kb, st, r);
  };

  // ---- query: q_abs rows (16 heads at the latent row pitch), raw q_pe (2 KB)
  // and the angles of pos_q (256 B), DMA'd into stage 1 (first written by block
  // 1's DMA, after the barrier at block 0), together with block 0.
  const uint32_t q_lds = ring0 + kStageBytes;
  const uint32_t qp_lds = q_lds + kHeads * kLatPitch;           // [16][64] raw q_pe
  const uint32_t ang_lds = qp_lds + kHeads * kRope * 2;         // cos row; sin row 1 KB on
  if (wave < kWaves) {
    const char* qa = reinterpret_cast<const char*>(a.q_abs + tok * a.qa_tok);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int h = 4 * wave + j;
      dma_1kb(qa, (uint32_t)(h * a.qa_head * 2 + (lane << 4)), q_lds + h * kLatPitch);
    }
    if (wave < 2) {  // raw q_pe: lane l -> head 8 wave + l / 8, piece l % 8
      const char* qp = reinterpret_cast<const char*>(a.q_pe + tok * a.qp_tok);
      const int h = 8 * wave + (lane >> 3);
      dma_1kb(qp, (uint32_t)(h * a.qp_head * 2 + ((lane & 7) << 4)), qp_lds + wave * 1024);
    } else {  // the cos (wave 2) or sin (wave 3) row of pos_q: lanes 0..7 (the rest repeat)
      const char* tab = reinterpret_cast<const char*>(wave == 2 ? a.cos_t : a.sin_t);
      dma_1kb(tab, (uint32_t)((int64_t)pos_q * kRope * 2 + (min(lane, 7) << 4)),
              ang_lds + (wave - 2) * 1024);
    }
    if (kProducers == 0 && n_blk > 0) dma_block(k_begin, ring0);
  } else if (n_blk > 0) {
    dma_block(k_begin, ring0);
  }
  wait_vmcnt<0>();
  lds_barrier();
  if (kProducers > 0 && wave >= kWaves) {
    // Producer: block i + 1's DMA right after the barrier that frees its stage,
    // then the compute waves' two barriers of the block; the same barrier
    // count as theirs, to the end.
    for (int i = 0; i < n_blk; ++i) {
      wait_vmcnt<0>();
      lds_barrier();
      if (i + 1 < n_blk) dma_block(k_begin + (i + 1) * kBlock, ring0 + ((i + 1) & 1) * kStageBytes);
      lds_barrier_lgkm();  // s_max
      lds_barrier_lgkm();  // s_p
    }
    wait_vmcnt<0>();
    lds_barrier_lgkm();
    if (a.n_splits == 1) lds_barrier_lgkm();
    return;
  }
  u32x4_t qv[kLat / 32], qr[2];  // scores operand B: head r16, dims 8g.. of each 32-dim step
#pragma unroll
  for (int ks = 0; ks < kLat / 32; ++ks) qv[ks] = lds_read16(q_lds + r16 * kLatPitch + (4 * ks + g) * 16);
  {
    const u32x4_t x[2] = {lds_read16(qp_lds + r16 * 128 + 2 * g * 16),
                          lds_read16(qp_lds + r16 * 128 + (2 * g + 1) * 16)};
    rope_pieces(x, lds_read16(ang_lds + g * 16), lds_read16(ang_lds + (4 + g) * 16),
                lds_read16(ang_lds + 1024 + g * 16), lds_read16(ang_lds + 1024 + (4 + g) * 16),
                qr[0], qr[1]);
  }
  // the query is in registers before block 1's DMA reuses the staging (the
  // barrier at the top of block 0 publishes that)
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  float m_run = -INFINITY;  // running max of head r16 (same in every wave)
  float l_lane = 0.f;       // this lane's share of the running sum of head r16
  floatx4_t acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  const uint16_t* kpe_b = a.kpe + (int64_t)b * a.ld_batch;
  uint16_t* krope_b = a.krope + (int64_t)b * a.ld_batch;

  for (int i = 0; i < n_blk; ++i) {
    const int kb = k_begin + i * kBlock;
    const uint32_t st = ring0 + (i & 1) * kStageBytes;
    const uint32_t st_next = ring0 + ((i + 1) & 1) * kStageBytes;
    const bool more = i + 1 < n_blk;
    // Block i has landed (every wave waited for its own DMA), and every wave
    // is past its P.X of block i - 1, so the other stage is free.
    wait_vmcnt<0>();
    lds_barrier();
    const int key0 = kb + 16 * wave;

    // ---- scores of the wave's 16 keys, block i + 1's DMA in between
    floatx4_t acc_n = {0.f, 0.f, 0.f, 0.f}, acc_r = {0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
    u32x4_t xa[kLat / 32];
#pragma unroll
    for (int ks = 0; ks < kLat / 32; ++ks)
      xa[ks] = lds_read16(st + (16 * wave + r16) * kLatPitch + (4 * ks + g) * 16);
#pragma unroll
    for (int ks = 0; ks < kLat / 32; ++ks) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // the element goes through a scalar first: hipcc (ROCm 7.2) compiles
        // bit_cast(bf16x2, vector[e]) to element 0 for every e
        const uint32_t w = xa[ks][e];
        const bf16x2_t wb = __builtin_bit_cast(bf16x2_t, w);
        ss = __builtin_amdgcn_fdot2_f32_bf16(wb, wb, ss, false);
      }
      acc_n = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[ks]),
                                                      __builtin_bit_cast(bf16x8_t, qv[ks]),
                                                      acc_n, 0, 0, 0);
      if (kProducers == 0 && more) dma_lat(kb + kBlock, st_next, ks);
    }
    if (kProducers == 0 && more)
      for (int r = wave; r < kRopeDma; r += 4) dma_rope(kb + kBlock, st_next, r);
    u32x4_t kr[2];
    if (key0 + 16 > a.rope_len) {
      // keys not rotated yet: rotate from the raw k_pe; the last query token's
      // workgroup stores them for later calls (every other workgroup that
      // reads these keys in this launch rotates them itself)
      const int key = min(key0 + r16, L - 1);
      const uint16_t* xr = kpe_b + (int64_t)key * a.ld_tok + 16 * g;
      const u32x4_t x[2] = {*reinterpret_cast<const u32x4_t*>(xr),
                            *reinterpret_cast<const u32x4_t*>(xr + 8)};
      const uint16_t* cr = a.cos_t + (int64_t)key * kRope + 8 * g;
      const uint16_t* sr = a.sin_t + (int64_t)key * kRope + 8 * g;
      rope_pieces(x, *reinterpret_cast<const u32x4_t*>(cr), *reinterpret_cast<const u32x4_t*>(cr + 32),
                  *reinterpret_cast<const u32x4_t*>(sr), *reinterpret_cast<const u32x4_t*>(sr + 32),
                  kr[0], kr[1]);
      if (qi == a.Q - 1 && key0 + r16 >= a.rope_len && key0 + r16 < L) {
        uint16_t* kw = krope_b + (int64_t)(key0 + r16) * a.ld_tok + 8 * g;
        *reinterpret_cast<u32x4_t*>(kw) = kr[0];
        *reinterpret_cast<u32x4_t*>(kw + 32) = kr[1];
      }
    } else {
      const uint32_t kp = st + kRopeOff + (16 * wave + r16) * kRopePitch;
      kr[0] = lds_read16(kp + g * 16);
      kr[1] = lds_read16(kp + (4 + g) * 16);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      acc_r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[ks]),
                                                      __builtin_bit_cast(bf16x8_t, qr[ks]),
                                                      acc_r, 0, 0, 0);
    // RMS scale of this lane's key: lanes r16 + 16 g (g < 4) hold its 4 dim groups
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    const float r_key = rsqrtf(ss * (1.f / kLat) + a.eps);

    // ---- scores in the MFMA output layout: lane holds keys 4g + i of head r16
    float sc[4], rk[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
      const int kr_ = 4 * g + i2;
      rk[i2] = __shfl(r_key, kr_, 64);  // lane kr_ holds key kr_'s scale
      sc[i2] = key0 + kr_ < k_end ? a.scale * (rk[i2] * acc_n[i2] + acc_r[i2]) : -INFINITY;
      mx = fmaxf(mx, sc[i2]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (lane < 16) s_max[wave][lane] = mx;
    lds_barrier_lgkm();  // s_max complete
    // key kb is visible, so the block max is finite
    const float m_new = fmaxf(m_run, fmaxf(fmaxf(s_max[0][r16], s_max[1][r16]),
                                           fmaxf(s_max[2][r16], s_max[3][r16])));
    const float alpha = __expf(m_run - m_new);  // 0 on the first block
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
      const float p = sc[i2] == -INFINITY ? 0.f : __expf(sc[i2] - m_new);
      psum += p;
      const int kr_ = 16 * wave + 4 * g + i2;  // key within the block
      s_p[r16][(kr_ & 32) + slot_of_key(kr_ & 31)] = f32_to_bf16(p * rk[i2]);
    }
    l_lane = fmaf(l_lane, alpha, psum);
    lds_barrier_lgkm();  // s_p complete

    // ---- O^T[dims][heads] += X^T P'^T over the block's 64 keys (2 MFMA steps)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] *= alpha;  // output lane holds head r16
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4_t bp = *reinterpret_cast<const u32x4_t*>(&s_p[r16][ks * 32 + 8 * g]);
      u32x4_t w[8];  // 8 keys x dims wave*128 + 8 r16 .. +7
#pragma unroll
      for (int e = 0; e < 8; ++e)
        w[e] = lds_read16(st + (ks * 32 + key_of_slot(g, e)) * kLatPitch + (wave * 16 + r16) * 16);
#pragma unroll
      for (int t = 0; t < 8; ++t) {  // tile t: dim wave*128 + 8 r16 + t of each key
        const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
        u32x4_t fa;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          fa[j] = __builtin_amdgcn_perm(w[2 * j + 1][t >> 1], w[2 * j][t >> 1], sel);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, fa),
                                                         __builtin_bit_cast(bf16x8_t, bp),
                                                         acc[t], 0, 0, 0);
      }
    }
  }

  // ---- split statistics and partial output
  l_lane += __shfl_xor(l_lane, 16, 64);
  l_lane += __shfl_xor(l_lane, 32, 64);
  if (lane < 16) s_l[wave][lane] = l_lane;
  wait_vmcnt<0>();
  lds_barrier_lgkm();  // also: every wave is past its last read of the ring
  if (a.n_splits == 1) {
    // The only split holds every visible key (key 0 among them, so the sum is
    // >= 1): normalise here and write bf16, staged through the ring for
    // whole-row stores; no merge pass follows.
    const float inv = 1.f / ((s_l[0][r16] + s_l[1][r16]) + (s_l[2][r16] + s_l[3][r16]));
    uint16_t* s_o = reinterpret_cast<uint16_t*>(s_ring);  // [16][512]
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int i2 = 0; i2 < 4; ++i2) s_o[r16 * kLat + frag_dim(wave, t, lane, i2)] = f32_to_bf16(acc[t][i2] * inv);
    lds_barrier_lgkm();
    uint16_t* op = a.out + tok * a.o_tok;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int cidx = threadIdx.x + 256 * j;  // 16 heads x 256 bf16 pairs (compute waves)
      const int h = cidx >> 8, d = (cidx & 255) * 2;
      *reinterpret_cast<uint32_t*>(op + h * a.o_head + d) =
          *reinterpret_cast<const uint32_t*>(&s_o[h * kLat + d]);
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
  if (n_blk > 0) {  // a split with no visible key leaves its partial unwritten
    float* po = a.part_o + part * (kHeads * kLat) + wave * 8 * 256;
#pragma unroll
    for (int t = 0; t < 8; ++t)
      *reinterpret_cast<floatx4_t*>(po + t * 256 + lane * 4) = acc[t];
  }
}

// Merge of a query token's splits: out = sum_s exp(m_s - m) O_s / sum_s exp(m_s - m) l_s
// per head. Workgroup (slice, token) owns 16 fragment-order float4s (256 B of
// each split's partial, one per head); its 16 split lanes take consecutive
// sixteenths of the splits. Every load (the partial slices and each split's
// max and sum) is issued up front, so the merge costs one memory round trip;
// the sums run in a fixed order (splits in order within a lane, lanes in
// order), with no atomics. Splits with no visible key (m_s = -inf) contribute
// nothing. NPL >= ceil(S / 16) splits per lane are loaded unconditionally (an
// index past the lane's last split repeats the token's last split and is
// masked), which keeps the loads free of branches and all in flight together.
template <int NPL>
__global__ __launch_bounds__(256) void attn_merge_kernel(DecodeArgs a) {
  __shared__ float s_m[16][kHeads];
  __shared__ float s_den[16][kHeads];
  __shared__ floatx4_t s_acc[16][16];
  const int S = a.n_splits;
  const int64_t tok = blockIdx.y;
  const int h16 = threadIdx.x & 15, sl = threadIdx.x >> 4;  // slot (= head), split lane
  const int s0 = (S * sl) >> 4, s1 = (S * (sl + 1)) >> 4;
  const float* ml = a.part_ml + tok * S * 2 * kHeads;
  const int e4 = blockIdx.x * 16 + h16;  // fragment-order float4 index; its head is h16
  const float* po = a.part_o + tok * S * (kHeads * kLat) + (int64_t)e4 * 4;
  floatx4_t v[NPL];
  float mv[NPL], lv[NPL];
#pragma unroll
  for (int u = 0; u < NPL; ++u) {
    const int sp = min(s0 + u, S - 1);
    mv[u] = ml[sp * 2 * kHeads + h16];
    lv[u] = ml[sp * 2 * kHeads + kHeads + h16];
    v[u] = *reinterpret_cast<const floatx4_t*>(po + (int64_t)sp * (kHeads * kLat));
  }
#pragma unroll
  for (int u = 0; u < NPL; ++u)
    if (s0 + u >= s1) mv[u] = -INFINITY;  // not this lane's split
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < NPL; ++u) m = fmaxf(m, mv[u]);
  s_m[sl][h16] = m;
  __syncthreads();
  m = -INFINITY;
#pragma unroll
  for (int i = 0; i < 16; ++i) m = fmaxf(m, s_m[i][h16]);
  float den = 0.f;
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < NPL; ++u) {
    // a split with no visible key wrote no partial: its slice is not used
    if (mv[u] != -INFINITY) {
      const float f = __expf(mv[u] - m);
      den = fmaf(f, lv[u], den);
      acc += f * v[u];
    }
  }
  s_den[sl][h16] = den;
  s_acc[sl][h16] = acc;
  __syncthreads();
  if (sl == 0) {
    acc = s_acc[0][h16];
    den = s_den[0][h16];
#pragma unroll
    for (int i = 1; i < 16; ++i) {  // fixed order
      acc += s_acc[i][h16];
      den += s_den[i][h16];
    }
    const float inv = 1.f / den;  // split 0 holds key 0, so den >= 1
    const int ln = e4 & 63, wv = e4 >> 9, t = (e4 >> 6) & 7;
    uint16_t* o = a.out + tok * a.o_tok + h16 * a.o_head;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[frag_dim(wv, t, ln, i)] = f32_to_bf16(acc[i] * inv);
  }
}

}  // namespace dsk

using namespace dsk;

namespace {

#ifndef DSK_DECODE_WGS
#define DSK_DECODE_WGS 256
#endif

// Key splits per query token: enough workgroups to give every CU one
// (DSK_DECODE_WGS; the split kernel's LDS ring admits one workgroup per CU), at
// most kMaxSplits, at least one 64-key block each. Each split writes a 32 KB
// partial that the merge reads back, against 74 KB of cache per block, so a
// plan of one block per split takes two wherever that still leaves half the CUs
// busy: at L = 4096, b = 4 runs 13.6 us on 32 splits of two blocks against
// 15.1 us on 64 of one, while b = 1 keeps its 64 single-block splits (9.9 us
// against 11.2).
void split_plan(int batch, int q_len, int kv_len, int* n_splits, int* split_blocks) {
  const int blocks = (kv_len + kBlock - 1) / kBlock;
  const int64_t tokens = (int64_t)batch * q_len;
  int want = (int)std::min<int64_t>(blocks, std::max<int64_t>(1, (DSK_DECODE_WGS + tokens - 1) / tokens));
  want = std::min(want, kMaxSplits);
  int per = (blocks + want - 1) / want;
  if (per == 1 && blocks >= 2 && tokens * ((blocks + 1) / 2) >= DSK_DECODE_WGS / 2) per = 2;
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

namespace dsk {
// Whether two cache views of `wa` and `wb` columns per token row, with the same
// token and batch strides (elements), share an element: disjoint extents never
// do; inside one buffer the column offset of b relative to a's row start decides
// (token rows of the same width repeat every ld elements).
static bool rows_overlap(const dsk_bf16* a, int wa, const dsk_bf16* b, int wb, int64_t ld,
                         int64_t ld_batch, int batch, int kv_len) {
  const int64_t span = (int64_t)(batch - 1) * ld_batch + (int64_t)(kv_len - 1) * ld;
  const int64_t d = b - a;  // elements
  if (d >= span + wa || -d >= span + wb) return false;  // disjoint extents
  if (ld_batch % ld != 0) return true;                  // cannot reason per row: refuse
  const int64_t c = ((d % ld) + ld) % ld;               // b's column in a's row frame
  return c < wa || c + wb > ld;
}
}  // namespace dsk

extern "C" int dsk_mla_decode_attention(const dsk_bf16* q_abs, int64_t qa_tok, int64_t qa_head,
                                        const dsk_bf16* q_pe, int64_t qp_tok, int64_t qp_head,
                                        const dsk_bf16* latent, const dsk_bf16* k_pe,
                                        dsk_bf16* k_rope, int rope_len, int64_t ld_tok,
                                        int64_t ld_batch, const dsk_bf16* cos_tab,
                                        const dsk_bf16* sin_tab, float eps, float scale, int batch,
                                        int q_len, int kv_len, dsk_bf16* o_latent, int64_t o_tok,
                                        int64_t o_head, void* workspace, size_t bytes,
                                        void* stream) {
  DSK_REQUIRE(batch >= 0 && q_len >= 0, DSK_ERR_INVALID_ARG,
              "mla_decode_attention: batch and q_len must be >= 0");
  if (batch == 0 || q_len == 0) return DSK_OK;
  DSK_REQUIRE(kv_len >= q_len, DSK_ERR_INVALID_ARG,
              "mla_decode_attention: need q_len <= kv_len (the new tokens are in the cache)");
  DSK_REQUIRE(rope_len >= 0 && rope_len <= kv_len, DSK_ERR_INVALID_ARG,
              "mla_decode_attention: need 0 <= rope_len <= kv_len");
  DSK_REQUIRE(ld_tok >= kRope && ld_tok % 8 == 0 && ld_batch % 8 == 0 &&
                  (batch == 1 || ld_batch >= (int64_t)kv_len * ld_tok),
              DSK_ERR_INVALID_ARG,
              "mla_decode_attention: token stride must be a multiple of 8 (>= 64) and the batch "
              "stride a multiple of 8 covering kv_len tokens");
  DSK_REQUIRE((int64_t)kv_len * ld_tok * 2 < ((int64_t)1 << 31), DSK_ERR_INVALID_ARG,
              "mla_decode_attention: one sequence of the cache must span less than 2 GiB");
  DSK_REQUIRE(qa_tok % 8 == 0 && qa_head % 8 == 0 && qp_tok % 8 == 0 && qp_head % 8 == 0 &&
                  o_tok % 2 == 0 && o_head % 2 == 0,
              DSK_ERR_ALIGNMENT,
              "mla_decode_attention: query strides must be multiples of 8, output strides of 2");
  DSK_REQUIRE(qa_head * 16 < ((int64_t)1 << 30) && qp_head * 16 < ((int64_t)1 << 30),
              DSK_ERR_INVALID_ARG, "mla_decode_attention: query head strides too large");
  DSK_REQUIRE(q_abs && q_pe && latent && k_pe && k_rope && cos_tab && sin_tab && o_latent &&
                  workspace,
              DSK_ERR_NULL_PTR, "mla_decode_attention: NULL pointer");
  DSK_REQUIRE(aligned16(q_abs) && aligned16(q_pe) && aligned16(latent) && aligned16(k_pe) &&
                  aligned16(k_rope) && aligned16(cos_tab) && aligned16(sin_tab) &&
                  (reinterpret_cast<uintptr_t>(o_latent) & 3u) == 0,
              DSK_ERR_ALIGNMENT,
              "mla_decode_attention: inputs must be 16-byte aligned, the output 4-byte aligned");
  DSK_REQUIRE((int64_t)batch * q_len <= 65535, DSK_ERR_INVALID_ARG,
              "mla_decode_attention: batch * q_len must be <= 65535");
  // k_rope is written by the kernel: it must not overlap the latent or k_pe rows
  // it is read beside. Views sharing one buffer (the same strides) overlap where
  // their column ranges meet inside a token row.
  DSK_REQUIRE(!rows_overlap(k_rope, kRope, latent, kLat, ld_tok, ld_batch, batch, kv_len) &&
                  !rows_overlap(k_rope, kRope, k_pe, kRope, ld_tok, ld_batch, batch, kv_len),
              DSK_ERR_INVALID_ARG,
              "mla_decode_attention: k_rope overlaps latent or k_pe (it is written while they "
              "are read)");
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
  a.krope = reinterpret_cast<uint16_t*>(k_rope);
  a.ld_tok = ld_tok;
  a.ld_batch = ld_batch;
  a.cos_t = reinterpret_cast<const uint16_t*>(cos_tab);
  a.sin_t = reinterpret_cast<const uint16_t*>(sin_tab);
  a.eps = eps;
  a.scale = scale;
  a.L = kv_len;
  a.Q = q_len;
  a.rope_len = rope_len;
  a.n_splits = S;
  a.split_blocks = per;
  a.part_ml = reinterpret_cast<float*>(workspace);
  a.part_o = a.part_ml + (size_t)batch * q_len * S * 2 * kHeads;  // 128-byte multiple
  a.out = reinterpret_cast<uint16_t*>(o_latent);
  a.o_tok = o_tok;
  a.o_head = o_head;
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(attn_split_kernel, dim3(S, q_len, batch), dim3(kSplitThreads), 0, st, a);
  int rc = check_launch("attn_split_kernel");
  if (rc || S == 1) return rc;
  const dim3 mgrid(kHeads * kLat / 4 / 16, batch * q_len);
  const int npl = (S + 15) / 16;
  if (npl <= 1)
    hipLaunchKernelGGL(attn_merge_kernel<1>, mgrid, dim3(256), 0, st, a);
  else if (npl <= 2)
    hipLaunchKernelGGL(attn_merge_kernel<2>, mgrid, dim3(256), 0, st, a);
  else if (npl <= 4)
    hipLaunchKernelGGL(attn_merge_kernel<4>, mgrid, dim3(256), 0, st, a);
  else if (npl <= 8)
    hipLaunchKernelGGL(attn_merge_kernel<8>, mgrid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(attn_merge_kernel<16>, mgrid, dim3(256), 0, st, a);
  return check_launch("attn_merge_kernel");
}
