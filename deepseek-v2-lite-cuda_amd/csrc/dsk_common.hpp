// Shared device/host helpers for libdsk (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "../../include/dsk.h"

namespace dsk {

constexpr int kWave = 64;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------ errors --
// Thread-local error string behind dsk_last_error().
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

#define DSK_REQUIRE(cond, code, msg)                  \
  do {                                                \
    if (!(cond)) return ::dsk::fail((code), (msg));   \
  } while (0)

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// -------------------------------------------------------------- bf16 <-> f32 --
__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
// Round-to-nearest-even; the compiler lowers this to v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) |
         (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ------------------------------------------------------------------ RoPE --
// RoPE of one raw pair (x0, x1) = (x[2k], x[2k+1]) (mla.py:196-205): the
// reference maps it to outputs k and k + d/2,
//   lo = out[k] = x0 cos[k] - x1 sin[k], hi = out[k + d/2] = x1 cos[k + d/2] + x0 sin[k + d/2].
// Every kernel that rotates keys uses this one expression, so rotated keys
// written by different kernels are bitwise equal.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c_lo, float c_hi, float s_lo,
                                          float s_hi, float& lo, float& hi) {
  lo = x0 * c_lo - x1 * s_lo;
  hi = x1 * c_hi + x0 * s_hi;
}

// ------------------------------------------------- memory-counter helpers --
// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the release/acquire fences of __syncthreads():
// those would wait for every in-flight DMA (vmcnt(0)) and drain the ring. The
// DMA completion this barrier publishes is waited for explicitly (wait_vmcnt)
// by every wave before it arrives; the "memory" clobber keeps the compiler
// from moving LDS accesses across the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Global->LDS DMA of 16 bytes per lane (1 KB per wave to lds_addr) from
// base + voff, as inline asm. The compiler's wait-count bookkeeping does not
// model this LDS-writing load alongside ordinary register loads (with both in
// flight it falls back to waiting for every outstanding load before each use);
// hidden from it, the register loads keep exact counts, which can only be
// stricter than needed since this DMA is not counted. The "memory" clobber
// keeps every other memory access in program order around it; completion is
// waited for explicitly (wait_vmcnt) before the data is read.
__device__ __forceinline__ void dma_1kb(const char* base, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(base), "s"(lds_addr) : "memory", "m0");
}

// ----------------------------------------------------------- wave reductions --
// DPP-based full-wave reductions (quad_perm / row mirrors inside a 16-lane row,
// then row_bcast15 / row_bcast31 across rows); the result is read from lane 63
// and returned wave-uniform.
template <int kCtrl, int kRowMask = 0xf, int kBankMask = 0xf>
__device__ __forceinline__ float dpp_f32(float old, float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      __float_as_int(old), __float_as_int(v), kCtrl, kRowMask, kBankMask, false));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v, v));         // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v, v));         // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v, v));        // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v, v));        // row_mirror
  v = fmaxf(v, dpp_f32<0x142, 0xa>(v, v));   // row_bcast:15
  v = fmaxf(v, dpp_f32<0x143, 0xc>(v, v));   // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(0.f, v);
  v += dpp_f32<0x4E>(0.f, v);
  v += dpp_f32<0x141>(0.f, v);
  v += dpp_f32<0x140>(0.f, v);
  v += dpp_f32<0x142, 0xa>(0.f, v);
  v += dpp_f32<0x143, 0xc>(0.f, v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Reductions over each 16-lane row (quad swaps, then the half-row and row
// mirrors): every lane of the row ends with the row's result. Each step pairs
// lane i with a partner p(i) that pairs back with i, so both compute the same
// op(v_i, v_p) and the sums are bitwise equal on all 16 lanes.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v, v));
  v = fmaxf(v, dpp_f32<0x4E>(v, v));
  v = fmaxf(v, dpp_f32<0x141>(v, v));
  v = fmaxf(v, dpp_f32<0x140>(v, v));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<0xB1>(0.f, v);
  v += dpp_f32<0x4E>(0.f, v);
  v += dpp_f32<0x141>(0.f, v);
  v += dpp_f32<0x140>(0.f, v);
  return v;
}
template <int kCtrl>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(v, v, kCtrl, 0xf, 0xf, false);
}
__device__ __forceinline__ int row16_min(int v) {
  v = min(v, dpp_i32<0xB1>(v));
  v = min(v, dpp_i32<0x4E>(v));
  v = min(v, dpp_i32<0x141>(v));
  v = min(v, dpp_i32<0x140>(v));
  return v;
}

// Inclusive prefix sum of an int over the 64 lanes (Hillis-Steele on shuffles;
// only used by the small scan kernels).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

__device__ __forceinline__ int readlane_i(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

}  // namespace dsk
