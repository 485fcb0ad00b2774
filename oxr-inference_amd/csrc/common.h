// Shared device helpers for the gfx950 verify-step kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, MFMA
// 16x16x32 bf16 tiles, 160 KB LDS per CU.  bf16 values travel as raw uint16_t
// bits so that the C-ABI never exposes a compiler-specific bf16 type.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/oxr_verify.h"

namespace oxr {

typedef uint16_t bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// bf16 <-> fp32.  fp32 -> bf16 is round-to-nearest-even with NaN mapped to the
// canonical quiet NaN 0x7FC0, the same convention torch's CPU BFloat16 uses.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Round an fp32 value to the nearest bf16 and return it widened back to fp32.
__device__ __forceinline__ float round_bf16(float f) { return bf2f(f2bf(f)); }

// Low / high bf16 of a packed pair.
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }

// Hardware round-to-nearest-even pack of two fp32 values (v_cvt_pk_bf16_f32).
// Same bits as pack_bf for every non-NaN input; a NaN keeps its own payload
// instead of becoming 0x7FC0, so use it only where NaN cannot occur or its
// bits do not matter.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf_hw(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// Upper 16 bits of two 32-bit words, packed lo | hi << 16 (one v_perm_b32):
// the bf16 value of an fp32 that holds an exact bf16.
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// ---------------------------------------------------------------------------
// Wave-level helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// Exchanges between the lane groups of a wave on the vector ALU (no LDS round trip).  gfx950's
// v_permlane16_swap / v_permlane32_swap give every lane {v[l], v[l ^ 16]} (resp. l ^ 32) as an
// unordered pair, so a commutative combination of the two is exactly `v op shfl_xor(v, 16 | 32)`.
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// v + v[lane ^ m] for m = 1, 2 (quad_perm), and for m = 4, 8 on values already equal within each
// quad (resp. 8 lanes), where the half-row / row mirror supplies the same partner value: so
// wave_sum gives the bits of the butterfly `for m = 1 .. 32: v += shfl_xor(v, m)`.
template <int kCtrl>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]: lane ^ 1
  v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]: lane ^ 2
  v = dpp_add<0x141>(v);  // row_half_mirror (quad-uniform values): lane ^ 4
  v = dpp_add<0x140>(v);  // row_mirror (8-lane-uniform values): lane ^ 8
  return xor32_sum(xor16_sum(v));
}

__device__ __forceinline__ f32x4 mfma_16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

// 128-bit global loads/stores.  `nt` variants mark data that is streamed once
// (weights, KV pages) so it does not evict reusable lines from L2.
__device__ __forceinline__ u32x4 ld128(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 ld128_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st128(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

// Element (row, k) of a [rows, K] bf16 matrix in the packed layout the GEMMs
// stream (weights, and token rows between kernels): 16-row tiles; per tile and
// 128-column step four contiguous 1 KiB blocks, block i holding, for lane
// 16g + r, row r's columns [32i + 8g, +8).  K is a multiple of 128.
__device__ __forceinline__ int64_t packed_offset(int64_t row, int64_t k, int64_t K) {
  return ((((row >> 4) * (K >> 7) + (k >> 7)) * 4 + ((k >> 5) & 3)) * 64 + ((k >> 3) & 3) * 16 + (row & 15)) * 8 +
         (k & 7);
}

}  // namespace oxr

// Host-side helpers shared by the entry points.
#define OXR_RETURN_IF(cond, code) \
  do {                            \
    if (cond) return (code);      \
  } while (0)

#define OXR_LAUNCH_STATUS() ((int)hipGetLastError())
