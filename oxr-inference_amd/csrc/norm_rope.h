// Per-head q/k RMSNorm + NeoX RoPE on 16 lanes (gfx950), shared by the
// standalone kernel (qk_norm_rope.hip) and the attention kernel that fuses it
// (paged_attention.hip).
//
// One head (128 bf16 = 256 B) is owned by 16 consecutive lanes (s = lane % 16),
// each holding 8 consecutive elements.  Bit-exact with the reference rounding
// chain (oxr_runtime/kernels.py:47-63):
//   h   = f32(x)
//   var = (S(h[0:64]) + S(h[64:128])) / 128, S = the fixed addition tree of
//         kernels.py:31-44 / 158-165: per 32-element chunk pairwise adds at
//         element strides 16, 8, 4, 2, 1, then chunk0 + chunk1
//   r   = 1 / sqrt(var + eps)            (both correctly rounded)
//   y   = f32(bf16(w * bf16(h * r)))     (w * bf16 is exact in fp32)
//   out = bf16(y1*c - y2*s | y1*s + y2*c) (products exact, one rounding)
// With 8 elements per lane the stride-16 and stride-8 adds are lane exchanges
// (xor 2, xor 1 inside a 4-lane chunk) and strides 4, 2, 1 are in lane; chunk
// and half sums are xor 4 and xor 8.  Every lane of the wave must execute the
// exchanges.  Files including this are built with -ffp-contract=off and
// correctly rounded fp32 sqrt/divide.
#pragma once

#include "common.h"

namespace oxr {

constexpr int kNormRopeDim = 128;

__device__ __forceinline__ void unpack8(const u32x4& w, float (&v)[8]) {
  v[0] = lo_bf(w.x); v[1] = hi_bf(w.x);
  v[2] = lo_bf(w.y); v[3] = hi_bf(w.y);
  v[4] = lo_bf(w.z); v[5] = hi_bf(w.z);
  v[6] = lo_bf(w.w); v[7] = hi_bf(w.w);
}

__device__ __forceinline__ u32x4 pack8(const float (&v)[8]) {
  u32x4 w;
  w.x = pack_bf(v[0], v[1]);
  w.y = pack_bf(v[2], v[3]);
  w.z = pack_bf(v[4], v[5]);
  w.w = pack_bf(v[6], v[7]);
  return w;
}

// raw: this lane's 8 elements of the head row; w8: its 8 norm weights
// (weight[8s .. 8s+7]); c8 / s8: cos / sin[8 (s % 8) .. +7] of the RoPE table
// row of the token's position.  Returns the lane's 8 outputs, packed bf16.
__device__ __forceinline__ u32x4 norm_rope_16v(const u32x4& raw, const u32x4& w8, const u32x4& c8, const u32x4& s8,
                                               float eps, int s) {
  float x[8];
  unpack8(raw, x);
  float q2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) q2[e] = x[e] * x[e];
#pragma unroll
  for (int e = 0; e < 8; ++e) q2[e] = q2[e] + shfl_xor_f(q2[e], 2);  // element stride 16
#pragma unroll
  for (int e = 0; e < 8; ++e) q2[e] = q2[e] + shfl_xor_f(q2[e], 1);  // element stride 8
  const float a0 = q2[0] + q2[4], a1 = q2[1] + q2[5], a2 = q2[2] + q2[6], a3 = q2[3] + q2[7];  // stride 4
  const float b0 = a0 + a2, b1 = a1 + a3;                                                     // stride 2
  const float chunk = b0 + b1;                                                                // stride 1
  const float half = chunk + shfl_xor_f(chunk, 4);  // chunk0 + chunk1 of each 64-element half
  const float total = half + shfl_xor_f(half, 8);   // half0 + half1
  const float var = total / (float)kNormRopeDim;
  const float r = 1.0f / sqrtf(var + eps);

  float w[8], y[8];
  unpack8(w8, w);
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf16(w[e] * round_bf16(x[e] * r));

  // NeoX rotation: element j of the first half pairs with j of the second,
  // which lives in lane s ^ 8 at the same register position.
  float c[8], sn[8], out[8];
  unpack8(c8, c);
  unpack8(s8, sn);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float other = shfl_xor_f(y[e], 8);
    out[e] = (s < 8) ? (y[e] * c[e] - other * sn[e]) : (other * sn[e] + y[e] * c[e]);
  }
  return pack8(out);
}

// The same with the weights and the table row read here (weight: [128];
// cos_row / sin_row: [64]).
__device__ __forceinline__ u32x4 norm_rope_16(const u32x4& raw, const bf16_t* __restrict__ weight,
                                              const bf16_t* __restrict__ cos_row,
                                              const bf16_t* __restrict__ sin_row, float eps, int s) {
  const int j0 = (s & 7) * 8;
  return norm_rope_16v(raw, ld128(weight + s * 8), ld128(cos_row + j0), ld128(sin_row + j0), eps, s);
}

}  // namespace oxr
