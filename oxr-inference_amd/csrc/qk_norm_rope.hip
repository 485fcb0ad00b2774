// Fused q/k RMSNorm + NeoX RoPE + paged KV-cache write (gfx950).
//
// Replaces the Triton kernel of oxr_runtime/kernels.py:114-147 and its CPU
// restatement kernels.py:181-213.  One head (128 bf16 = 256 B) is owned by 16
// lanes, each holding 8 consecutive elements loaded with one 128-bit load, so
// a 64-lane wave works on 4 heads and every load and store is a full 128-bit
// access.  The work is flattened over (token, head) so the grid scales with
// n * (H + 2*KV) instead of launching one program per token and part.
//
// Bit-exactness with the reference rounding chain (kernels.py:95-111):
//   h   = f32(x)
//   var = (S(h[0:64]) + S(h[64:128])) / 128, S = the fixed addition tree of
//         kernels.py:79-92 / 206-213: per 32-element chunk pairwise adds at
//         element strides 16, 8, 4, 2, 1, then chunk0 + chunk1
//   r   = 1 / sqrt(var + eps)            (both correctly rounded)
//   y   = f32(bf16(w * bf16(h * r)))     (w * bf16 is exact in fp32)
//   out = bf16(y1*c - y2*s | y1*s + y2*c) (products exact, one rounding)
// With 8 elements per lane the stride-16 and stride-8 adds are lane
// exchanges (xor 2, xor 1 inside a 4-lane chunk) and strides 4, 2, 1 are in
// lane; chunk and half sums are xor 4 and xor 8.  The file is built with
// -ffp-contract=off and correctly rounded fp32 sqrt/divide.
#include "common.h"

namespace oxr {
namespace {

constexpr int kHeadDim = 128;
constexpr int kLanesPerHead = 16;
constexpr int kThreads = 256;
constexpr int kHeadsPerBlock = kThreads / kLanesPerHead;

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

template <bool kNeedKV>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_store_kernel(
    const bf16_t* __restrict__ qkv, const bf16_t* __restrict__ q_weight, const bf16_t* __restrict__ k_weight,
    const bf16_t* __restrict__ cos_table, const bf16_t* __restrict__ sin_table, float eps,
    bf16_t* __restrict__ k_cache, bf16_t* __restrict__ v_cache, const int64_t* __restrict__ slots,
    int64_t num_slots, int64_t total_heads, int num_heads, int num_kv_heads, bf16_t* __restrict__ q_out,
    bf16_t* __restrict__ k_out, bf16_t* __restrict__ v_out, const int64_t* __restrict__ positions,
    int64_t table_rows) {
  const int heads_per_token = num_heads + 2 * num_kv_heads;
  int64_t g = (int64_t)blockIdx.x * kHeadsPerBlock + threadIdx.x / kLanesPerHead;
  const int s = threadIdx.x % kLanesPerHead;
  const bool active = g < total_heads;
  // Lanes past the end keep running on the last head so every lane takes part
  // in the exchanges below; they store nothing.
  if (!active) g = total_heads - 1;
  const int64_t t = g / heads_per_token;
  const int head = (int)(g - t * heads_per_token);

  u32x4 raw = ld128(qkv + g * kHeadDim + s * 8);
  float x[8];
  unpack8(raw, x);

  // Sum of squares in the reference's tree order.
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
  const float var = total / (float)kHeadDim;
  const float r = 1.0f / sqrtf(var + eps);

  const bool is_q = head < num_heads;
  const bool is_k = !is_q && head < num_heads + num_kv_heads;
  const bf16_t* weight = is_q ? q_weight : k_weight;
  float w[8], y[8];
  unpack8(ld128(weight + s * 8), w);
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf16(w[e] * round_bf16(x[e] * r));

  // NeoX rotation: element j of the first half pairs with j of the second,
  // which lives in lane s ^ 8 at the same register position.
  float c[8], sn[8], out[8];
  const int j0 = (s & 7) * 8;
  // cos/sin row: the token's own row, or the table row of its position
  // (rope_cos[positions], language.py:204) when positions are given.
  int64_t trow = t;
  if (positions) {
    trow = positions[t];
    trow = trow < 0 ? 0 : (trow >= table_rows ? table_rows - 1 : trow);
  }
  unpack8(ld128(cos_table + trow * (kHeadDim / 2) + j0), c);
  unpack8(ld128(sin_table + trow * (kHeadDim / 2) + j0), sn);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float other = shfl_xor_f(y[e], 8);
    out[e] = (s < 8) ? (y[e] * c[e] - other * sn[e]) : (other * sn[e] + y[e] * c[e]);
  }
  if (!active) return;

  const int64_t slot = slots[t];
  const bool slot_ok = slot >= 0 && slot < num_slots;
  if (is_q) {
    st128(q_out + (t * num_heads + head) * kHeadDim + s * 8, pack8(out));
  } else if (is_k) {
    const int kh = head - num_heads;
    const u32x4 packed = pack8(out);
    if (slot_ok) st128(k_cache + (slot * num_kv_heads + kh) * kHeadDim + s * 8, packed);
    if (kNeedKV) st128(k_out + (t * num_kv_heads + kh) * kHeadDim + s * 8, packed);
  } else {
    const int vh = head - num_heads - num_kv_heads;
    if (slot_ok) st128(v_cache + (slot * num_kv_heads + vh) * kHeadDim + s * 8, raw);
    if (kNeedKV) st128(v_out + (t * num_kv_heads + vh) * kHeadDim + s * 8, raw);
  }
}

}  // namespace
}  // namespace oxr

namespace oxr {
namespace {
int launch_qk(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight, const oxr_bf16* cos,
              const oxr_bf16* sin, float eps, oxr_bf16* k_cache, oxr_bf16* v_cache, const int64_t* slots,
              int64_t num_slots, int64_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
              oxr_bf16* q_out, oxr_bf16* k_out, oxr_bf16* v_out, const int64_t* positions, int64_t table_rows,
              oxr_stream_t stream) {
  OXR_RETURN_IF(n < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_slots < 0, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(head_dim != kHeadDim, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF((k_out == nullptr) != (v_out == nullptr), OXR_ERR_INVALID_ARG);
  if (n == 0) return OXR_OK;
  OXR_RETURN_IF(!qkv || !q_weight || !k_weight || !cos || !sin || !k_cache || !v_cache || !slots || !q_out,
                OXR_ERR_INVALID_ARG);
  const int64_t total = n * (int64_t)(num_heads + 2 * num_kv_heads);
  const int64_t blocks = (total + kHeadsPerBlock - 1) / kHeadsPerBlock;
  OXR_RETURN_IF(blocks > 0x7fffffff, OXR_ERR_UNSUPPORTED);
  hipStream_t s = (hipStream_t)stream;
  if (k_out) {
    hipLaunchKernelGGL(qk_norm_rope_store_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, s, qkv, q_weight,
                       k_weight, cos, sin, eps, k_cache, v_cache, slots, num_slots, total, num_heads, num_kv_heads,
                       q_out, k_out, v_out, positions, table_rows);
  } else {
    hipLaunchKernelGGL(qk_norm_rope_store_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, s, qkv,
                       q_weight, k_weight, cos, sin, eps, k_cache, v_cache, slots, num_slots, total, num_heads,
                       num_kv_heads, q_out, nullptr, nullptr, positions, table_rows);
  }
  return OXR_LAUNCH_STATUS();
}
}  // namespace
}  // namespace oxr

extern "C" int oxr_qk_norm_rope_store(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight,
                                      const oxr_bf16* cos, const oxr_bf16* sin, float eps, oxr_bf16* k_cache,
                                      oxr_bf16* v_cache, const int64_t* slots, int64_t num_slots, int64_t n,
                                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, oxr_bf16* q_out,
                                      oxr_bf16* k_out, oxr_bf16* v_out, oxr_stream_t stream) {
  return oxr::launch_qk(qkv, q_weight, k_weight, cos, sin, eps, k_cache, v_cache, slots, num_slots, n, num_heads,
                        num_kv_heads, head_dim, q_out, k_out, v_out, nullptr, 0, stream);
}

extern "C" int oxr_qk_norm_rope_store_at(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight,
                                         const oxr_bf16* cos_table, const oxr_bf16* sin_table, int64_t table_rows,
                                         const int64_t* positions, float eps, oxr_bf16* k_cache, oxr_bf16* v_cache,
                                         const int64_t* slots, int64_t num_slots, int64_t n, int32_t num_heads,
                                         int32_t num_kv_heads, int32_t head_dim, oxr_bf16* q_out, oxr_bf16* k_out,
                                         oxr_bf16* v_out, oxr_stream_t stream) {
  if (n > 0 && (!positions || table_rows <= 0)) return OXR_ERR_INVALID_ARG;
  return oxr::launch_qk(qkv, q_weight, k_weight, cos_table, sin_table, eps, k_cache, v_cache, slots, num_slots, n,
                        num_heads, num_kv_heads, head_dim, q_out, k_out, v_out, positions, table_rows, stream);
}
