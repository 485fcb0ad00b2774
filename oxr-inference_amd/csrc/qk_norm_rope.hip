// Fused q/k RMSNorm + NeoX RoPE + paged KV-cache write (gfx950).
//
// Replaces the Triton kernel of oxr_runtime/kernels.py:66-99 and its CPU
// restatement kernels.py:133-165.  One head (128 bf16 = 256 B) is owned by 16
// lanes, each holding 8 consecutive elements loaded with one 128-bit load, so
// a 64-lane wave works on 4 heads and every load and store is a full 128-bit
// access.  The work is flattened over (token, head) so the grid scales with
// n * (H + 2*KV) instead of launching one program per token and part.
//
// The per-head arithmetic and its bit-exact rounding chain are in norm_rope.h.
#include "norm_rope.h"

namespace oxr {
namespace {

constexpr int kHeadDim = kNormRopeDim;
constexpr int kLanesPerHead = 16;
constexpr int kThreads = 256;
constexpr int kHeadsPerBlock = kThreads / kLanesPerHead;

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

  const u32x4 raw = ld128(qkv + g * kHeadDim + s * 8);
  const bool is_q = head < num_heads;
  const bool is_k = !is_q && head < num_heads + num_kv_heads;
  // cos/sin row: the token's own row, or the table row of its position
  // (rope_cos[positions], language.py:204) when positions are given.
  int64_t trow = t;
  if (positions) {
    trow = positions[t];
    trow = trow < 0 ? 0 : (trow >= table_rows ? table_rows - 1 : trow);
  }
  const u32x4 packed = norm_rope_16(raw, is_q ? q_weight : k_weight, cos_table + trow * (kHeadDim / 2),
                                    sin_table + trow * (kHeadDim / 2), eps, s);
  if (!active) return;

  const int64_t slot = slots[t];
  const bool slot_ok = slot >= 0 && slot < num_slots;
  if (is_q) {
    st128(q_out + (t * num_heads + head) * kHeadDim + s * 8, packed);
  } else if (is_k) {
    const int kh = head - num_heads;
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
