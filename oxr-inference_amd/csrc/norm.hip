// Row RMSNorm and the embedding gather that feeds the first one (gfx950).
//
// Replaces _rms_norm (oxr_runtime/language.py:69-72) as used by the decoder
// layers' input/post-attention norms and the final norm (language.py:211,
// 253-257, 267-268), and the embedding lookup of the verify step
// (decode_graph.py:164, embed_tokens(ids)):
//   h   = f32(x)
//   var = sum(h^2) / D            (fp32; one wave per row, lane-local sums of
//                                   D/64 values then a butterfly across lanes)
//   out = bf16(w * bf16(h * (1 / sqrt(var + eps))))
// The residual add that precedes the norm in _add_rms_norm is fused into the
// GEMM that produces its input (csrc/gemm.hip), so this kernel only
// normalises.  With kEmbed the row is gathered from the embedding table by
// token id and also stored as the new residual stream.
#include "common.h"

namespace oxr {
namespace {

constexpr int kMaxVec = 8;  // up to 8 x 16 B per lane: D <= 4096

template <bool kEmbed, int VEC>
__global__ __launch_bounds__(256) void rms_norm_kernel(const bf16_t* __restrict__ x, int64_t ldx,
                                                       const int64_t* __restrict__ ids, int64_t vocab, int rows,
                                                       int D, const bf16_t* __restrict__ w, float eps,
                                                       bf16_t* __restrict__ residual, bf16_t* __restrict__ out,
                                                       int64_t ldo) {
  const int row = blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const bf16_t* src;
  if constexpr (kEmbed) {
    int64_t id = ids[row];
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // stay inside the table
    src = x + id * ldx;
  } else {
    src = x + (int64_t)row * ldx;
  }
  u32x4 v[VEC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    v[i] = ld128(src + (i * kWave + lane) * 8);
    const uint32_t wd[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = lo_bf(wd[e]), b = hi_bf(wd[e]);
      ss += a * a;
      ss += b * b;
    }
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) ss += shfl_xor_f(ss, m);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const int col = (i * kWave + lane) * 8;
    const u32x4 wt = ld128(w + col);
    const uint32_t xd[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    const uint32_t wd[4] = {wt.x, wt.y, wt.z, wt.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float y0 = lo_bf(wd[e]) * round_bf16(lo_bf(xd[e]) * r);
      const float y1 = hi_bf(wd[e]) * round_bf16(hi_bf(xd[e]) * r);
      o[e] = pack_bf(y0, y1);
    }
    st128(out + (int64_t)row * ldo + col, u32x4{o[0], o[1], o[2], o[3]});
    if constexpr (kEmbed) st128(residual + (int64_t)row * ldo + col, v[i]);
  }
}

template <bool kEmbed>
int launch(const bf16_t* x, int64_t ldx, const int64_t* ids, int64_t vocab, int rows, int D, const bf16_t* w,
           float eps, bf16_t* residual, bf16_t* out, int64_t ldo, hipStream_t s) {
  const dim3 grid((rows + 3) / 4), block(256);
  switch (D / (kWave * 8)) {
#define OXR_CASE(n)                                                                                                \
  case n:                                                                                                          \
    hipLaunchKernelGGL((rms_norm_kernel<kEmbed, n>), grid, block, 0, s, x, ldx, ids, vocab, rows, D, w, eps, residual, \
                       out, ldo);                                                                                  \
    break;
    OXR_CASE(1) OXR_CASE(2) OXR_CASE(3) OXR_CASE(4) OXR_CASE(5) OXR_CASE(6) OXR_CASE(7) OXR_CASE(8)
#undef OXR_CASE
    default:
      return OXR_ERR_UNSUPPORTED;
  }
  return OXR_LAUNCH_STATUS();
}

int check(int64_t rows, int64_t D, int64_t ld, int64_t ldo) {
  OXR_RETURN_IF(rows < 0 || D <= 0 || ld < D || ldo < D, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(D % (kWave * 8) != 0 || D > kWave * 8 * kMaxVec || ld % 8 != 0 || ldo % 8 != 0, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(rows > 0x7fffffff - 3, OXR_ERR_UNSUPPORTED);
  return OXR_OK;
}

}  // namespace
}  // namespace oxr

extern "C" int oxr_rms_norm(const oxr_bf16* x, int64_t ldx, int64_t rows, int64_t hidden, const oxr_bf16* weight,
                            float eps, oxr_bf16* out, int64_t ldo, oxr_stream_t stream) {
  using namespace oxr;
  int st = check(rows, hidden, ldx, ldo);
  if (st) return st;
  if (rows == 0) return OXR_OK;
  OXR_RETURN_IF(!x || !weight || !out, OXR_ERR_INVALID_ARG);
  return launch<false>(x, ldx, nullptr, 0, (int)rows, (int)hidden, weight, eps, nullptr, out, ldo,
                       (hipStream_t)stream);
}

extern "C" int oxr_embed_rms_norm(const int64_t* ids, int64_t rows, const oxr_bf16* table, int64_t vocab,
                                  int64_t hidden, const oxr_bf16* weight, float eps, oxr_bf16* residual,
                                  oxr_bf16* out, oxr_stream_t stream) {
  using namespace oxr;
  int st = check(rows, hidden, hidden, hidden);
  if (st) return st;
  if (rows == 0) return OXR_OK;
  OXR_RETURN_IF(!ids || !table || vocab <= 0 || !weight || !residual || !out, OXR_ERR_INVALID_ARG);
  return launch<true>(table, hidden, ids, vocab, (int)rows, (int)hidden, weight, eps, residual, out, hidden,
                      (hipStream_t)stream);
}
