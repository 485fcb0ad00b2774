// Row RMSNorm and the embedding gather that feeds the first one (gfx950).
//
// Replaces _rms_norm (oxr_runtime/language.py:69-72) as used by the decoder
// layers' input/post-attention norms and the final norm (language.py:211,
// 253-257, 267-268), and the embedding lookup of the verify step
// (decode_graph.py:164, embed_tokens(ids)):
//   h   = f32(x)
//   var = sum(h^2) / D            (fp32; per thread 8 values, then a butterfly
//                                   across the wave and a sum over the waves)
//   out = bf16(w * bf16(h * (1 / sqrt(var + eps))))
// Three sources for the row: a plain row (kRows); the embedding table row of
// a token id, also stored as the new residual stream (kEmbed); or the residual
// add of _add_rms_norm with the preceding GEMM's fp32 k-split partials summed
// here (kAddPartials), so the GEMM needs no cross-workgroup reduction.
#include "common.h"

namespace oxr {
namespace {

constexpr int kMaxThreads = 512;  // one 8-element vector per thread: D <= 4096

enum Source { kRows = 0, kEmbed = 1, kAddPartials = 2 };

// One workgroup per row, one 16-byte vector (8 elements) per thread, so a row
// is read in one round of loads by D/8 threads across the CUs, and the norm
// weights are fetched at the same time.  MODE kRows: x is [rows, ldx].
// kEmbed: row = table[ids[row]], also stored as the residual.  kAddPartials:
// row = bf16(bf16(sum of the k-split fp32 partials of the GEMM that produced
// it) + residual), stored as the residual (read from x when given, else from
// `residual` itself; the add of _add_rms_norm,
// language.py:94-99, with the GEMM's bf16 output rounding first, as the
// reference's nn.Linear does).
template <int MODE, int SPLITS>
__global__ __launch_bounds__(kMaxThreads) void rms_norm_kernel(const bf16_t* __restrict__ x, int64_t ldx,
                                                               const int64_t* __restrict__ ids, int64_t vocab,
                                                               const float* __restrict__ partials, int k_splits,
                                                               int rows, int D, const bf16_t* __restrict__ w, float eps,
                                                               bf16_t* __restrict__ residual, bf16_t* __restrict__ out,
                                                               int64_t ldo, int out_packed) {
  __shared__ float wave_ss[kMaxThreads / kWave];
  const int row = blockIdx.x;
  const int col = threadIdx.x * 8;
  const u32x4 wt = ld128(w + col);
  const bf16_t* src;
  if constexpr (MODE == kEmbed) {
    int64_t id = ids[row];
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // stay inside the table
    src = x + id * ldx;
  } else if constexpr (MODE == kAddPartials) {
    src = (x ? x : residual) + (int64_t)row * ldo;  // x: the residual to read, when not `residual` itself
  } else {
    src = x + (int64_t)row * ldx;
  }
  u32x4 v = ld128(src + col);
  if constexpr (MODE == kAddPartials) {
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
    const int n = SPLITS > 0 ? SPLITS : k_splits;
#pragma unroll
    for (int sp = 0; sp < n; ++sp) {
      const float* p = partials + ((int64_t)sp * rows + row) * D + col;
      lo += *reinterpret_cast<const f32x4*>(p);
      hi += *reinterpret_cast<const f32x4*>(p + 4);
    }
    const uint32_t rd[4] = {v.x, v.y, v.z, v.w};
    const float sum[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf(round_bf16(sum[2 * e]) + lo_bf(rd[e]), round_bf16(sum[2 * e + 1]) + hi_bf(rd[e]));
    v = u32x4{o[0], o[1], o[2], o[3]};
  }
  const uint32_t xd[4] = {v.x, v.y, v.z, v.w};
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = lo_bf(xd[e]), b = hi_bf(xd[e]);
    ss += a * a;
    ss += b * b;
  }
  ss = wave_sum(ss);  // the butterfly over lane ^ 1 .. 32, on the vector ALU
  if (threadIdx.x % kWave == 0) wave_ss[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = 0.f;
  for (int i = 0; i < (int)(blockDim.x / kWave); ++i) ss += wave_ss[i];
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  const uint32_t wd[4] = {wt.x, wt.y, wt.z, wt.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float y0 = lo_bf(wd[e]) * round_bf16(lo_bf(xd[e]) * r);
    const float y1 = hi_bf(wd[e]) * round_bf16(hi_bf(xd[e]) * r);
    o[e] = pack_bf(y0, y1);
  }
  st128(out + (out_packed ? packed_offset(row, col, D) : (int64_t)row * ldo + col), u32x4{o[0], o[1], o[2], o[3]});
  if constexpr (MODE != kRows) st128(residual + (int64_t)row * ldo + col, v);
}

template <int MODE>
int launch(const bf16_t* x, int64_t ldx, const int64_t* ids, int64_t vocab, const float* partials, int k_splits,
           int rows, int D, const bf16_t* w, float eps, bf16_t* residual, bf16_t* out, int64_t ldo, int out_packed,
           hipStream_t s) {
  const dim3 grid(rows), block(D / 8);
  if (MODE == kAddPartials && k_splits == 2)
    hipLaunchKernelGGL((rms_norm_kernel<MODE, 2>), grid, block, 0, s, x, ldx, ids, vocab, partials, k_splits, rows, D,
                       w, eps, residual, out, ldo, out_packed);
  else if (MODE == kAddPartials && k_splits == 4)
    hipLaunchKernelGGL((rms_norm_kernel<MODE, 4>), grid, block, 0, s, x, ldx, ids, vocab, partials, k_splits, rows, D,
                       w, eps, residual, out, ldo, out_packed);
  else if (MODE == kAddPartials && k_splits == 8)
    hipLaunchKernelGGL((rms_norm_kernel<MODE, 8>), grid, block, 0, s, x, ldx, ids, vocab, partials, k_splits, rows, D,
                       w, eps, residual, out, ldo, out_packed);
  else
    hipLaunchKernelGGL((rms_norm_kernel<MODE, 0>), grid, block, 0, s, x, ldx, ids, vocab, partials, k_splits, rows, D,
                       w, eps, residual, out, ldo, out_packed);
  return OXR_LAUNCH_STATUS();
}

// The embedding lookup alone (nn.Embedding, language.py:155, as the eager paths call it:
// engine.py:595, 717): out[row] = table[ids[row]], one 16-byte vector per thread.
__global__ __launch_bounds__(kMaxThreads) void embed_gather_kernel(const int64_t* __restrict__ ids, int64_t vocab,
                                                                   const bf16_t* __restrict__ table, int D,
                                                                   bf16_t* __restrict__ out, int64_t ldo) {
  int64_t id = ids[blockIdx.x];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // stay inside the table
  const int col = threadIdx.x * 8;
  st128(out + (int64_t)blockIdx.x * ldo + col, ld128(table + id * D + col));
}

int check(int64_t rows, int64_t D, int64_t ld, int64_t ldo) {
  OXR_RETURN_IF(rows < 0 || D <= 0 || ld < D || ldo < D, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(D % (kWave * 8) != 0 || D > kMaxThreads * 8 || ld % 8 != 0 || ldo % 8 != 0, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(rows > 0x7fffffff, OXR_ERR_UNSUPPORTED);
  return OXR_OK;
}

}  // namespace
}  // namespace oxr

extern "C" int oxr_rms_norm(const oxr_bf16* x, int64_t ldx, int64_t rows, int64_t hidden, const oxr_bf16* weight,
                            float eps, oxr_bf16* out, int64_t ldo, int32_t out_packed, oxr_stream_t stream) {
  using namespace oxr;
  int st = check(rows, hidden, ldx, out_packed ? hidden : ldo);
  if (st) return st;
  if (rows == 0) return OXR_OK;
  OXR_RETURN_IF(!x || !weight || !out, OXR_ERR_INVALID_ARG);
  return launch<kRows>(x, ldx, nullptr, 0, nullptr, 0, (int)rows, (int)hidden, weight, eps, nullptr, out, ldo,
                       out_packed ? 1 : 0, (hipStream_t)stream);
}

extern "C" int oxr_embed_rms_norm(const int64_t* ids, int64_t rows, const oxr_bf16* table, int64_t vocab,
                                  int64_t hidden, const oxr_bf16* weight, float eps, oxr_bf16* residual,
                                  oxr_bf16* out, int32_t out_packed, oxr_stream_t stream) {
  using namespace oxr;
  int st = check(rows, hidden, hidden, hidden);
  if (st) return st;
  if (rows == 0) return OXR_OK;
  OXR_RETURN_IF(!ids || !table || vocab <= 0 || !weight || !residual || !out, OXR_ERR_INVALID_ARG);
  return launch<kEmbed>(table, hidden, ids, vocab, nullptr, 0, (int)rows, (int)hidden, weight, eps, residual, out,
                        hidden, out_packed ? 1 : 0, (hipStream_t)stream);
}

extern "C" int oxr_add_partials_rms_norm(const float* partials, int32_t k_splits, int64_t rows, int64_t hidden,
                                         oxr_bf16* residual, const oxr_bf16* weight, float eps, oxr_bf16* out,
                                         int32_t out_packed, oxr_stream_t stream) {
  using namespace oxr;
  int st = check(rows, hidden, hidden, hidden);
  if (st) return st;
  OXR_RETURN_IF(k_splits < 1, OXR_ERR_INVALID_ARG);
  if (rows == 0) return OXR_OK;
  OXR_RETURN_IF(!partials || !residual || !weight || !out, OXR_ERR_INVALID_ARG);
  return launch<kAddPartials>(nullptr, hidden, nullptr, 0, partials, k_splits, (int)rows, (int)hidden, weight, eps,
                              residual, out, hidden, out_packed ? 1 : 0, (hipStream_t)stream);
}

extern "C" int oxr_add_partials_rms_norm_from(const float* partials, int32_t k_splits, int64_t rows, int64_t hidden,
                                              const oxr_bf16* residual_in, oxr_bf16* residual, const oxr_bf16* weight,
                                              float eps, oxr_bf16* out, int32_t out_packed, oxr_stream_t stream) {
  using namespace oxr;
  int st = check(rows, hidden, hidden, hidden);
  if (st) return st;
  OXR_RETURN_IF(k_splits < 1, OXR_ERR_INVALID_ARG);
  if (rows == 0) return OXR_OK;
  OXR_RETURN_IF(!partials || !residual_in || !residual || !weight || !out, OXR_ERR_INVALID_ARG);
  return launch<kAddPartials>(residual_in, hidden, nullptr, 0, partials, k_splits, (int)rows, (int)hidden, weight,
                              eps, residual, out, hidden, out_packed ? 1 : 0, (hipStream_t)stream);
}

extern "C" int oxr_embed_gather(const int64_t* ids, int64_t rows, const oxr_bf16* table, int64_t vocab, int64_t hidden,
                                oxr_bf16* out, int64_t ldo, oxr_stream_t stream) {
  using namespace oxr;
  int st = check(rows, hidden, hidden, ldo);
  if (st) return st;
  if (rows == 0) return OXR_OK;
  OXR_RETURN_IF(!ids || !table || vocab <= 0 || !out, OXR_ERR_INVALID_ARG);
  hipLaunchKernelGGL(embed_gather_kernel, dim3((unsigned)rows), dim3((unsigned)(hidden / 8)), 0, (hipStream_t)stream,
                     ids, vocab, table, (int)hidden, out, ldo);
  return OXR_LAUNCH_STATUS();
}
