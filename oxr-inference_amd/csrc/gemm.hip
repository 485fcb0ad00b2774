// Weight-streaming bf16 GEMMs for the verify step (gfx950): Y = X * W^T.
//
// The verify step multiplies a handful of token rows (M = B * S = 32 at B=8,
// S=4) by large weights: every projection and the LM head is HBM-bound on the
// weight read.  So the kernel is organised around streaming W exactly once:
//
// * A workgroup owns one tile of 16 * NA weight rows (output columns) and all
//   M <= 16 * NB token rows.  Its kSplit waves split K; each wave streams its
//   slice of the tile's rows with 64-byte-per-lane loads that are directly the
//   A-operand fragments of v_mfma_f32_16x16x32_bf16 (lane (r, g) holds
//   W[row r][k + 32g .. 32g + 31], i.e. four MFMA k-steps), prefetching the
//   next 128 k while the current ones are multiplied.  X fragments use the
//   same k-slot mapping and come from L2 (X is at most 64 rows).
// * The waves' fp32 partial tiles are summed in LDS in a fixed order, then the
//   epilogue runs on the finished tile:
//     kStore   Y = bf16(acc)
//     kSiluMul rows [0, N) are gate and [N, 2N) up (the fused gate_up weight,
//              language.py:238): Y = bf16(bf16(silu(bf16(g))) * bf16(u))
//              (the reference's bf16 rounding points, language.py:102-104)
//     kArgmax  per token the largest bf16-rounded logit of the tile, lowest
//              column on ties, as a 64-bit key for a later cross-tile max;
//              optionally also stores the bf16 logits.
//     kAddResidual  R = bf16(bf16(acc) + R): the residual add of
//              _add_rms_norm (language.py:94-99), in place on R.
// C layout: lane (l % 16, g) holds rows 4g..4g+3 of the tile for token l % 16.
#include "common.h"

namespace oxr {
namespace {

enum Epilogue { kStore = 0, kSiluMul = 1, kArgmax = 2, kAddResidual = 3 };

constexpr int kKStep = 128;  // k per prefetch stage: 4 MFMA k-steps of 32

// Order-preserving key of a bf16 logit (as fp32 bits) and its column: larger
// value wins, then lower column.  NaN sorts above everything (torch argmax
// returns the first NaN); -0 and +0 compare equal.
__device__ __forceinline__ uint64_t argmax_key(uint32_t fbits, uint32_t col) {
  uint32_t key;
  if ((fbits & 0x7fffffffu) > 0x7f800000u) key = 0xffffffffu;
  else {
    if ((fbits & 0x7fffffffu) == 0u) fbits = 0u;
    key = (fbits & 0x80000000u) ? ~fbits : (fbits | 0x80000000u);
  }
  return ((uint64_t)key << 32) | (uint32_t)(~col);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const uint32_t lo = __shfl_xor((uint32_t)v, mask, kWave);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), mask, kWave);
  return ((uint64_t)hi << 32) | lo;
}

struct GemmArgs {
  const bf16_t* x;  // [M, ldx]
  int64_t ldx;
  int M;
  const bf16_t* w;  // [rows, K]
  int64_t K;
  int64_t N;        // output columns (weight rows; gate rows for kSiluMul)
  bf16_t* y;        // kStore / kSiluMul: [M, ldy]; kArgmax: optional logits [M, ldy]; kAddResidual: R [M, ldy]
  int64_t ldy;
  uint64_t* best;   // kArgmax: [num_tiles, M]
};

template <int NA, int NB, int EPI, int KSPLIT>
__global__ __launch_bounds__(64 * KSPLIT) void gemm_kernel(GemmArgs args) {
  constexpr int kTileRows = 16 * NA;            // output columns of this workgroup
  constexpr int kLoadTiles = (EPI == kSiluMul) ? 2 * NA : NA;  // gate + up tiles for kSiluMul
  __shared__ f32x4 red[KSPLIT > 1 ? KSPLIT - 1 : 1][KSPLIT > 1 ? kLoadTiles * NB : 1][KSPLIT > 1 ? 64 : 1];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * kTileRows;
  const int64_t K = args.K;
  const int64_t k_per_wave = K / KSPLIT;
  const int64_t k_begin = wave * k_per_wave, k_end = k_begin + k_per_wave;

  // Weight row pointers of this lane, one per loaded tile (rows past N clamp
  // to the last row; their results are dropped).
  const bf16_t* wrow[kLoadTiles];
#pragma unroll
  for (int a = 0; a < kLoadTiles; ++a) {
    int64_t row = n0 + 16 * (a % NA) + r;
    row = row < args.N ? row : args.N - 1;
    if (EPI == kSiluMul && a >= NA) row += args.N;
    wrow[a] = args.w + row * K + 32 * g;
  }
  const bf16_t* xrow[NB];
  bool xvalid[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int tok = 16 * bt + r;
    xvalid[bt] = tok < args.M;
    xrow[bt] = args.x + (int64_t)(xvalid[bt] ? tok : 0) * args.ldx + 32 * g;
  }

  f32x4 acc[kLoadTiles][NB];
#pragma unroll
  for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) acc[a][bt] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 wa[kLoadTiles][4], wn[kLoadTiles][4];
#pragma unroll
  for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
    for (int i = 0; i < 4; ++i) wa[a][i] = ld128_nt(wrow[a] + k_begin + 8 * i);

  for (int64_t k = k_begin; k < k_end; k += kKStep) {
    const bool more = k + kKStep < k_end;
    if (more) {
#pragma unroll
      for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) wn[a][i] = ld128_nt(wrow[a] + k + kKStep + 8 * i);
    }
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
      u32x4 xb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) xb[i] = xvalid[bt] ? ld128(xrow[bt] + k + 8 * i) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[a][bt] = mfma_16x16x32(wa[a][i], xb[i], acc[a][bt]);
    }
    if (more) {
#pragma unroll
      for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) wa[a][i] = wn[a][i];
    }
  }

  if constexpr (KSPLIT > 1) {
    if (wave > 0) {
#pragma unroll
      for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) red[wave - 1][a * NB + bt][lane] = acc[a][bt];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < KSPLIT - 1; ++w)
#pragma unroll
      for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) acc[a][bt] += red[w][a * NB + bt][lane];
  }

  // Epilogue on wave 0: lane holds tile rows 4g + j (j < 4) for token 16 bt + r.
  if constexpr (EPI == kArgmax) {
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
      const int tok = 16 * bt + r;
      uint64_t best = 0;
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        const int64_t col0 = n0 + 16 * a + 4 * g;
        uint32_t packed[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t b16 = f2bf(acc[a][bt][j]);
          packed[j >> 1] |= b16 << (16 * (j & 1));
          if (col0 + j < args.N) {
            const uint64_t key = argmax_key(b16 << 16, (uint32_t)(col0 + j));
            best = key > best ? key : best;
          }
        }
        if (args.y && tok < args.M && col0 + 3 < args.N)
          *reinterpret_cast<u32x2*>(args.y + (int64_t)tok * args.ldy + col0) = u32x2{packed[0], packed[1]};
        else if (args.y && tok < args.M) {
          for (int j = 0; j < 4; ++j)
            if (col0 + j < args.N)
              args.y[(int64_t)tok * args.ldy + col0 + j] = (bf16_t)((packed[j >> 1] >> (16 * (j & 1))) & 0xffffu);
        }
      }
      uint64_t o = shfl_xor_u64(best, 16);
      best = o > best ? o : best;
      o = shfl_xor_u64(best, 32);
      best = o > best ? o : best;
      if (g == 0 && tok < args.M) args.best[(int64_t)blockIdx.x * args.M + tok] = best;
    }
  } else {
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
      const int tok = 16 * bt + r;
      if (tok >= args.M) continue;
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        const int64_t col0 = n0 + 16 * a + 4 * g;
        float out[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = round_bf16(acc[a][bt][j]);
          if constexpr (EPI == kSiluMul) {
            const float u = round_bf16(acc[NA + a][bt][j]);
            const float s = round_bf16(v / (1.0f + expf(-v)));
            out[j] = s * u;
          } else {
            out[j] = v;
          }
        }
        bf16_t* dst = args.y + (int64_t)tok * args.ldy + col0;
        if constexpr (EPI == kAddResidual) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (col0 + j < args.N) out[j] = out[j] + bf2f(dst[j]);
        }
        if (col0 + 3 < args.N) {
          *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf(out[0], out[1]), pack_bf(out[2], out[3])};
        } else {
          for (int j = 0; j < 4; ++j)
            if (col0 + j < args.N) dst[j] = (bf16_t)f2bf(out[j]);
        }
      }
    }
  }
}

// Cross-tile argmax: predicted[m] = column of the largest key over all tiles.
__global__ __launch_bounds__(256) void argmax_reduce_kernel(const uint64_t* __restrict__ best, int num_tiles, int M,
                                                            int64_t* __restrict__ predicted) {
  __shared__ uint64_t part[256 / kWave];
  const int m = blockIdx.x;
  uint64_t b = 0;
  for (int t = threadIdx.x; t < num_tiles; t += blockDim.x) {
    const uint64_t v = best[(int64_t)t * M + m];
    b = v > b ? v : b;
  }
#pragma unroll
  for (int mask = 1; mask < kWave; mask <<= 1) {
    const uint64_t o = shfl_xor_u64(b, mask);
    b = o > b ? o : b;
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 256 / kWave; ++w) b = part[w] > b ? part[w] : b;
    b = part[0] > b ? part[0] : b;
    predicted[m] = (int64_t)(uint32_t)(~(uint32_t)b);
  }
}

template <int NA, int NB, int EPI, int KSPLIT>
int launch_gemm(const GemmArgs& a, int64_t tiles, hipStream_t s) {
  hipLaunchKernelGGL((gemm_kernel<NA, NB, EPI, KSPLIT>), dim3((unsigned)tiles), dim3(64 * KSPLIT), 0, s, a);
  return OXR_LAUNCH_STATUS();
}

template <int NA, int EPI, int KSPLIT>
int dispatch_nb(const GemmArgs& a, int64_t tiles, hipStream_t s) {
  const int nb = (a.M + 15) / 16;
  switch (nb) {
    case 1: return launch_gemm<NA, 1, EPI, KSPLIT>(a, tiles, s);
    case 2: return launch_gemm<NA, 2, EPI, KSPLIT>(a, tiles, s);
    case 3: return launch_gemm<NA, 3, EPI, KSPLIT>(a, tiles, s);
    case 4: return launch_gemm<NA, 4, EPI, KSPLIT>(a, tiles, s);
    default: return OXR_ERR_UNSUPPORTED;
  }
}

template <int NA, int EPI>
int dispatch_split(const GemmArgs& a, int64_t tiles, int ksplit, hipStream_t s) {
  switch (ksplit) {
    case 1: return dispatch_nb<NA, EPI, 1>(a, tiles, s);
    case 2: return dispatch_nb<NA, EPI, 2>(a, tiles, s);
    case 4: return dispatch_nb<NA, EPI, 4>(a, tiles, s);
    case 8: return dispatch_nb<NA, EPI, 8>(a, tiles, s);
    default: return OXR_ERR_UNSUPPORTED;
  }
}

// Waves per workgroup: enough workgroups and waves to keep every CU
// streaming, with at least one 128-k stage per wave.
int choose_split(int64_t tiles, int64_t K) {
  int split = 1;
  while (split < 8 && tiles * split < 1024 && (K / (split * 2)) % kKStep == 0 && K / (split * 2) >= kKStep) split *= 2;
  return split;
}

int check_common(const void* x, int64_t ldx, int64_t M, const void* w, int64_t K, int64_t N) {
  OXR_RETURN_IF(M < 0 || K <= 0 || N <= 0 || ldx < K, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(M > 64 || K % kKStep != 0, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(M > 0 && (!x || !w), OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(((uintptr_t)x | (uintptr_t)w) % 16 != 0 || ldx % 8 != 0, OXR_ERR_UNSUPPORTED);
  return OXR_OK;
}

}  // namespace
}  // namespace oxr

extern "C" int oxr_gemm_bf16(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w, int64_t k, int64_t n,
                             int32_t epilogue, oxr_bf16* y, int64_t ldy, oxr_stream_t stream) {
  using namespace oxr;
  int st = check_common(x, ldx, m, w, k, n);
  if (st) return st;
  OXR_RETURN_IF(epilogue != kStore && epilogue != kSiluMul && epilogue != kAddResidual, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(!y || ldy < n || ldy % 4 != 0 || (uintptr_t)y % 8 != 0, OXR_ERR_INVALID_ARG);
  if (m == 0) return OXR_OK;
  GemmArgs a{x, ldx, (int)m, w, k, n, y, ldy, nullptr};
  hipStream_t s = (hipStream_t)stream;
  if (epilogue == kSiluMul) {
    const int64_t tiles = (n + 15) / 16;
    return dispatch_split<1, kSiluMul>(a, tiles, choose_split(tiles, k), s);
  }
  const int64_t tiles = (n + 15) / 16;
  if (epilogue == kAddResidual) return dispatch_split<1, kAddResidual>(a, tiles, choose_split(tiles, k), s);
  return dispatch_split<1, kStore>(a, tiles, choose_split(tiles, k), s);
}

extern "C" size_t oxr_lm_head_workspace_bytes(int64_t m, int64_t vocab) {
  if (m <= 0 || vocab <= 0) return 0;
  return (size_t)((vocab + 31) / 32) * (size_t)m * sizeof(uint64_t);
}

extern "C" int oxr_lm_head_argmax(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight, int64_t hidden_size,
                                  int64_t vocab, oxr_bf16* logits, int64_t* predicted, void* workspace,
                                  size_t workspace_bytes, oxr_stream_t stream) {
  using namespace oxr;
  int st = check_common(hidden, hidden_size, m, weight, hidden_size, vocab);
  if (st) return st;
  OXR_RETURN_IF(!predicted, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(logits && (uintptr_t)logits % 8 != 0, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(vocab > 0x7fffffffLL, OXR_ERR_UNSUPPORTED);
  if (m == 0) return OXR_OK;
  const size_t need = oxr_lm_head_workspace_bytes(m, vocab);
  OXR_RETURN_IF(!workspace || workspace_bytes < need, OXR_ERR_WORKSPACE);
  const int64_t tiles = (vocab + 31) / 32;
  GemmArgs a{hidden, hidden_size, (int)m, weight, hidden_size, vocab, logits, vocab, static_cast<uint64_t*>(workspace)};
  hipStream_t s = (hipStream_t)stream;
  st = dispatch_split<2, kArgmax>(a, tiles, 1, s);
  if (st) return st;
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3((unsigned)m), dim3(256), 0, s, static_cast<const uint64_t*>(workspace),
                     (int)tiles, (int)m, predicted);
  return OXR_LAUNCH_STATUS();
}
