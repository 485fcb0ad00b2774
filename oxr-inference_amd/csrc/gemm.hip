// Weight-streaming bf16 GEMMs for the verify step (gfx950): Y = X * W^T.
//
// The verify step multiplies a handful of token rows (M = B * S = 32 at B=8,
// S=4) by large weights: every projection and the LM head is HBM-bound on the
// weight read.  So the kernel is organised around streaming W exactly once:
//
// * A workgroup owns one tile of 16 * NA weight rows (output columns), all
//   M <= 16 * NB token rows, and one of `k_splits` slices of K; its WAVES
//   waves split that slice further.  A wave walks its k range in 128-k steps
//   of four load instructions per 16-row tile: instruction i brings lane
//   (r, g) W[row r][k + 32i + 8g, +8), its A-operand fragment of
//   v_mfma_f32_16x16x32_bf16 for k-step i, and the X fragments follow the
//   same mapping (X is at most 64 rows and stays in L2).  Step i + 1's W and
//   X are in flight while step i is multiplied; there are no dependent loads
//   in the loop, so the in-order vmcnt waits only ever wait for the step
//   being consumed.
// * What bounds these kernels is the vector memory pipeline's rate over cache
//   lines, not HBM bytes: an instruction of the row-major mapping touches 16
//   rows' worth of lines.  Weights may therefore come pre-packed (PW, written
//   once by oxr_pack_weight_bf16): for every 16-row tile t and 128-k step q,
//   four contiguous 1 KiB blocks, block i holding the fragments of k-step i in
//   lane order (lane 16g + r: W[16t + r][128q + 32i + 8g, +8)), so each load
//   instruction reads 1 KiB of contiguous memory.  Same arithmetic, same
//   order: packed and row-major results are bit-identical.  The token rows X
//   may come packed the same way (PX: 16-token tiles, written so by the
//   kernels that produce them), and kStore / kSiluMul can write Y packed for
//   the next GEMM.
// * The waves' fp32 tiles are summed in LDS in a fixed order, then the
//   epilogue runs on the finished tile:
//     kStore        Y = bf16(acc)
//     kSiluMul      rows [0, N) are gate and [N, 2N) up (the fused gate_up
//                   weight, language.py:238): Y = bf16(bf16(silu(bf16(g))) * bf16(u))
//                   (the reference's rounding points, language.py:102-104)
//     kArgmax       per token the largest bf16-rounded logit of the tile,
//                   lowest column on ties, as a 64-bit key for a later
//                   cross-tile max; optionally also stores the bf16 logits
//     kAddResidual  R = bf16(bf16(acc) + R) in place: the residual add of
//                   _add_rms_norm (language.py:94-99)
//     kPartial      fp32 partial sums of k-slice blockIdx.y, for weights too
//                   narrow to fill the chip with whole-K tiles; the
//                   add + RMSNorm that follows sums them (csrc/norm.hip), so
//                   no workgroup ever waits for another.
// C layout: lane (l % 16, g) holds rows 4g..4g+3 of the tile for token l % 16.
#include <algorithm>

#include "common.h"
#include "lm_head_keys.h"

namespace oxr {
namespace {

enum Epilogue { kStore = 0, kSiluMul = 1, kArgmax = 2, kAddResidual = 3, kPartial = 4 };

constexpr int kKStep = 128;  // k per pipeline stage: 4 MFMA k-steps of 32

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
  int y_packed;     // kStore / kSiluMul: y in the packed layout with row length N (ldy unused)
  uint64_t* best;   // kArgmax: [num_tiles, M]
  float* part;      // kPartial: [k_splits, part_rows, N], this launch's rows first
  int64_t part_rows;
};

// Weight fragments are streamed once per step, so they are loaded non-temporally: measured on the
// verify step, 2225 vs 2255 us, the 32-row LM head 103 vs 117 us (6.0 TB/s).  (The context K/V in
// the attention kernel, also read once, got slower that way: 41.6 vs 36.0 us per launch.)  The fp32
// partials use ordinary stores: non-temporal ones made the step 20 us slower (their reader, the
// add + RMSNorm that follows, gains from the lines staying cached).
__device__ __forceinline__ u32x4 ld_w(const void* p) { return ld128_nt(p); }

template <int NT, int NB>
struct Stage {
  u32x4 w[NT][4];
  u32x4 x[NB][4];
};

template <int NA, int NB, int EPI, int WAVES, bool PW, bool PX>
__global__ __launch_bounds__(64 * WAVES) void gemm_kernel(GemmArgs args) {
  constexpr int kTileRows = 16 * NA;                          // output columns of this workgroup
  constexpr int kLoadTiles = (EPI == kSiluMul) ? 2 * NA : NA;  // gate + up tiles for kSiluMul
  __shared__ f32x4 red[WAVES > 1 ? WAVES - 1 : 1][WAVES > 1 ? kLoadTiles * NB : 1][WAVES > 1 ? 64 : 1];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * kTileRows;
  const int64_t K = args.K;
  const int64_t k_slice = K / gridDim.y;
  const int64_t k_per_wave = k_slice / WAVES;
  const int64_t k_begin = blockIdx.y * k_slice + wave * k_per_wave;  // this wave walks [k_begin, k_begin + k_per_wave)

  // Weight pointers of this lane, one per loaded tile (rows past N clamp to
  // the last row, or tile, whose results are dropped).  Packed: the lane's
  // fragment of the tile's first block; step k's block i is at + 16k + 512i.
  const bf16_t* wrow[kLoadTiles];
#pragma unroll
  for (int a = 0; a < kLoadTiles; ++a) {
    int64_t row = n0 + 16 * (a % NA) + r;
    row = row < args.N ? row : args.N - 1;
    if (EPI == kSiluMul && a >= NA) row += args.N;
    wrow[a] = PW ? args.w + (row >> 4) * (K * 16) + lane * 8 : args.w + row * K + 8 * g;
  }
  // Token rows past M read row 0 (packed: the tile's padding) and multiply
  // into accumulators nobody stores.
  const bf16_t* xrow[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int tok = 16 * bt + r;
    xrow[bt] = PX ? args.x + (int64_t)bt * (K * 16) + lane * 8
                  : args.x + (int64_t)(tok < args.M ? tok : 0) * args.ldx + 8 * g;
  }

  f32x4 acc[kLoadTiles][NB];
#pragma unroll
  for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) acc[a][bt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto load = [&](Stage<kLoadTiles, NB>& st, int64_t k) {
#pragma unroll
    for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) st.w[a][i] = ld_w(PW ? wrow[a] + 16 * k + 512 * i : wrow[a] + k + 32 * i);
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int i = 0; i < 4; ++i) st.x[bt][i] = ld128(PX ? xrow[bt] + 16 * k + 512 * i : xrow[bt] + k + 32 * i);
  };

  auto compute = [&](const Stage<kLoadTiles, NB>& st) {
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[a][bt] = mfma_16x16x32(st.w[a][i], st.x[bt][i], acc[a][bt]);
  };

  // Two stages, A and B, alternate without register copies, and every load in
  // the loop is unconditional, so the vmcnt wait before each multiply leaves
  // the other stage's loads in flight (a conditional load, or a copy of a
  // stage still being loaded, would make the compiler wait for everything).
  // The last one or two steps are peeled off.  The scheduling barriers keep
  // the loads ahead of the multiplies that they overlap.
  const int steps = (int)(k_per_wave / kKStep);
  Stage<kLoadTiles, NB> sa, sb;
  load(sa, k_begin);
  __builtin_amdgcn_sched_barrier(0);
  int i = 0;
  for (; i + 2 < steps; i += 2) {
    const int64_t k = k_begin + (int64_t)i * kKStep;
    load(sb, k + kKStep);
    __builtin_amdgcn_sched_barrier(0);
    compute(sa);
    __builtin_amdgcn_sched_barrier(0);
    load(sa, k + 2 * kKStep);
    __builtin_amdgcn_sched_barrier(0);
    compute(sb);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (i + 1 < steps) {
    load(sb, k_begin + (int64_t)(i + 1) * kKStep);
    __builtin_amdgcn_sched_barrier(0);
    compute(sa);
    __builtin_amdgcn_sched_barrier(0);
    compute(sb);
  } else {
    compute(sa);
  }

  if constexpr (WAVES > 1) {
    if (wave > 0) {
#pragma unroll
      for (int a = 0; a < kLoadTiles; ++a)
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) red[wave - 1][a * NB + bt][lane] = acc[a][bt];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < WAVES - 1; ++w)
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
  } else if constexpr (EPI == kPartial) {
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
      const int tok = 16 * bt + r;
      if (tok >= args.M) continue;
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        const int64_t col0 = n0 + 16 * a + 4 * g;
        float* dst = args.part + ((int64_t)blockIdx.y * args.part_rows + tok) * args.N + col0;
        if (col0 + 3 < args.N) {
          *reinterpret_cast<f32x4*>(dst) = acc[a][bt];
        } else {
          for (int j = 0; j < 4; ++j)
            if (col0 + j < args.N) dst[j] = acc[a][bt][j];
        }
      }
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
        bf16_t* dst = args.y + (args.y_packed ? packed_offset(tok, col0, args.N) : (int64_t)tok * args.ldy + col0);
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


// Argmax of logits the caller already holds (fp32 or bf16 [rows, ld], first `vocab` columns):
// the eager path's logits.argmax(dim=-1) (engine.py:726).  Each row is cut into `gridDim.x`
// column chunks, one workgroup each, so a few rows still spread over the chip; every thread
// keeps the best key of its strided 16-byte pieces, the workgroup reduces them, and
// argmax_reduce_kernel merges the chunks (the keys order values, then lower columns first).
template <typename T>
__device__ __forceinline__ uint32_t logit_bits(T v);
template <>
__device__ __forceinline__ uint32_t logit_bits<float>(float v) { return __float_as_uint(v); }
template <>
__device__ __forceinline__ uint32_t logit_bits<bf16_t>(bf16_t v) { return (uint32_t)v << 16; }

template <typename T, bool kVec>
__global__ __launch_bounds__(256) void argmax_rows_kernel(const T* __restrict__ logits, int64_t ld, int64_t vocab,
                                                          int rows, uint64_t* __restrict__ best) {
  constexpr int kPer = 16 / sizeof(T);  // elements per 16-byte piece
  __shared__ uint64_t part[256 / kWave];
  const int row = blockIdx.y;
  const T* src = logits + (int64_t)row * ld;
  const int64_t pieces = (vocab + kPer - 1) / kPer;
  const int64_t per_chunk = (pieces + gridDim.x - 1) / gridDim.x;
  const int64_t p0 = (int64_t)blockIdx.x * per_chunk;
  const int64_t p1 = p0 + per_chunk < pieces ? p0 + per_chunk : pieces;
  uint64_t b = 0;
  for (int64_t p = p0 + threadIdx.x; p < p1; p += blockDim.x) {
    const int64_t c0 = p * kPer;
    T v[kPer];
    if (kVec && c0 + kPer <= vocab) {
      *reinterpret_cast<u32x4*>(v) = ld128(src + c0);
    } else {
#pragma unroll
      for (int e = 0; e < kPer; ++e) v[e] = c0 + e < vocab ? src[c0 + e] : src[0];
    }
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      if (c0 + e < vocab) {
        const uint64_t key = argmax_key(logit_bits<T>(v[e]), (uint32_t)(c0 + e));
        b = key > b ? key : b;
      }
    }
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
    best[(int64_t)blockIdx.x * rows + row] = b;
  }
}

// Column chunks per row: about 1024 workgroups in all, each at least 4096 columns.
int argmax_chunks(int64_t rows, int64_t vocab) {
  int64_t c = (1024 + rows - 1) / rows;
  const int64_t by_cols = (vocab + 4095) / 4096;
  c = c < by_cols ? c : by_cols;
  return (int)(c < 1 ? 1 : (c > 1024 ? 1024 : c));
}

// ---------------------------------------------------------------------------
// Persistent LM head for M <= 32 token rows.  Every weight byte is read once,
// so the kernel is bound by the rate at which the CUs' vector memory path
// returns data -- and a per-wave copy of the token rows X would cost as much
// of that path as the weights themselves (the tile kernel above loads X once
// per wave).  Here one workgroup per CU stages all of X in LDS once, in MFMA
// fragment order, and its 8 waves stream 16-row weight tiles through a
// kLmDepth-stage register ring, reading X fragments from LDS.  Each wave keeps
// a running best key per token across its tiles; the workgroup writes one key
// per token, reduced across workgroups by argmax_reduce_kernel.
// ---------------------------------------------------------------------------
constexpr int kLmWaves = 8;
constexpr int kLmDepth = 4;          // weight stages in flight per wave
constexpr int kLmMaxK = 2048;        // X in LDS: NB * 16 * K * 2 bytes <= 128 KB
constexpr int kLmStageThreads = 64 * kLmWaves;

template <int NB, int K, bool PW>
__global__ __launch_bounds__(64 * kLmWaves) void lm_head_lds_kernel(const bf16_t* __restrict__ x, int64_t ldx, int M,
                                                                   const bf16_t* w, int64_t N,
                                                                   bf16_t* __restrict__ logits, int64_t ldl,
                                                                   uint64_t* __restrict__ best_out) {
  static_assert(K % (kKStep * kLmDepth) == 0 && K <= kLmMaxK, "unsupported hidden size");
  // xs[((q * 4 + i) * NB + bt) * 64 + lane] = X[16 bt + lane % 16][128 q + 32 i + 8 (lane / 16), +8): the B
  // fragment of MFMA i of k-stage q for token tile bt, matching the weight fragments' k-slot mapping.
  extern __shared__ u32x4 xs[];
  __shared__ uint64_t wave_best[kLmWaves][NB * 16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  constexpr int ksteps = K / kKStep;
  const int64_t num_tiles = (N + 15) / 16;
  const int64_t gw = (int64_t)blockIdx.x * kLmWaves + wave, nw = (int64_t)gridDim.x * kLmWaves;
  const int64_t my_tiles = gw < num_tiles ? (num_tiles - 1 - gw) / nw + 1 : 0;
  const int64_t total = my_tiles * ksteps;  // weight stages of this wave, in (tile, q) order

  // Stage s of this wave: tile gw + (s / ksteps) * nw, k-stage s % ksteps.  Past the end it re-reads the
  // last stage (an L2 hit), so every load in the loop is unconditional and the vmcnt waits are exact.
  auto stage_ptr = [&](int64_t s) {
    s = s < total ? s : total - 1;
    s = s > 0 ? s : 0;  // a wave without tiles reads (and never uses) the last weight row
    int64_t row = (gw + (s / ksteps) * nw) * 16 + r;
    row = row < N ? row : N - 1;
    if constexpr (PW) return w + (row >> 4) * (K * 16) + (s % ksteps) * (16 * kKStep) + lane * 8;
    return w + row * K + (s % ksteps) * kKStep + 8 * g;
  };
  auto load = [&](u32x4 (&dst)[4], int64_t s) {
    const bf16_t* p = stage_ptr(s);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = ld_w(p + (PW ? 512 * i : 32 * i));
  };

  // 1. X rows into registers (unconditional: indices past the end re-read the last chunk), then the first
  //    weight stages, then X into LDS -- the LDS writes wait only for the X loads.
  constexpr int kChunks = NB * 16 * (K / 8) / kLmStageThreads;  // 16-byte pieces of X per thread
  static_assert(NB * 16 * (K / 8) % kLmStageThreads == 0, "X staging must divide evenly");
  u32x4 xr[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int idx = threadIdx.x + c * kLmStageThreads;
    const int m = idx / (K / 8), k = (idx % (K / 8)) * 8;
    xr[c] = ld128(x + (int64_t)(m < M ? m : M - 1) * ldx + k);  // rows past M: results never read
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 ring[kLmDepth][4];
#pragma unroll
  for (int d = 0; d < kLmDepth; ++d) load(ring[d], d);
  // Keep these loads here, in flight during the LDS writes and the barrier
  // (the compiler would otherwise sink them to their first use).
  __asm__ __volatile__("" ::: "memory");
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int idx = threadIdx.x + c * kLmStageThreads;
    const int m = idx / (K / 8), k = (idx % (K / 8)) * 8;
    const int q = k / kKStep, kk = k % kKStep, ii = kk / 32, gg = (kk % 32) / 8;
    xs[((q * 4 + ii) * NB + m / 16) * 64 + gg * 16 + (m % 16)] = xr[c];
  }
  __syncthreads();

  uint64_t best[NB];
  f32x4 acc[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    best[bt] = 0;
    acc[bt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // ksteps is a multiple of kLmDepth (checked on the host), so a tile ends at d == kLmDepth - 1.
  for (int64_t s = 0; s < total; s += kLmDepth) {
#pragma unroll
    for (int d = 0; d < kLmDepth; ++d) {
      const int q = (int)((s + d) % ksteps);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int bt = 0; bt < NB; ++bt)
          acc[bt] = mfma_16x16x32(ring[d][i], xs[((q * 4 + i) * NB + bt) * 64 + lane], acc[bt]);
      load(ring[d], s + d + kLmDepth);
    }
    if ((s + kLmDepth) % ksteps == 0) {
      const int64_t col0 = (gw + (s / ksteps) * nw) * 16 + 4 * g;
#pragma unroll
      for (int bt = 0; bt < NB; ++bt) {
        const int tok = 16 * bt + r;
        uint32_t b16[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          b16[j] = f2bf(acc[bt][j]);
          if (col0 + j < N) {
            const uint64_t key = argmax_key(b16[j] << 16, (uint32_t)(col0 + j));
            best[bt] = key > best[bt] ? key : best[bt];
          }
        }
        if (logits && tok < M) {
          bf16_t* dst = logits + (int64_t)tok * ldl + col0;
          if (col0 + 3 < N) {
            *reinterpret_cast<u32x2*>(dst) = u32x2{b16[0] | (b16[1] << 16), b16[2] | (b16[3] << 16)};
          } else {
            for (int j = 0; j < 4; ++j)
              if (col0 + j < N) dst[j] = (bf16_t)b16[j];
          }
        }
        acc[bt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }

  // Best key per token: across the 4 lane groups, then the waves, then one store per workgroup.
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    uint64_t o = shfl_xor_u64(best[bt], 16);
    best[bt] = o > best[bt] ? o : best[bt];
    o = shfl_xor_u64(best[bt], 32);
    best[bt] = o > best[bt] ? o : best[bt];
    if (g == 0) wave_best[wave][16 * bt + r] = best[bt];
  }
  __syncthreads();
  if (threadIdx.x < M) {
    uint64_t b = 0;
#pragma unroll
    for (int wv = 0; wv < kLmWaves; ++wv) b = wave_best[wv][threadIdx.x] > b ? wave_best[wv][threadIdx.x] : b;
    best_out[(int64_t)blockIdx.x * M + threadIdx.x] = b;
  }
}

// ---------------------------------------------------------------------------
// LM head for 33..256 token rows (packed weight): with M = 256 the head does
// 159 GFLOP on 622 MB, close to the MFMA/HBM ridge, so the products use the
// 32x32x16 MFMA (twice the work per issue of the 16x16x32 form on gfx950) and
// the weight is still read exactly once.  One persistent workgroup per CU
// owns a balanced contiguous range of 32-row vocab tiles, taken 8 at a time
// (a group): wave w multiplies vocab tile w of the group by all token rows
// (128 accumulators and a 2-chunk weight ring per wave).
// * Each wave streams its own weight rows straight into registers through a
//   kWideDepth-chunk ring (64 k per chunk; a lane's 16-byte fragment of the
//   packed layout -- four contiguous 256-byte runs per instruction).
// * The token rows (packed by the entry point into the workspace) are shared
//   by all 8 waves: chunk by chunk, loaded straight into LDS (four buffers,
//   two chunks ahead of use -- at least as far ahead as the weight ring, so
//   that waiting for a chunk (the vector memory counter is in order) never
//   waits for a weight chunk that is not due yet -- one
//   barrier per chunk) in the packed order, so each 16-lane fragment read is
//   one contiguous 256-byte run.
// * Epilogue per group: bf16-rounded logits -> per-token best keys, merged
//   into the wave's slot in LDS; at the end one key per token per workgroup,
//   reduced across workgroups by argmax_reduce_kernel.
// ---------------------------------------------------------------------------
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWideWaves = 8;      // waves per workgroup (two per SIMD) = vocab tiles per group
constexpr int kWideTokTiles = 8;   // 32-token tiles (M <= 256)
constexpr int kWideChunk = 64;     // k per stage
constexpr int kWideDepth = 2;      // weight chunks in flight per wave (two waves per SIMD: 256 registers)
constexpr int kXBlocksPerWave = 32 / kWideWaves;  // 1 KiB blocks of a token-row chunk staged per wave
constexpr int kUnroll = 8;         // stages per unrolled step: ring slot and LDS buffer fixed per position
constexpr int kWideMaxGrid = 1024; // bound on the workgroups (sizes the workspace)
constexpr int kWideMaxRows = 32 * kWideTokTiles;

// s_waitcnt immediate (gfx9 encoding) waiting until at most `n` vector memory operations are outstanding,
// with the other counters unconstrained: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

__device__ __forceinline__ f32x16 mfma_32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

// The TT token-row fragments of one k16 step from LDS: 16 bytes per lane at byte address a + 4096 tt,
// all requested before one wait, in one asm block.  As inline asm the reads are invisible to the
// compiler's tracking of the token-row loads into LDS; that tracking cannot tell across the loop's back
// edge which load wrote a buffer, and would otherwise wait for every load in flight once per pass.
// The counted waits and barriers around the reads already order them after those loads.
template <int TT>
__device__ __forceinline__ void lds_fragments(u32x4 (&x)[TT], uint32_t a);
template <>
__device__ __forceinline__ void lds_fragments<2>(u32x4 (&x)[2], uint32_t a) {
  asm volatile(
      "ds_read_b128 %0, %2\n\t"
      "ds_read_b128 %1, %2 offset:4096\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1])
      : "v"(a));
}
template <>
__device__ __forceinline__ void lds_fragments<4>(u32x4 (&x)[4], uint32_t a) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %4 offset:4096\n\t"
      "ds_read_b128 %2, %4 offset:8192\n\t"
      "ds_read_b128 %3, %4 offset:12288\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3])
      : "v"(a));
}
template <>
__device__ __forceinline__ void lds_fragments<8>(u32x4 (&x)[8], uint32_t a) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %8 offset:4096\n\t"
      "ds_read_b128 %2, %8 offset:8192\n\t"
      "ds_read_b128 %3, %8 offset:12288\n\t"
      "ds_read_b128 %4, %8 offset:16384\n\t"
      "ds_read_b128 %5, %8 offset:20480\n\t"
      "ds_read_b128 %6, %8 offset:24576\n\t"
      "ds_read_b128 %7, %8 offset:28672\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7])
      : "v"(a));
}

// TT: 32-token tiles computed (2, 4 or 8; rows past M are padding whose results nobody reads).
template <int K, int TT>
__global__ __launch_bounds__(64 * kWideWaves) void lm_head_wide_kernel(const bf16_t* __restrict__ xp, int M,
                                                                      const bf16_t* w, int64_t N,
                                                                      bf16_t* __restrict__ logits, int64_t ldl,
                                                                      uint64_t* __restrict__ best_out) {
  constexpr int kChunks = K / kWideChunk;
  static_assert(K % 128 == 0, "packed k steps are 128 wide");
  // X chunk: token row tile t (16 tokens) x block i (32 k) at (2t + i) * 512 elements, lane order inside.
  // Four buffers (stage s reads s % 4; chunks go in two stages ahead), as separate arrays so the compiler
  // can tell a load into one from reads of another.
  __shared__ bf16_t xs0[kWideTokTiles * 2 * 2 * 512], xs1[kWideTokTiles * 2 * 2 * 512];
  __shared__ bf16_t xs2[kWideTokTiles * 2 * 2 * 512], xs3[kWideTokTiles * 2 * 2 * 512];
  __shared__ uint64_t wave_best[kWideWaves][kWideMaxRows];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, h = lane >> 5, r = lane & 15;
  const int x_tiles = (M + 15) / 16;             // packed 16-row token tiles present
  const int64_t w_last = (N + 15) / 16 - 1;       // last packed 16-row weight tile
  const int64_t nt32 = (N + 31) / 32;
  const int64_t lo = (int64_t)blockIdx.x * nt32 / gridDim.x, hi = (int64_t)(blockIdx.x + 1) * nt32 / gridDim.x;
  const int64_t groups = (hi - lo + kWideWaves - 1) / kWideWaves;
  const int64_t stages = groups * kChunks;

  for (int i = tid; i < kWideWaves * kWideMaxRows; i += 64 * kWideWaves) (&wave_best[0][0])[i] = 0;

  // Weight fragment of stage s (group s / kChunks, chunk s % kChunks), k16 step kk: lane (n, h) holds
  // W[32 vt + n][64 c + 16 kk + 8h, +8).  A wave without a vocab tile in a group (the last group of a
  // range that is not a multiple of kWideWaves, or past the last stage) still issues the load, so every
  // wave's counted waits hold, but reads the same offset in the first token-row tile (cached, in range:
  // the offset is below 16 K) and computes nothing with it.
  auto wfrag = [&](int64_t s, int kk) {
    s = s < stages ? s : stages - 1;
    const int64_t gi = s / kChunks;
    const int c = (int)(s - gi * kChunks);
    const int64_t vt = lo + gi * kWideWaves + wave;
    int64_t t = 2 * vt + (n >> 4);
    t = t < w_last ? t : w_last;
    const int i = 2 * (c & 1) + (kk >> 1), g = 2 * (kk & 1) + h;
    const int64_t inner = (c >> 1) * (16 * kKStep) + i * 512 + (16 * g + r) * 8;
    return ld_w((vt < hi ? w + t * (K * 16) : xp) + inner);  // vt < hi is wave-uniform
  };
  // Token rows of chunk c straight into an LDS buffer (global_load_lds, 16 bytes per lane: lane i of an
  // instruction writes bytes [16i, 16i + 16) of a 1 KiB block): 32 blocks (block j: token row tile j / 2,
  // half j % 2 of the chunk's 64 k), kXBlocksPerWave per wave.  Tiles past the last one re-read it.
  auto xdma = [&](int c, bf16_t* dst) {
#pragma unroll
    for (int u = 0; u < kXBlocksPerWave; ++u) {
      const int j = kXBlocksPerWave * wave + u, t = j >> 1;
      const int tl = t < x_tiles ? t : x_tiles - 1;
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(xp + (int64_t)tl * (K * 16) + (c >> 1) * (16 * kKStep) +
                                                          (2 * (c & 1) + (j & 1)) * 512 + lane * 8),
          (void __attribute__((address_space(3)))*)(dst + j * 512), 16, 0, 0);
    }
  };

  u32x4 ring[kWideDepth][4];
#pragma unroll
  for (int d = 0; d < kWideDepth; ++d)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) ring[d][kk] = wfrag(d, kk);
  // Stage s's token rows go in at stage s - 2 (chunk c of stage s is s % kChunks; past the last stage the
  // loads repeat a valid chunk into a buffer nobody reads), so every stage issues the same loads: its
  // token-row block loads, then its 4 weight loads.  At the end of stage s, the loads issued after
  // stage s + 1's token rows are 4 + (kXBlocksPerWave + 4); everything older has landed.
  auto xchunk = [&](int64_t st) { return (int)((st < stages ? st : stages - 1) % kChunks); };
  xdma(xchunk(0), xs0);
  xdma(xchunk(1), xs1);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(kXBlocksPerWave));
  __syncthreads();

  f32x16 acc[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[tt][e] = 0.f;

  // Stage s = gi * kChunks + c: chunk c of group gi.  kChunks is a multiple of kWideDepth (even), so
  // stage s uses ring slot s % kWideDepth and LDS buffer s % 2, both fixed per unrolled position.
  static_assert(kChunks % kUnroll == 0 && kUnroll % kWideDepth == 0 && kUnroll % 4 == 0,
                "ring slots and buffers must be static");
  for (int64_t gi = 0; gi < groups; ++gi) {
    // Waves without a vocab tile in this group skip the products (wave-uniform); their loads and
    // barriers are the same as everyone's.
    const bool active = lo + gi * kWideWaves + wave < hi;
    for (int c0 = 0; c0 < kChunks; c0 += kUnroll) {
#pragma unroll
      for (int d = 0; d < kUnroll; ++d) {
        const int c = c0 + d;
        const int64_t s = gi * kChunks + c;
        bf16_t* const bufs[4] = {xs0, xs1, xs2, xs3};
        xdma(xchunk(s + 2), bufs[(d + 2) & 3]);  // read at stage s - 2, before the last barrier
        __builtin_amdgcn_sched_barrier(0);
        // This stage's weight chunk (loaded during stage s - 2) is in: the loads issued after it are stage
        // s - 1's and this stage's token rows and stage s - 1's weights.
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kXBlocksPerWave + 4));
        // Lane (n, h)'s fragment of token tile tt, k16 step kk: X[32 tt + n][64 c + 16 kk + 8h, +8) at element
        // (4 tt + 2 (n / 16)) * 512 + (kk / 2) * 512 + (16 (2 (kk % 2) + h) + r) * 8 of the buffer.
        const uint32_t xb = (uint32_t)(uintptr_t)bufs[d & 3] + 2048 * (n >> 4) + 16 * (16 * h + r);
        if (active) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            u32x4 xf[TT];
            lds_fragments<TT>(xf, xb + 1024 * (kk >> 1) + 512 * (kk & 1));
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) acc[tt] = mfma_32x32x16(ring[d % kWideDepth][kk], xf[tt], acc[tt]);
          }
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) ring[d % kWideDepth][kk] = wfrag(s + kWideDepth, kk);
        __builtin_amdgcn_sched_barrier(0);
        // The only LDS data that crosses waves in the loop is what the token-row loads write, and the
        // count above covers it; a barrier with fences (or __syncthreads) would also wait for every
        // weight load in flight.  The memory clobber keeps LDS reads on their side of the barrier.
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(4 + (kXBlocksPerWave + 4)));  // a wait the compiler can count on
        asm volatile("s_barrier" ::: "memory");
      }
    }
    // Group epilogue: vocab tile vt of this wave; lane (n, h) holds logits of vocab rows
    // 32 vt + 8 (e / 4) + 4h + e % 4 for token 32 tt + n.
    const int64_t vt = lo + gi * kWideWaves + wave;
    if (vt < hi) {  // wave-uniform
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const int tok = 32 * tt + n;
        uint64_t best = 0;
#pragma unroll
        for (int m4 = 0; m4 < 4; ++m4) {
          const int64_t col0 = 32 * vt + 8 * m4 + 4 * h;
          uint32_t b16[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            b16[j] = f2bf(acc[tt][4 * m4 + j]);
            if (col0 + j < N) {
              const uint64_t key = argmax_key(b16[j] << 16, (uint32_t)(col0 + j));
              best = key > best ? key : best;
            }
          }
          if (logits && tok < M) {
            bf16_t* dst = logits + (int64_t)tok * ldl + col0;
            if (col0 + 3 < N) {
              *reinterpret_cast<u32x2*>(dst) = u32x2{b16[0] | (b16[1] << 16), b16[2] | (b16[3] << 16)};
            } else {
              for (int j = 0; j < 4; ++j)
                if (col0 + j < N) dst[j] = (bf16_t)b16[j];
            }
          }
        }
        const uint64_t o = shfl_xor_u64(best, 32);
        best = o > best ? o : best;
        if (h == 0 && best > wave_best[wave][tok]) wave_best[wave][tok] = best;
      }
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[tt][e] = 0.f;
  }
  __syncthreads();

  if (tid < M) {
    uint64_t b = 0;
#pragma unroll
    for (int wv = 0; wv < kWideWaves; ++wv) b = wave_best[wv][tid] > b ? wave_best[wv][tid] : b;
    best_out[(int64_t)blockIdx.x * M + tid] = b;
  }
}

// Workspace of the wide path: per-workgroup keys (at most kWideMaxGrid workgroups), then the packed token
// rows (hidden size at most 2048).
size_t wide_x_offset(int64_t m) { return ((size_t)kWideMaxGrid * (size_t)m * sizeof(uint64_t) + 255) / 256 * 256; }
size_t wide_workspace_bytes(int64_t m) { return wide_x_offset(m) + (size_t)((m + 15) / 16 * 16) * 2048 * sizeof(bf16_t); }

// Row counts and hidden sizes the wide LM head takes (packed weight only).
bool lm_head_wide_supported(int64_t m, int64_t k, bool packed) {
  return packed && m > 32 && m <= kWideMaxRows && (k == 512 || k == 1024 || k == 2048);
}

template <int TT>
int launch_lm_head_wide_tt(const bf16_t* xp, int M, const bf16_t* w, int64_t K, int64_t N, bf16_t* logits,
                           uint64_t* best, int grid, hipStream_t s) {
  const dim3 g((unsigned)grid), b(64 * kWideWaves);
  switch (K) {
    case 512: hipLaunchKernelGGL((lm_head_wide_kernel<512, TT>), g, b, 0, s, xp, M, w, N, logits, N, best); break;
    case 1024: hipLaunchKernelGGL((lm_head_wide_kernel<1024, TT>), g, b, 0, s, xp, M, w, N, logits, N, best); break;
    case 2048: hipLaunchKernelGGL((lm_head_wide_kernel<2048, TT>), g, b, 0, s, xp, M, w, N, logits, N, best); break;
    default: return OXR_ERR_UNSUPPORTED;
  }
  return OXR_LAUNCH_STATUS();
}

int launch_lm_head_wide(const bf16_t* xp, int M, const bf16_t* w, int64_t K, int64_t N, bf16_t* logits,
                        uint64_t* best, int grid, hipStream_t s) {
  if (M <= 64) return launch_lm_head_wide_tt<2>(xp, M, w, K, N, logits, best, grid, s);
  if (M <= 128) return launch_lm_head_wide_tt<4>(xp, M, w, K, N, logits, best, grid, s);
  return launch_lm_head_wide_tt<8>(xp, M, w, K, N, logits, best, grid, s);
}

// Compute units of the current device (one persistent LM-head workgroup each).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int NB, int K, bool PW>
int launch_lm_head_lds(const bf16_t* x, int64_t ldx, int M, const bf16_t* w, int64_t N, bf16_t* logits,
                       uint64_t* best, int grid, hipStream_t s) {
  constexpr size_t lds = (size_t)NB * 16 * K * sizeof(bf16_t);
  static bool attr_set = false;  // per instantiation; setting it twice is harmless
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute((const void*)lm_head_lds_kernel<NB, K, PW>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    attr_set = true;
  }
  hipLaunchKernelGGL((lm_head_lds_kernel<NB, K, PW>), dim3((unsigned)grid), dim3(64 * kLmWaves), lds, s, x, ldx, M, w,
                     N, logits, N, best);
  return OXR_LAUNCH_STATUS();
}

// Hidden sizes with a persistent LM-head instantiation (X of up to 32 rows fits LDS).
bool lm_head_lds_supported(int64_t m, int64_t k) { return m <= 32 && (k == 512 || k == 1024 || k == 2048); }

template <int NB, bool PW>
int launch_lm_head_lds_k(const bf16_t* x, int64_t ldx, int M, const bf16_t* w, int64_t K, int64_t N, bf16_t* logits,
                         uint64_t* best, int grid, hipStream_t s) {
  switch (K) {
    case 512: return launch_lm_head_lds<NB, 512, PW>(x, ldx, M, w, N, logits, best, grid, s);
    case 1024: return launch_lm_head_lds<NB, 1024, PW>(x, ldx, M, w, N, logits, best, grid, s);
    case 2048: return launch_lm_head_lds<NB, 2048, PW>(x, ldx, M, w, N, logits, best, grid, s);
    default: return OXR_ERR_UNSUPPORTED;
  }
}

struct LaunchConfig {
  int na;        // 16-row tiles per workgroup
  int waves;     // waves per workgroup, each a k sub-slice
  int k_splits;  // k slices across workgroups (kPartial only)
};

template <int NA, int NB, int EPI, int WAVES, bool PW, bool PX>
int launch_gemm(const GemmArgs& a, const LaunchConfig& c, hipStream_t s) {
  const int64_t tiles = (a.N + 16 * NA - 1) / (16 * NA);
  hipLaunchKernelGGL((gemm_kernel<NA, NB, EPI, WAVES, PW, PX>), dim3((unsigned)tiles, (unsigned)c.k_splits),
                     dim3(64 * WAVES), 0, s, a);
  return OXR_LAUNCH_STATUS();
}

template <int NA, int EPI, int WAVES, bool PW, bool PX>
int dispatch_nb(const GemmArgs& a, const LaunchConfig& c, hipStream_t s) {
  switch ((a.M + 15) / 16) {
    case 1: return launch_gemm<NA, 1, EPI, WAVES, PW, PX>(a, c, s);
    case 2: return launch_gemm<NA, 2, EPI, WAVES, PW, PX>(a, c, s);
    case 3: return launch_gemm<NA, 3, EPI, WAVES, PW, PX>(a, c, s);
    case 4: return launch_gemm<NA, 4, EPI, WAVES, PW, PX>(a, c, s);
    default: return OXR_ERR_UNSUPPORTED;
  }
}

template <int NA, int EPI, bool PW, bool PX>
int dispatch_waves(const GemmArgs& a, const LaunchConfig& c, hipStream_t s) {
  switch (c.waves) {
    case 1: return dispatch_nb<NA, EPI, 1, PW, PX>(a, c, s);
    case 2: return dispatch_nb<NA, EPI, 2, PW, PX>(a, c, s);
    case 4: return dispatch_nb<NA, EPI, 4, PW, PX>(a, c, s);
    default: return OXR_ERR_UNSUPPORTED;
  }
}

// Operand layouts: row-major weight and X; packed weight, row-major X; both
// packed (the verify forward's own path; the LM head stages X itself).
enum Layout { kRowMajor = 0, kPackedW = 1, kPackedWX = 2 };

template <int EPI>
int dispatch(const GemmArgs& a, const LaunchConfig& c, Layout layout, hipStream_t s) {
  if (EPI == kArgmax && layout == kPackedWX) return OXR_ERR_UNSUPPORTED;
  switch (c.na * 4 + (int)layout) {
    case 4: return dispatch_waves<1, EPI, false, false>(a, c, s);
    case 5: return dispatch_waves<1, EPI, true, false>(a, c, s);
    case 6: return dispatch_waves<1, EPI, true, EPI != kArgmax>(a, c, s);
    case 8: return dispatch_waves<2, EPI, false, false>(a, c, s);
    case 9: return dispatch_waves<2, EPI, true, false>(a, c, s);
    case 10: return dispatch_waves<2, EPI, true, EPI != kArgmax>(a, c, s);
    default: return OXR_ERR_UNSUPPORTED;
  }
}

// Launch shape, from a sweep of the verify shapes on MI355X (M = 32, packed
// and row-major weights alike): 32-row tiles, or 16-row tiles when fewer than
// 160 workgroups of 32 rows would remain (qkv); weights with fp32-partial
// output (o_proj, down_proj: 2048 columns) split k until there are >= 256
// workgroups; a workgroup's k slice goes to the fewest waves that leave each
// at most 8 steps of 128 (o_proj: 1 wave; qkv, gate_up, down_proj: 2).  More
// waves per workgroup only add requests in flight to an already saturated
// memory pipeline (4 waves: gate_up 18.1 vs 15.7 us, down_proj 9.9 vs 8.5).
constexpr int kWaveSteps = 8;            // most 128-k steps per wave before a GEMM adds waves
constexpr int kNa2Tiles = 160;           // 32-row tiles from which a whole-K GEMM takes two tiles per workgroup
constexpr int kTargetWorkgroups = 256;   // workgroups a k-split GEMM aims for
LaunchConfig choose_config(int64_t n_rows, int64_t K, bool allow_k_splits) {
  LaunchConfig c{1, 1, 1};
  if (allow_k_splits) {
    c.na = 2;
    const int64_t tiles = (n_rows + 31) / 32;
    while (tiles * c.k_splits < kTargetWorkgroups && K % (2 * c.k_splits * kKStep) == 0 && c.k_splits < 16)
      c.k_splits *= 2;
  } else {
    c.na = (n_rows + 31) / 32 >= kNa2Tiles ? 2 : 1;
  }
  const int64_t k_slice = K / c.k_splits;
  // At most 4 waves: an 8-wave workgroup has 256 registers per wave, and its 3- and 4-tile token
  // forms spill (up to 1.1 KiB per lane).
  while (k_slice / c.waves > kWaveSteps * kKStep && k_slice % (2 * c.waves * kKStep) == 0 && c.waves < 4)
    c.waves *= 2;
  return c;
}

// Token rows one launch of gemm_kernel takes (4 tiles of 16); the entry points take up to kMaxRows
// and run one launch per 64 rows over the same weight.  The first launch streams the weight from
// HBM; it is at most a few tens of MB, so the later ones find it in the 256 MB Infinity Cache.
constexpr int64_t kPassRows = 64;
constexpr int64_t kMaxRows = 256;

int check_common(const void* x, int64_t ldx, int64_t M, const void* w, int64_t K, int64_t N) {
  OXR_RETURN_IF(M < 0 || K <= 0 || N <= 0 || ldx < K, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(M > kMaxRows || K % kKStep != 0, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(M > 0 && (!x || !w), OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(((uintptr_t)x | (uintptr_t)w) % 16 != 0 || ldx % 8 != 0, OXR_ERR_UNSUPPORTED);
  return OXR_OK;
}

// Packed layout (see the top of this file): one thread per 16-byte fragment
// of the output, in output order; rows past `rows` (the last tile's padding)
// are zero.
__global__ __launch_bounds__(256) void pack_weight_kernel(const bf16_t* __restrict__ w, int64_t rows, int64_t K,
                                                          int64_t chunks, bf16_t* __restrict__ packed) {
  const int64_t ksteps = K / kKStep;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(c & 63), r = lane & 15, g = lane >> 4;
    const int64_t blk = c >> 6;
    const int i = (int)(blk & 3);
    const int64_t q = (blk >> 2) % ksteps, t = (blk >> 2) / ksteps;
    const int64_t row = 16 * t + r;
    const u32x4 v = row < rows ? ld128(w + row * K + q * kKStep + 32 * i + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(packed + c * 8) = v;
  }
}

// flags: OXR_GEMM_X_PACKED (x packed; ldx unused), OXR_GEMM_Y_PACKED (y packed
// with row length n; ldy unused; kStore / kSiluMul).  Row-major weights take
// neither.
int gemm_entry(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w, int64_t k, int64_t n, int32_t epilogue,
               oxr_bf16* y, int64_t ldy, bool packed, int32_t flags, oxr_stream_t stream) {
  const bool xp = flags & OXR_GEMM_X_PACKED, yp = flags & OXR_GEMM_Y_PACKED;
  OXR_RETURN_IF((flags & ~(OXR_GEMM_X_PACKED | OXR_GEMM_Y_PACKED)) != 0 || (!packed && flags != 0), OXR_ERR_INVALID_ARG);
  if (xp) ldx = k;
  if (yp) ldy = n;
  int st = check_common(x, ldx, m, w, k, n);
  if (st) return st;
  OXR_RETURN_IF(epilogue != kStore && epilogue != kSiluMul && epilogue != kAddResidual, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(!y || ldy < n || ldy % 4 != 0 || (uintptr_t)y % 8 != 0, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(packed && epilogue == kSiluMul && n % 16 != 0, OXR_ERR_UNSUPPORTED);  // up rows start a tile
  OXR_RETURN_IF(yp && (epilogue == kAddResidual || n % kKStep != 0), OXR_ERR_UNSUPPORTED);
  if (m == 0) return OXR_OK;
  hipStream_t s = (hipStream_t)stream;
  const LaunchConfig c = choose_config(n, k, false);
  const Layout layout = !packed ? kRowMajor : (xp ? kPackedWX : kPackedW);
  for (int64_t r0 = 0; r0 < m; r0 += kPassRows) {
    // Rows [r0, r0 + 64): a packed operand's rows start r0 * row_length elements in (r0 is a
    // multiple of 16, a whole number of tiles).
    GemmArgs a{x + (xp ? r0 * k : r0 * ldx), ldx, (int)std::min(kPassRows, m - r0), w, k, n,
               y + (yp ? r0 * n : r0 * ldy), ldy, yp ? 1 : 0, nullptr, nullptr, 0};
    const int st = epilogue == kSiluMul       ? dispatch<kSiluMul>(a, c, layout, s)
                   : epilogue == kAddResidual ? dispatch<kAddResidual>(a, c, layout, s)
                                              : dispatch<kStore>(a, c, layout, s);
    if (st) return st;
  }
  return OXR_OK;
}

int gemm_partial_entry(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w, int64_t k, int64_t n,
                       float* partials, int32_t k_splits, bool packed, int32_t flags, oxr_stream_t stream) {
  OXR_RETURN_IF((flags & ~OXR_GEMM_X_PACKED) != 0 || (!packed && flags != 0), OXR_ERR_INVALID_ARG);
  const bool xp = flags & OXR_GEMM_X_PACKED;
  if (xp) ldx = k;
  int st = check_common(x, ldx, m, w, k, n);
  if (st) return st;
  OXR_RETURN_IF(!partials || (uintptr_t)partials % 16 != 0 || n % 4 != 0, OXR_ERR_INVALID_ARG);
  const LaunchConfig c = choose_config(n, k, true);
  OXR_RETURN_IF(k_splits != c.k_splits, OXR_ERR_INVALID_ARG);
  if (m == 0) return OXR_OK;
  for (int64_t r0 = 0; r0 < m; r0 += kPassRows) {
    GemmArgs a{x + (xp ? r0 * k : r0 * ldx), ldx, (int)std::min(kPassRows, m - r0), w, k, n, nullptr, 0, 0, nullptr,
               partials + r0 * n, m};
    const int st = dispatch<kPartial>(a, c, !packed ? kRowMajor : (xp ? kPackedWX : kPackedW), (hipStream_t)stream);
    if (st) return st;
  }
  return OXR_OK;
}

int lm_head_keys_impl(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight, int64_t hidden_size, int64_t vocab,
                      oxr_bf16* logits, void* workspace, size_t workspace_bytes, bool packed, hipStream_t s,
                      const uint64_t** best_out, int* num_best_out) {
  *num_best_out = 0;
  // More than 64 rows only on the wide path (packed weight, up to 256 rows); the common checks see at most 64.
  OXR_RETURN_IF(m > 64 && !lm_head_wide_supported(m, hidden_size, packed), OXR_ERR_UNSUPPORTED);
  int st = check_common(hidden, hidden_size, std::min<int64_t>(m, 64), weight, hidden_size, vocab);
  if (st) return st;
  OXR_RETURN_IF(logits && (uintptr_t)logits % 8 != 0, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(vocab > 0x7fffffffLL, OXR_ERR_UNSUPPORTED);
  if (m == 0) return OXR_OK;
  const size_t need = oxr_lm_head_workspace_bytes(m, vocab);
  OXR_RETURN_IF(!workspace || workspace_bytes < need, OXR_ERR_WORKSPACE);
  uint64_t* best = static_cast<uint64_t*>(workspace);
  int num_best;  // partial maxima per token for the final reduction
  if (lm_head_wide_supported(m, hidden_size, packed)) {
    // Token rows packed into the workspace (after the per-workgroup keys), then the wide kernel.
    const int64_t nt32 = (vocab + 31) / 32;
    num_best = (int)std::min<int64_t>(std::min(device_cus(), kWideMaxGrid), nt32);
    bf16_t* xp = reinterpret_cast<bf16_t*>(static_cast<char*>(workspace) + wide_x_offset(m));
    const int64_t chunks = (int64_t)oxr_packed_weight_elems(m, hidden_size) / 8;
    hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)std::min<int64_t>((chunks + 255) / 256, 4096)), dim3(256),
                       0, s, hidden, m, hidden_size, chunks, xp);
    st = OXR_LAUNCH_STATUS();
    if (!st) st = launch_lm_head_wide(xp, (int)m, weight, hidden_size, vocab, logits, best, num_best, s);
  } else if (lm_head_lds_supported(m, hidden_size)) {
    const int64_t num_tiles = (vocab + 15) / 16;
    num_best = (int)std::min<int64_t>(device_cus(), num_tiles);
    const int key = (m <= 16 ? 0 : 2) + (packed ? 1 : 0);
    st = key == 0   ? launch_lm_head_lds_k<1, false>(hidden, hidden_size, (int)m, weight, hidden_size, vocab, logits,
                                                     best, num_best, s)
         : key == 1 ? launch_lm_head_lds_k<1, true>(hidden, hidden_size, (int)m, weight, hidden_size, vocab, logits,
                                                    best, num_best, s)
         : key == 2 ? launch_lm_head_lds_k<2, false>(hidden, hidden_size, (int)m, weight, hidden_size, vocab, logits,
                                                     best, num_best, s)
                    : launch_lm_head_lds_k<2, true>(hidden, hidden_size, (int)m, weight, hidden_size, vocab, logits,
                                                    best, num_best, s);
  } else {
    GemmArgs a{hidden, hidden_size, (int)m, weight, hidden_size, vocab, logits, vocab, 0, best, nullptr, 0};
    const LaunchConfig c = choose_config(vocab, hidden_size, false);
    num_best = (int)((vocab + 16 * c.na - 1) / (16 * c.na));
    st = dispatch<kArgmax>(a, c, packed ? kPackedW : kRowMajor, s);
  }
  if (st) return st;
  *best_out = best;
  *num_best_out = num_best;
  return OXR_OK;
}

int lm_head_entry(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight, int64_t hidden_size, int64_t vocab,
                  oxr_bf16* logits, int64_t* predicted, void* workspace, size_t workspace_bytes, bool packed,
                  oxr_stream_t stream) {
  hipStream_t s = (hipStream_t)stream;
  // Checked in the order of the key launch's own checks, with predicted after the operands.
  OXR_RETURN_IF(m > 64 && !lm_head_wide_supported(m, hidden_size, packed), OXR_ERR_UNSUPPORTED);
  const int common = check_common(hidden, hidden_size, std::min<int64_t>(m, 64), weight, hidden_size, vocab);
  if (common) return common;
  OXR_RETURN_IF(!predicted, OXR_ERR_INVALID_ARG);
  const uint64_t* best = nullptr;
  int num_best = 0;
  const int st = lm_head_keys_impl(hidden, m, weight, hidden_size, vocab, logits, workspace, workspace_bytes, packed,
                                   s, &best, &num_best);
  if (st || m == 0) return st;
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3((unsigned)m), dim3(256), 0, s, best, num_best, (int)m, predicted);
  return OXR_LAUNCH_STATUS();
}

}  // namespace

int lm_head_keys(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight, int64_t hidden_size, int64_t vocab,
                 oxr_bf16* logits, void* workspace, size_t workspace_bytes, bool packed, hipStream_t stream,
                 const uint64_t** best, int* num_best) {
  return lm_head_keys_impl(hidden, m, weight, hidden_size, vocab, logits, workspace, workspace_bytes, packed, stream,
                           best, num_best);
}
}  // namespace oxr

extern "C" size_t oxr_packed_weight_elems(int64_t rows, int64_t k) {
  if (rows <= 0 || k <= 0) return 0;
  return (size_t)((rows + 15) / 16 * 16) * (size_t)k;
}

extern "C" int oxr_pack_weight_bf16(const oxr_bf16* w, int64_t rows, int64_t k, oxr_bf16* packed,
                                    oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(rows <= 0 || k <= 0 || !w || !packed, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(k % kKStep != 0 || ((uintptr_t)w | (uintptr_t)packed) % 16 != 0, OXR_ERR_UNSUPPORTED);
  const int64_t elems = (int64_t)oxr_packed_weight_elems(rows, k);
  const uintptr_t wb = (uintptr_t)w, pb = (uintptr_t)packed;
  OXR_RETURN_IF(wb < pb + 2 * (uintptr_t)elems && pb < wb + 2 * (uintptr_t)(rows * k), OXR_ERR_INVALID_ARG);  // overlap
  const int64_t chunks = elems / 8;
  const int64_t blocks = std::min<int64_t>((chunks + 255) / 256, 4096);
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, w, rows, k, chunks,
                     packed);
  return OXR_LAUNCH_STATUS();
}

extern "C" int oxr_gemm_bf16(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w, int64_t k, int64_t n,
                             int32_t epilogue, oxr_bf16* y, int64_t ldy, oxr_stream_t stream) {
  return oxr::gemm_entry(x, ldx, m, w, k, n, epilogue, y, ldy, false, 0, stream);
}

extern "C" int oxr_gemm_bf16_packed(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w_packed, int64_t k,
                                    int64_t n, int32_t epilogue, oxr_bf16* y, int64_t ldy, int32_t flags,
                                    oxr_stream_t stream) {
  return oxr::gemm_entry(x, ldx, m, w_packed, k, n, epilogue, y, ldy, true, flags, stream);
}

extern "C" int32_t oxr_gemm_bf16_partial_splits(int64_t n, int64_t k) {
  return oxr::choose_config(n, k, true).k_splits;
}

extern "C" int oxr_gemm_bf16_partial(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w, int64_t k,
                                     int64_t n, float* partials, int32_t k_splits, oxr_stream_t stream) {
  return oxr::gemm_partial_entry(x, ldx, m, w, k, n, partials, k_splits, false, 0, stream);
}

extern "C" int oxr_gemm_bf16_partial_packed(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w_packed,
                                            int64_t k, int64_t n, float* partials, int32_t k_splits, int32_t flags,
                                            oxr_stream_t stream) {
  return oxr::gemm_partial_entry(x, ldx, m, w_packed, k, n, partials, k_splits, true, flags, stream);
}

extern "C" size_t oxr_lm_head_workspace_bytes(int64_t m, int64_t vocab) {
  if (m <= 0 || vocab <= 0) return 0;
  const size_t tiles = (size_t)((vocab + 15) / 16) * (size_t)m * sizeof(uint64_t);  // enough for 16-row tiles
  return m > 32 ? std::max(tiles, oxr::wide_workspace_bytes(m)) : tiles;
}

extern "C" int oxr_lm_head_argmax(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight, int64_t hidden_size,
                                  int64_t vocab, oxr_bf16* logits, int64_t* predicted, void* workspace,
                                  size_t workspace_bytes, oxr_stream_t stream) {
  return oxr::lm_head_entry(hidden, m, weight, hidden_size, vocab, logits, predicted, workspace, workspace_bytes, false,
                            stream);
}

extern "C" int oxr_lm_head_argmax_packed(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight_packed,
                                         int64_t hidden_size, int64_t vocab, oxr_bf16* logits, int64_t* predicted,
                                         void* workspace, size_t workspace_bytes, oxr_stream_t stream) {
  return oxr::lm_head_entry(hidden, m, weight_packed, hidden_size, vocab, logits, predicted, workspace,
                            workspace_bytes, true, stream);
}

extern "C" size_t oxr_argmax_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return (size_t)oxr::argmax_chunks(rows, vocab) * (size_t)rows * sizeof(uint64_t);
}

extern "C" int oxr_argmax(const void* logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t ld,
                          int64_t* predicted, void* workspace, size_t workspace_bytes, oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(rows < 0 || vocab <= 0 || ld < vocab, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(dtype != OXR_DTYPE_F32 && dtype != OXR_DTYPE_BF16, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(rows > 65535 || vocab > 0x7fffffffLL, OXR_ERR_UNSUPPORTED);
  if (rows == 0) return OXR_OK;
  OXR_RETURN_IF(!logits || !predicted, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(!workspace || workspace_bytes < oxr_argmax_workspace_bytes(rows, vocab), OXR_ERR_WORKSPACE);
  hipStream_t s = (hipStream_t)stream;
  const int chunks = argmax_chunks(rows, vocab);
  uint64_t* best = static_cast<uint64_t*>(workspace);
  const dim3 grid((unsigned)chunks, (unsigned)rows), block(256);
  const size_t elem = dtype == OXR_DTYPE_F32 ? 4 : 2;
  const bool vec = ((uintptr_t)logits % 16 == 0) && ((size_t)ld * elem) % 16 == 0;
  if (dtype == OXR_DTYPE_F32) {
    const float* p = static_cast<const float*>(logits);
    if (vec) hipLaunchKernelGGL((argmax_rows_kernel<float, true>), grid, block, 0, s, p, ld, vocab, (int)rows, best);
    else hipLaunchKernelGGL((argmax_rows_kernel<float, false>), grid, block, 0, s, p, ld, vocab, (int)rows, best);
  } else {
    const bf16_t* p = static_cast<const bf16_t*>(logits);
    if (vec) hipLaunchKernelGGL((argmax_rows_kernel<bf16_t, true>), grid, block, 0, s, p, ld, vocab, (int)rows, best);
    else hipLaunchKernelGGL((argmax_rows_kernel<bf16_t, false>), grid, block, 0, s, p, ld, vocab, (int)rows, best);
  }
  int st = OXR_LAUNCH_STATUS();
  if (st) return st;
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3((unsigned)rows), dim3(256), 0, s, static_cast<const uint64_t*>(best),
                     chunks, (int)rows, predicted);
  return OXR_LAUNCH_STATUS();
}
