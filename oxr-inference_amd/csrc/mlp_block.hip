// A decoder layer's MLP block in one launch, for the verify step's few token rows (gfx950).
//
// DecoderLayer._mlp (oxr_runtime/language.py:266-269) for T <= 32 token rows:
//   residual' = bf16(bf16(o_proj(attn)) + residual)             (_add_rms_norm, language.py:94-99)
//   h         = bf16(w * bf16(residual' / rms(residual')))        (_rms_norm, language.py:69-72)
//   act       = bf16(bf16(silu(bf16(h gate^T))) * bf16(h up^T))   (_silu_mul, language.py:102-104)
//   out       = act down^T, as 8 fp32 partial sums over slices of the intermediate dimension
// o_proj's output arrives as the fp32 k-split partials of its GEMM (summed here exactly as the
// add + RMSNorm launch of csrc/norm.hip sums them); the block's output leaves as partials that the
// next norm sums.  As three launches (norm, gate_up with the SiLU epilogue, down) the block pays
// three ramps and drains around 77 MB of weights; here the weight stream starts at the first
// instruction and runs through every dependency of the block.
//
// Partition.  Each of the 8 XCDs owns one eighth of the intermediate dimension (768 of 6144
// columns): the gate/up rows of those columns and the down_proj columns that read them.  Every
// dependency inside the block then stays inside one XCD, whose 32 workgroups (one per CU) hand data
// to each other through that XCD's L2:
//   1. norm: workgroup r normalises token row r into the XCD's own copy of h (all 8 XCDs compute
//      every row; XCD r % 8 writes the new residual row, to a buffer nobody reads in this launch),
//   2. XCD barrier; the XCD's h (T x 2048, packed) is copied into LDS,
//   3. gate/up: workgroup r multiplies the 48 gate_up rows of intermediate columns [24 g, 24 g + 24),
//      g = 32 x + r: three 16-row tiles of the 8-row-interleaved weight (tile j = gate rows
//      8j..8j+7, then up rows 8j..8j+7), so it applies silu * up to its own columns,
//   4. its 24 act columns go to the XCD's act buffer; XCD barrier; act (T x 768) into LDS,
//   5. down: workgroup r multiplies down_proj rows [64 r, 64 r + 64) by the XCD's 768 columns of act
//      and stores fp32 partial slice x.
// Placement, counters and waits: csrc/xcd_sync.h (the XCD from the hardware, rank blockIdx.x / 8, a
// census that reports a placement breaking this, bounded waits that end with an error bit).
//
// Waves.  Four worker waves stream weights and multiply; a fifth, the helper, does everything that
// waits on other workgroups (the stores that feed them, the XCD barriers, the copies into LDS).  The
// vector memory counter is in order, so a wave that waited for a flag or a store would first wait for
// every weight load it had issued; the helper has none in flight, and the workers meet it only at
// s_barrier, which waits for no memory counter.  Worker w streams, for each gate/up tile, the 128-k
// steps [4w, 4w + 4) (a K quarter: the four quarters are summed in LDS in wave order), then
// down_proj row tile 4r + w over the XCD's six 128-k steps, through a register ring of kRing steps;
// the down_proj weights are all in flight before the gate/up products end.
// Order of requests.  A CU's vector memory path returns in order and a wave that issues many loads
// stalls on the CU's outstanding-miss limit until earlier ones return (measured: 32 loads per wave
// took ~3 us to issue at the start of the block).  So the block requests what its critical path needs
// first -- the norm's inputs, the helper's stores of the normalised row, the copy of h into LDS -- and
// the workers issue the weight ring only once the helper has requested that copy.  Requesting the
// ring earlier (before or right after the norm) delayed the norm's stores or the copy behind it by
// 3-5 us and made the block no faster.
#include "xcd_sync.h"

namespace oxr {
namespace {

using namespace xcd;

constexpr int kWorkers = 4;
constexpr int kThreads = 64 * (kWorkers + 1);
constexpr int kMaxRows = 32;
constexpr int kRing = 8;  // 128-k weight steps in flight per worker wave (4 KiB each)

// Block shape: the config-5 decoder (hidden 2048, intermediate 6144).
constexpr int kH = 2048, kI = 6144;
constexpr int kIx = kI / kXcds;                 // intermediate columns per XCD (768)
constexpr int kIw = kIx / kXcdWgs;              // per workgroup (24)
constexpr int kGTiles = kIw / 8;                // interleaved gate/up tiles per workgroup (3)
constexpr int kGq = kH / 128 / kWorkers;        // 128-k steps of a gate/up tile per worker (4)
constexpr int kGSteps = kGTiles * kGq;          // 12
constexpr int kDSteps = kIx / 128;              // 6
constexpr int kSteps = kGSteps + kDSteps;       // 18
static_assert(kH / 16 / kXcdWgs == kWorkers, "one down_proj row tile per worker");
static_assert(kIw % 8 == 0 && kIx % 128 == 0 && kH % (128 * kWorkers) == 0, "block shape");

enum MlpCtl { kNormDone = kPhase0, kActDone = kPhase1 };
constexpr size_t kHElems = (size_t)kMaxRows * kH;      // one XCD's copy of h, packed
constexpr size_t kActElems = (size_t)kMaxRows * kIx;   // one XCD's act slice, packed
constexpr size_t kWorkspaceBytes = kCtlBytes + kXcds * (kHElems + kActElems) * sizeof(bf16_t);

struct MlpArgs {
  const float* o_part;    // [o_splits][rows][kH]
  int o_splits;
  int rows;
  const bf16_t* res_in;   // [rows][kH]
  bf16_t* res_out;        // [rows][kH]
  const bf16_t* norm_w;   // [kH]
  float eps;
  const bf16_t* gate_up;  // [2 kI][kH], rows 8-interleaved, packed
  const bf16_t* down;     // [kH][kI], packed
  float* d_part;          // [kXcds][rows][kH]
  uint32_t* ctl;
  bf16_t* h_x;            // [kXcds][kHElems]
  bf16_t* act_x;          // [kXcds][kActElems]
};

template <int NB, int P>
__global__ __launch_bounds__(kThreads) void mlp_block_kernel(MlpArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t lx[NB * 16 * kH];   // h, then act: the products' x
  // Gate/up K-quarter sums; before the products, the norm output and new residual row (row_stage).
  __shared__ f32x4 red[kWorkers][kGTiles][NB][64];
  static_assert(sizeof(red) >= 2 * kH / 8 * sizeof(u32x4), "row_stage fits in red");
  u32x4(&row_stage)[2][kH / 8] = *reinterpret_cast<u32x4(*)[2][kH / 8]>(&red[0][0][0][0]);
  __shared__ u32x2 act_stage[NB * 16][kGTiles][2];                    // act of this workgroup's columns
  __shared__ float wave_ss[kWorkers];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rank = blockIdx.x >> 3;
  const uint32_t xcc = xcc_id();
  const int x = (int)(xcc & 7u);
  uint32_t* const ctl = a.ctl + x * kCtlStride;
  bf16_t* const h_x = a.h_x + x * kHElems;
  bf16_t* const act_x = a.act_x + x * kActElems;
  const int rows = a.rows;
  const bool has_row = rank < rows;

  if (wave == kWorkers) {
    // ---------------------------------------------------------------- helper wave
    census(a.ctl, ctl, rank, xcc, lane);
    barrier();  // S1: the workers' norm sums
    barrier();  // S2: the norm row in LDS
    if (has_row) {
#pragma unroll
      for (int j = 0; j < kH / 8 / 64; ++j) {
        const int c = lane + 64 * j;
        st128(h_x + packed_offset(rank, 8 * c, kH), row_stage[0][c]);
        if ((rank & 7) == x) st128(a.res_out + (int64_t)rank * kH + 8 * c, row_stage[1][c]);
      }
      stores_done();
      arrive(ctl + kNormDone, lane);
    }
    if (!wait_count(ctl + kNormDone, (uint32_t)rows) && lane == 0) set_error(a.ctl, kErrPhase0Wait);
    copy_to_lds(h_x, lx, NB * 16 * kH / 512, lane);
    barrier();  // S3: copy requested
    stores_done();
    barrier();  // S4: h in LDS
    barrier();  // S5: gate/up K-quarter sums in LDS
    barrier();  // S6: act columns in LDS
    for (int e = lane; e < NB * 16 * kGTiles; e += 64) {
      const int tok = e / kGTiles, m = e % kGTiles;
      const u32x2 lo = act_stage[tok][m][0], hi = act_stage[tok][m][1];
      st128(act_x + packed_offset(tok, kIw * rank + 8 * m, kIx), u32x4{lo.x, lo.y, hi.x, hi.y});
    }
    stores_done();
    arrive(ctl + kActDone, lane);
    if (!wait_count(ctl + kActDone, (uint32_t)kXcdWgs) && lane == 0) set_error(a.ctl, kErrPhase1Wait);
    copy_to_lds(act_x, lx, NB * 16 * kIx / 512, lane);
    stores_done();
    barrier();  // S7: act in LDS
    finish(ctl, lane);
    return;
  }

  // ------------------------------------------------------------------ worker waves
  const int w = wave;
  const int gidx = kXcdWgs * x + rank;
  const bf16_t* const gu = a.gate_up + (int64_t)kGTiles * gidx * (16 * kH) + lane * 8;
  const int dtile = kWorkers * rank + w;
  const bf16_t* const dw = a.down + (int64_t)dtile * (16 * kI) + (int64_t)kDSteps * x * 2048 + lane * 8;

  // Norm inputs first (thread c: columns [8c, 8c + 8), as the add + RMSNorm launch maps them), so
  // that waiting for them never waits for a weight load.  Workgroups without a row read row 0.
  const int c = threadIdx.x, col = 8 * c;
  const int row = has_row ? rank : 0;
  const u32x4 wt = ld128(a.norm_w + col);
  u32x4 v = ld128(a.res_in + (int64_t)row * kH + col);
  f32x4 pl[P], ph[P];
#pragma unroll
  for (int sp = 0; sp < P; ++sp) {
    const float* p = a.o_part + ((int64_t)sp * rows + row) * kH + col;
    pl[sp] = *reinterpret_cast<const f32x4*>(p);
    ph[sp] = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __builtin_amdgcn_sched_barrier(0);

  u32x4 ring[kRing][4];
  auto load_step = [&](int s, u32x4 (&dst)[4]) {
    const bf16_t* base = s < kGSteps ? gu + (int64_t)(s / kGq) * (16 * kH) + (kGq * w + s % kGq) * 2048
                                     : dw + (s - kGSteps) * 2048;
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = ld128_nt(base + i * 512);
  };

  // residual' = bf16(bf16(sum of partials) + residual); the sum of squares as rms_norm_kernel forms it.
  {
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < P; ++sp) {
      lo += pl[sp];
      hi += ph[sp];
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
  {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p0 = lo_bf(xd[e]), p1 = hi_bf(xd[e]);
      ss += p0 * p0;
      ss += p1 * p1;
    }
    ss = wave_sum(ss);
    if (lane == 0) wave_ss[w] = ss;
  }
  barrier();  // S1
  {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kWorkers; ++i) ss += wave_ss[i];
    const float r = 1.0f / sqrtf(ss / (float)kH + a.eps);
    const uint32_t wd[4] = {wt.x, wt.y, wt.z, wt.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float y0 = lo_bf(wd[e]) * round_bf16(lo_bf(xd[e]) * r);
      const float y1 = hi_bf(wd[e]) * round_bf16(hi_bf(xd[e]) * r);
      o[e] = pack_bf(y0, y1);
    }
    row_stage[0][c] = u32x4{o[0], o[1], o[2], o[3]};
    row_stage[1][c] = v;
  }
  barrier();  // S2
  barrier();  // S3: the copy of h into LDS is requested
  // The weight ring, behind the helper's requests: the CU's vector memory path returns in order, and
  // issuing 32 loads per wave stalls the wave on its outstanding-miss limit for microseconds, so a
  // store or copy on the block's critical path issued after them would wait as long.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < kRing; ++s) load_step(s, ring[s]);
  __builtin_amdgcn_sched_barrier(0);
  barrier();  // S4: h in LDS

  const int r = lane & 15, g = lane >> 4;
  f32x4 acc[kGTiles][NB];
#pragma unroll
  for (int t = 0; t < kGTiles; ++t)
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) acc[t][bt] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 dacc[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) dacc[bt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    if (s == kGSteps) {
      // Gate/up tiles done: K quarters summed in wave order, silu * up, act columns to the helper.
#pragma unroll
      for (int t = 0; t < kGTiles; ++t)
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) red[w][t][bt][lane] = acc[t][bt];
      barrier();  // S5
      {
        // Wave w finishes element w of every lane's four, for all tiles: lane L takes token tile
        // L / 32 and the gate lane l = L % 32 (tile rows 4 (l / 16) + w for token l % 16; the up row of
        // the same column is at lane l + 32), so all four waves and all their lanes share the work.
        const int bt = lane >> 5, l = lane & 31;
        if (bt < NB) {
          const float* const rf = reinterpret_cast<const float*>(&red[0][0][0][0]);
          uint16_t* const st = reinterpret_cast<uint16_t*>(&act_stage[0][0][0]);
#pragma unroll
          for (int t = 0; t < kGTiles; ++t) {
            auto at = [&](int q, int ln) { return rf[(((q * kGTiles + t) * NB + bt) * 64 + ln) * 4 + w]; };
            float gs = at(0, l), us = at(0, l + 32);
#pragma unroll
            for (int q = 1; q < kWorkers; ++q) {
              gs += at(q, l);
              us += at(q, l + 32);
            }
            const float gv = round_bf16(gs);
            const float sv = round_bf16(gv / (1.0f + expf(-gv)));
            st[((16 * bt + (l & 15)) * kGTiles + t) * 8 + 4 * (l >> 4) + w] = (uint16_t)f2bf(sv * round_bf16(us));
          }
        }
      }
      barrier();  // S6
      barrier();  // S7: act in LDS
    }
    const u32x4(&wf)[4] = ring[s % kRing];
    if (s < kGSteps) {
      const int t = s / kGq, q = kGq * w + s % kGq;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) {
          const u32x4 xf = *reinterpret_cast<const u32x4*>(lx + ((bt * (kH / 128) + q) * 4 + i) * 512 + lane * 8);
          acc[t][bt] = mfma_16x16x32(wf[i], xf, acc[t][bt]);
        }
    } else {
      const int q = s - kGSteps;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) {
          const u32x4 xf = *reinterpret_cast<const u32x4*>(lx + ((bt * kDSteps + q) * 4 + i) * 512 + lane * 8);
          dacc[bt] = mfma_16x16x32(wf[i], xf, dacc[bt]);
        }
    }
    if (s + kRing < kSteps) load_step(s + kRing, ring[s % kRing]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // fp32 partial slice x: lane (r, g) holds down_proj rows 16 dtile + 4g..+3 for token 16 bt + r.
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int tok = 16 * bt + r;
    if (tok < rows)
      *reinterpret_cast<f32x4*>(a.d_part + ((int64_t)x * rows + tok) * kH + 16 * dtile + 4 * g) = dacc[bt];
  }
}

template <int NB>
int launch_nb(const MlpArgs& a, hipStream_t s) {
  if (a.o_splits == 4)
    hipLaunchKernelGGL((mlp_block_kernel<NB, 4>), dim3(kGrid), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((mlp_block_kernel<NB, 8>), dim3(kGrid), dim3(kThreads), 0, s, a);
  return OXR_LAUNCH_STATUS();
}

}  // namespace
}  // namespace oxr

extern "C" size_t oxr_mlp_block_workspace_bytes(void) { return oxr::kWorkspaceBytes; }

extern "C" int oxr_mlp_block_supported(int64_t rows, int64_t hidden, int64_t intermediate, int32_t o_splits) {
  using namespace oxr;
  return rows >= 1 && rows <= kMaxRows && hidden == kH && intermediate == kI && (o_splits == 4 || o_splits == 8) &&
         device_fits();
}

extern "C" int oxr_mlp_block(const float* o_partials, int32_t o_splits, const oxr_bf16* residual_in, int64_t rows,
                             int64_t hidden, int64_t intermediate, const oxr_bf16* post_norm, float eps,
                             const oxr_bf16* gate_up_interleaved, const oxr_bf16* down, oxr_bf16* residual_out,
                             float* partials_out, void* workspace, size_t workspace_bytes, oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(rows < 0 || hidden <= 0 || intermediate <= 0, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(rows > kMaxRows || hidden != kH || intermediate != kI || (o_splits != 4 && o_splits != 8),
                OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(rows > 0 && (!o_partials || !residual_in || !post_norm || !gate_up_interleaved || !down ||
                             !residual_out || !partials_out),
                OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(residual_out == residual_in, OXR_ERR_INVALID_ARG);  // read by every XCD while written
  OXR_RETURN_IF(((uintptr_t)o_partials | (uintptr_t)residual_in | (uintptr_t)residual_out | (uintptr_t)post_norm |
                 (uintptr_t)gate_up_interleaved | (uintptr_t)down | (uintptr_t)partials_out) % 16 != 0,
                OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(!workspace || workspace_bytes < kWorkspaceBytes || (uintptr_t)workspace % 256 != 0,
                OXR_ERR_WORKSPACE);
  OXR_RETURN_IF(!device_fits(), OXR_ERR_UNSUPPORTED);
  if (rows == 0) return OXR_OK;
  char* ws = static_cast<char*>(workspace);
  MlpArgs a{o_partials, o_splits, (int)rows, residual_in, residual_out, post_norm, eps, gate_up_interleaved, down,
            partials_out, reinterpret_cast<uint32_t*>(ws), reinterpret_cast<bf16_t*>(ws + kCtlBytes),
            reinterpret_cast<bf16_t*>(ws + kCtlBytes + kXcds * kHElems * sizeof(bf16_t))};
  return rows <= 16 ? launch_nb<1>(a, (hipStream_t)stream) : launch_nb<2>(a, (hipStream_t)stream);
}
