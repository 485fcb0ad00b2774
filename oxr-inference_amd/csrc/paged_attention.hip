// Multi-query causal paged attention for the verify step (gfx950).
//
// Replaces attention.paged_extend (oxr_runtime/attention.py:96-109), whose math
// is the reference test stub (tests/test_language_fused.py:19-28, 50-57): for
// sequence b with L = seq_lens[b], new token s (absolute position L - S + s)
// of q head h attends keys [0, L - S + s] of kv head h / (H / KV), scores
// q.k * scale, fp32 softmax, then the probability-weighted sum of V.
//
// Work split.  A verify step has only B * KV (sequence, kv-head) pairs, each
// with R = S * (H / KV) query rows (8 at S=4, 16/8 heads), against contexts
// of thousands of tokens.  A workgroup of 8 waves owns HPW adjacent kv heads
// (2 when the fused row jobs fit, else 1) of one sequence and one of `splits`
// ranges of its context, so that about 256 workgroups (one per CU) cover the
// batch.  Each head gets 8 / HPW waves that walk the range in interleaved
// 32-key steps; at any time the workgroup reads neighbouring keys of the same
// pages, HPW adjacent 256-byte head slices of each 2 KB token row.  A head's
// waves' (max, sum, O) are merged on chip through LDS and written as the
// split's partial; a second small kernel merges the splits.  (A "last
// workgroup merges" scheme in one kernel needs a device-scope acquire-release
// per workgroup, i.e. an L2 writeback + invalidate across XCDs, which costs
// more than the second launch.)  A context that fits one split is stored
// directly by the main kernel.
//
// Per wave, 32 keys at a time (two 16-key MFMA tiles), all in registers:
//   K and V are read as whole 128-byte cache lines: load instruction q of a
//     tile gives lane l the 16 bytes [16c, +16) of key 8(q / 2) + l / 8, with
//     c = 8(q % 2) + l % 8, so 8 consecutive lanes cover one line.  The MFMA
//     wants lane (r = l % 16, g = l / 16) to hold K[key r][32i + 8g, +8) for
//     MFMA i; each wave passes its tiles through its own 4.25 KB of LDS to
//     get there (written in load order, read in fragment order, rows padded
//     so neither side has bank conflicts).  Measured on loads alone: full
//     lines with the LDS pass 27.3 us, half-line fragment loads 30.1 us.
//   S^T tile = K[16 keys x 128] * Q^T           4 v_mfma_f32_16x16x32_bf16 / tile
//     MFMA i takes dims [32i, 32i + 32); Q^T stays in registers in the same
//     mapping.  Lane (r, g) gets the scores of keys 4g..4g+3 of the tile for
//     query row r.
//   online softmax per row in the exp2 domain (scale * log2 e folded in)
//   V^T fragments by MFMA: V[16 keys x 32 dims] times a 0/1 selector gives
//     C[key][n] = V[key][n] (or [n + 16]) in the C layout, i.e. lane (n, g) holds
//     keys 4g..4g+3 of dim n -- the transposed fragment the PV product needs.
//     (Exact: each output is one bf16 value times 1 plus zeros.)  This replaces
//     an LDS transpose: no LDS, no barriers.
//   O^T += V^T[128 x 32 keys] * P^T             8 MFMAs (one per 16 dims)
//     P^T is the B operand as computed (bf16), key slot 4p + j of lane group g
//     standing for key 16p + 4g + j; accumulators hold O^T[d][r], so the
//     per-row rescale is a per-lane scalar.
// The next 32 keys' K and V are loaded before the current ones are used.
#include <algorithm>
#include <mutex>

#include "norm_rope.h"

namespace oxr {
namespace {

constexpr int kD = 128;
constexpr uint32_t kBf16One = 0x3f80u;

typedef float f32x2 __attribute__((ext_vector_type(2)));

// Context K/V rows are read once per layer and step, but through ordinary loads: non-temporal ones
// made the launch slower (41.6 vs 36.0 us).  The split partials use ordinary stores too: non-temporal
// ones made the step 11 us slower (the merge kernel gains from the lines staying cached).
__device__ __forceinline__ u32x4 ld_kv(const void* p) { return ld128(p); }

// As loaded, register q of tile p holds, in lane l, bytes [16c, +16) of key
// 16p + 8(q / 2) + l / 8 with c = 8(q % 2) + l % 8 (full lines).  After
// to_fragments: tile p, MFMA i, lane (r, g) holds key 16p + r, dims
// [32i + 8g, +8) (K), resp. [32c + 8g, +8) for V's register c.
struct PairRegs {
  u32x4 k[2][4];
  u32x4 v[2][4];
};

// Page numbers of the two 16-key tiles of the pair at t0 (wave-uniform: a
// 16-key tile lies inside one page since block_size >= 16 and tiles are
// aligned to 16), from the workgroup's LDS copy of its page-table range,
// clamped into the pool.  Keys past L use the page of key L - 1.
__device__ __forceinline__ void pair_pages(const int* s_pages, int page0, int t0, int L, int log2_bs,
                                           int64_t num_blocks, int64_t& blk0, int64_t& blk1) {
  const int tile0 = __builtin_amdgcn_readfirstlane(min(t0, L - 1));
  const int tile1 = __builtin_amdgcn_readfirstlane(min(t0 + 16, L - 1));
  blk0 = __builtin_amdgcn_readfirstlane(s_pages[(tile0 >> log2_bs) - page0]);
  blk1 = __builtin_amdgcn_readfirstlane(s_pages[(tile1 >> log2_bs) - page0]);
  blk0 = blk0 < 0 ? 0 : (blk0 >= num_blocks ? num_blocks - 1 : blk0);  // never leave the pool
  blk1 = blk1 < 0 ? 0 : (blk1 >= num_blocks ? num_blocks - 1 : blk1);
}

// K and V of the pair at t0 whose tiles lie in pages blk0, blk1, in the load
// layout (whole lines, see PairRegs).  Keys past L re-read key L - 1: their
// probabilities are exactly 0 and the cache rows below L hold finite values,
// so they add nothing.
__device__ __forceinline__ void load_pair(PairRegs& pr, const bf16_t* __restrict__ k_cache,
                                          const bf16_t* __restrict__ v_cache, int64_t blk0, int64_t blk1, int t0,
                                          int L, int kvh, int KV, int log2_bs, int lane) {
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int64_t page = ((p ? blk1 : blk0) << log2_bs) * KV * kD;  // wave-uniform
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // keys 8h .. 8h + 7 of the tile
      const uint32_t tok = (uint32_t)min(t0 + 16 * p + 8 * h + (lane >> 3), L - 1);
      const uint32_t off = ((tok & ((1u << log2_bs) - 1)) * (uint32_t)KV + (uint32_t)kvh) * kD + 8 * (lane & 7);
#pragma unroll
      for (int c3 = 0; c3 < 2; ++c3) {  // bytes [128 c3, +128) of the 256-byte row
        pr.k[p][2 * h + c3] = ld_kv(k_cache + page + off + 64 * c3);
        pr.v[p][2 * h + c3] = ld_kv(v_cache + page + off + 64 * c3);
      }
    }
  }
}

// A pair's K or V tiles from the load layout to the MFMA fragment layout
// through the wave's LDS exchange buffer, one tile at a time.  The tile is
// stored as 16 rows of 17 16-byte slots (key, then chunk c = dims [8c, +8)):
// the 8 lanes of a line write 128 contiguous bytes, and the 16 lanes of a
// fragment read (16 keys at one chunk) fall in distinct banks.  Both sides
// address one base register plus immediate offsets.  The wave's LDS
// operations complete in order, so the reads see the writes and the next
// tile's writes come after these reads, with no wait or barrier.
constexpr int kXRow = 17;                 // slots per key row
constexpr int kXSlots = 16 * kXRow;       // one tile: 4352 bytes
__device__ __forceinline__ void to_fragments(u32x4 (&t)[2][4], u32x4* xbuf, int lane) {
  const int wbase = kXRow * (lane >> 3) + (lane & 7);     // key 8h + l / 8, chunk 8c3 + l % 8
  const int rbase = kXRow * (lane & 15) + (lane >> 4);    // key r, chunk 4i + g
#pragma unroll
  for (int p = 0; p < 2; ++p) {
#pragma unroll
    for (int q = 0; q < 4; ++q) xbuf[wbase + 8 * kXRow * (q >> 1) + 8 * (q & 1)] = t[p][q];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[p][i] = xbuf[rbase + 4 * i];
  }
}

// Selector B operand: B[k][n] = 1 where k == n + shift (k = 8g + jj, n = r).
__device__ __forceinline__ u32x4 selector(int r, int g, int shift) {
  const int jj = r + shift - 8 * g;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e == jj) w[e >> 1] |= kBf16One << (16 * (e & 1));
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Output vector of 4 dims at (token, column) of out [B * S, H * 128]:
// row-major, or the packed layout of the o_proj GEMM's X operand.
__device__ __forceinline__ uint32_t* out_vec(bf16_t* out, int64_t tok, int64_t col, int64_t row_len, int packed) {
  return reinterpret_cast<uint32_t*>(out + (packed ? packed_offset(tok, col, row_len) : tok * row_len + col));
}

constexpr int kWaves = 8;            // waves per workgroup
constexpr int kMaxSpanPages = 4096;  // page-table entries of one split, staged in LDS
constexpr int kMaxRowTiles = 2;      // 16-row MFMA tiles of query rows per (sequence, kv head)
constexpr int kPartRows = 16 * kMaxRowTiles;  // row stride of the split partials
constexpr int kMaxNew = 16;          // new tokens per sequence (S) of the fused kernel
constexpr int kJobSlots = 64 * kWaves / 16;   // 16-lane row jobs per round of the fused prologue
constexpr int kPlanHead = 2;         // plan: [batch, splits, pieces per sequence..., slot entries...]

// Inputs of the fused q/k norm + RoPE + KV store (oxr_qk_norm_rope_paged_extend).
struct RopeArgs {
  const bf16_t* qkv;  // [B * S, H + 2 KV, 128]: the qkv projection of the new tokens
  const bf16_t* q_weight;
  const bf16_t* k_weight;
  const bf16_t* cos_table;  // [table_rows, 64]
  const bf16_t* sin_table;
  int64_t table_rows;
  const int64_t* positions;  // [B * S] RoPE table row of each token
  const int64_t* slots;      // [B * S] cache slot of each token (outside [0, num_slots): not stored)
  int64_t num_slots;
  float eps;
  bf16_t* k_store;  // the caches the kernel reads, for the new rows
  bf16_t* v_store;
};

// kFused: q comes from qkv through norm + RoPE (done here, into LDS), and the
// new tokens' K (norm + RoPE) and V rows are written to the cache by the
// workgroup whose key range holds their positions, before any wave reads them;
// otherwise q is read as given.  The caches are plain (not restrict) pointers
// because the fused kernel writes the rows it later reads.
// NT: 16-row tiles of query rows (R = S * H / KV <= 16 * NT); every pair of keys
// is multiplied by each tile, and the V^T fragments are shared by the tiles.
// JR: rounds of the fused prologue's 32 row jobs (HPW * (R + 2 S) <= 32 * JR).
// kPlanned: pieces from a plan (paged_extend_plan_kernel); otherwise `splits` even pieces per context.
template <bool kFused, int HPW, int NT, int JR, bool kPlanned>
__global__ __launch_bounds__(64 * kWaves) void paged_extend_kernel(
    const bf16_t* __restrict__ q, const bf16_t* k_cache, const bf16_t* v_cache, const int32_t* __restrict__ seq_lens,
    const int32_t* __restrict__ block_table, int64_t table_stride, int S, int H, int KV, int log2_bs,
    int64_t num_blocks, float scale_log2, int max_seq_len, int splits, const int32_t* __restrict__ plan,
    float* __restrict__ part_o, float* __restrict__ part_ml, bf16_t* __restrict__ out, int out_packed, RopeArgs ra) {
  constexpr int kStreams = kWaves / HPW;  // waves per kv head
  // Two row tiles' q fragments (32 registers) would not fit next to two tiles'
  // accumulators and the two pair buffers: with NT = 2 the MFMAs read them from LDS.
  constexpr bool kQinLds = NT == 2;
  __shared__ float s_o[kWaves][16][kD];   // per wave: the K/V exchange buffer, then one row tile's results
  __shared__ u32x4 s_q[kFused || kQinLds ? HPW : 1][kFused || kQinLds ? 16 * NT : 1][kD / 8];
  __shared__ u32x4 s_newk[kFused ? HPW : 1][kFused ? kMaxNew : 1][kD / 8];
  __shared__ u32x4 s_newv[kFused ? HPW : 1][kFused ? kMaxNew : 1][kD / 8];
  __shared__ float s_m[kWaves][16], s_l[kWaves][16];
  __shared__ int s_pages[kMaxSpanPages];

  // Which piece of which context this workgroup takes: piece blockIdx.x of sequence blockIdx.z of
  // `splits` even pieces, or, with a plan (paged_extend_plan_kernel), the entry of its slot.  A plan
  // whose header names another batch or split count was written for another launch: the launch then
  // runs on even pieces (the merge makes the same test), which read and write the same units.
  int split = blockIdx.x, b = blockIdx.z, pieces = 0;
  const bool use_plan = kPlanned && plan[0] == (int)gridDim.z && plan[1] == splits;
  if (use_plan) {
    const int a = plan[kPlanHead + gridDim.z + blockIdx.z * splits + blockIdx.x];
    // A spare slot the plan leaves idle (workgroup-uniform); entries out of range (a plan written for
    // another launch) are treated alike, so nothing is addressed outside the launch's arrays.
    if (a < 0 || (a >> 8) >= (int)gridDim.z || (a & 255) >= 2 * splits) return;
    b = a >> 8;
    split = a & 255;
    pieces = min(max(plan[kPlanHead + b], 1), 2 * splits);
  }
  const int G = H / KV, R = S * G;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform, so its addressing is scalar
  const int r = lane & 15, g = lane >> 4;
  // The workgroup owns kv heads [HPW * blockIdx.y, +HPW): wave w serves head
  // slot w % HPW and walks that head's keys as stream w / HPW of kStreams.
  const int hs = wave % HPW, stream = wave / HPW;
  const int kvh = (int)blockIdx.y * HPW + hs;

  // Fused: HPW * (R + 2S) row jobs of one 128-element row each, on 16 lanes, in
  // JR rounds of 32 -- per head slot, q rows [0, R), then the K rows and the V
  // rows of the S new tokens.  Lanes without a job redo job 0 (every lane must
  // take part in the norm's exchanges) and store nothing.  Their loads go out
  // first: none depends on the context length.
  const int f_s16 = tid & 15;
  const int f_per_head = R + 2 * S;
  bool f_valid[JR];
  int f_hs[JR], f_jj[JR], f_ss[JR];
  int64_t f_trow[JR], f_slot[JR];
  u32x4 f_raw[JR], f_w8[JR];
#pragma unroll
  for (int jr = 0; jr < JR; ++jr) {
    f_valid[jr] = false;
    f_hs[jr] = f_jj[jr] = f_ss[jr] = 0;
    f_trow[jr] = 0;
    f_slot[jr] = -1;
    f_raw[jr] = f_w8[jr] = u32x4{0u, 0u, 0u, 0u};
  }
  if constexpr (kFused) {
#pragma unroll
    for (int jr = 0; jr < JR; ++jr) {
      const int job = (tid >> 4) + kJobSlots * jr;
      f_valid[jr] = job < HPW * f_per_head;
      const int jv = f_valid[jr] ? job : 0;
      f_hs[jr] = jv / f_per_head;
      f_jj[jr] = jv % f_per_head;
      const int kvh_j = (int)blockIdx.y * HPW + f_hs[jr];
      int head;
      if (f_jj[jr] < R) {
        f_ss[jr] = f_jj[jr] / G;
        head = kvh_j * G + f_jj[jr] % G;
      } else if (f_jj[jr] < R + S) {
        f_ss[jr] = f_jj[jr] - R;
        head = H + kvh_j;
      } else {
        f_ss[jr] = f_jj[jr] - R - S;
        head = H + KV + kvh_j;
      }
      const int64_t tok = (int64_t)b * S + f_ss[jr];
      f_raw[jr] = ld128(ra.qkv + (tok * (H + 2 * KV) + head) * kD + f_s16 * 8);
      f_w8[jr] = ld128((f_jj[jr] < R ? ra.q_weight : ra.k_weight) + f_s16 * 8);
      f_slot[jr] = ra.slots[tok];
      f_trow[jr] = ra.positions[tok];
    }
  }

  const int L = min(seq_lens[b], max_seq_len);  // max_seq_len <= table span, checked on the host

  // This workgroup's keys: piece `split` of [0, L), in whole 32-key pairs.
  // (A plan's pieces are never longer than an even split of max_seq_len; the clamp keeps the page
  // range inside the LDS copy whatever the plan holds.)
  const int span = use_plan ? min(((L + pieces - 1) / pieces + 31) / 32 * 32,
                                  ((max_seq_len + splits - 1) / splits + 31) / 32 * 32)
                            : ((L + splits - 1) / splits + 31) / 32 * 32;
  const int t_begin = split * span;
  const int t_end = min(L, t_begin + span);
  const bool single = use_plan ? pieces == 1 : L <= span;  // the whole context is in piece 0
  // A plan built from other (shorter) lengths can leave keys past its pieces; that sequence's rows
  // are then written as NaN (here when it has one piece, else by the merge) instead of dropping keys.
  const bool uncovered = use_plan && (int64_t)pieces * span < L;
  if (single && split > 0) return;
  const int32_t* table_row = block_table + (int64_t)b * table_stride;

  // This split's page numbers (as stored; clamped when read), staged into LDS below.  One entry per thread
  // covers spans up to 512 pages; the load is unconditional (an empty split
  // reads entry 0) so the waits below count exactly.
  const int page0 = t_begin >> log2_bs;
  const int npages = t_end > t_begin ? ((t_end - 1) >> log2_bs) - page0 + 1 : 0;  // <= kMaxSpanPages (host check)
  const int64_t my_page = table_row[npages > 0 ? page0 + min(tid, npages - 1) : 0];
  __builtin_amdgcn_sched_barrier(0);

  // A head's streams take pairs stream, stream + kStreams, ... so at any time
  // the workgroup reads neighbouring pairs of the same pages, HPW adjacent
  // head slices of each token row.  Each wave's first pair is requested right
  // away, its pages read straight from the table, so it is in flight during
  // the page-table staging, the fused q/k work and the barrier.
  const int stride = 32 * kStreams;
  const int t_first = t_begin + 32 * stream;
  const int n = t_first < t_end ? (t_end - t_first + stride - 1) / stride : 0;
  // (Issued by every wave -- a wave without pairs reads a valid row it never
  // uses -- so that no branch blurs the wait counts that follow.)
  PairRegs kv_a, kv_b;
  u32x4 f_c8[JR], f_s8[JR];
  {
    const int Lc = L > 0 ? L : 1;  // an empty context still addresses key 0
    const int tile0 = min(t_first, Lc - 1), tile1 = min(t_first + 16, Lc - 1);
    const int e0 = table_row[tile0 >> log2_bs], e1 = table_row[tile1 >> log2_bs];  // both requested before either is used
    const int nb = (int)num_blocks;  // < 2^31, checked on the host
    const int64_t blk0 = e0 < 0 ? 0 : (e0 >= nb ? nb - 1 : e0);  // never leave the pool
    const int64_t blk1 = e1 < 0 ? 0 : (e1 >= nb ? nb - 1 : e1);
    // Fused: the RoPE row of each new token's position, requested while the
    // first pair's page numbers are on their way.
#pragma unroll
    for (int jr = 0; jr < JR; ++jr) {
      f_c8[jr] = f_s8[jr] = u32x4{0u, 0u, 0u, 0u};
      if constexpr (kFused) {
        const int64_t row = f_trow[jr] < 0 ? 0 : (f_trow[jr] >= ra.table_rows ? ra.table_rows - 1 : f_trow[jr]);
        f_c8[jr] = ld128(ra.cos_table + row * (kD / 2) + (f_s16 & 7) * 8);
        f_s8[jr] = ld128(ra.sin_table + row * (kD / 2) + (f_s16 & 7) * 8);
      }
    }
    load_pair(kv_a, k_cache, v_cache, blk0, blk1, t_first, Lc, kvh, KV, log2_bs, lane);
  }
  __builtin_amdgcn_sched_barrier(0);

  // (Every thread writes its entry, past npages too -- never read -- so the
  // load above is not moved into a branch.)
  s_pages[tid] = (int)my_page;
  for (int i = tid + 64 * kWaves; i < npages; i += 64 * kWaves) {  // spans beyond 512 pages
    s_pages[i] = table_row[page0 + i];
  }

  if constexpr (kFused) {
    // The new tokens' rows (see the top of the kernel for the job layout).
#pragma unroll
    for (int jr = 0; jr < JR; ++jr) {
      const u32x4 normed = norm_rope_16v(f_raw[jr], f_w8[jr], f_c8[jr], f_s8[jr], ra.eps, f_s16);
      if (f_valid[jr] && f_jj[jr] < R) {
        s_q[f_hs[jr]][f_jj[jr]][f_s16] = normed;
      } else if (f_valid[jr]) {
        // Kept in LDS for this workgroup's own reads of the new rows, and
        // written to the cache by the workgroup whose keys hold the token's
        // position (each row stored once; nothing in this launch reads it back
        // from memory, so the stores need not complete before the loop).
        const bool is_k = f_jj[jr] < R + S;
        if (is_k) s_newk[f_hs[jr]][f_ss[jr]][f_s16] = normed;
        else s_newv[f_hs[jr]][f_ss[jr]][f_s16] = f_raw[jr];
        const int pos = L - S + f_ss[jr];
        if (pos >= t_begin && pos < t_end && f_slot[jr] >= 0 && f_slot[jr] < ra.num_slots) {
          const int kvh_j = (int)blockIdx.y * HPW + f_hs[jr];
          bf16_t* dst = (is_k ? ra.k_store : ra.v_store) + (f_slot[jr] * KV + kvh_j) * kD + f_s16 * 8;
          st128(dst, is_k ? normed : f_raw[jr]);
        }
      }
    }
  }

  // Query row 16t + r of tile t: token (16t + r) / G, head (16t + r) % G of this kv head.
  u32x4 qf[NT][4];
  int qpos[NT];  // absolute position of the row; keys after it are masked
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int rr = 16 * t + r;
    qpos[t] = -1;
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[t][i] = u32x4{0u, 0u, 0u, 0u};
    if (rr < R) {
      const int s = rr / G, hh = rr % G;
      if constexpr (!kFused) {
        const bf16_t* src = q + (((int64_t)b * S + s) * H + kvh * G + hh) * kD + 8 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) qf[t][i] = ld128(src + 32 * i);
      }
      qpos[t] = L - S + s;
    }
    if constexpr (kQinLds && !kFused) {
      if (stream == 0) {  // wave-uniform: one wave per head stages its rows (zeros past R)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_q[hs][rr][4 * i + g] = qf[t][i];
      }
    }
  }
  const u32x4 sel_lo = selector(r, g, 0), sel_hi = selector(r, g, 16);
  // LDS (s_pages; fused: s_q and the new K/V rows) is complete; global loads
  // and stores stay in flight across the barrier.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if constexpr (kFused && !kQinLds) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (16 * t + r < R) {
#pragma unroll
        for (int i = 0; i < 4; ++i) qf[t][i] = s_q[hs][16 * t + r][4 * i + g];
      }
    }
  }

  // Per row tile: running row maximum of the raw scores (m_run) and the same in
  // the exp2 domain (mc_run = m_run * scale * log2 e; 0 while every key is masked).
  float m_run[NT], mc_run[NT], l_run[NT];
  f32x4 o[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    m_run[t] = -INFINITY;
    mc_run[t] = 0.f;
    l_run[t] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // The wave's LDS exchange buffer is its own slice of s_o, which the merge
  // below only uses after this wave's loop.
  u32x4* const xbuf = reinterpret_cast<u32x4*>(&s_o[wave][0][0]);

  auto step = [&](PairRegs& cur, const int t0) {
    to_fragments(cur.k, xbuf, lane);
    to_fragments(cur.v, xbuf, lane);
    if constexpr (kFused) {
      if (t0 + 31 >= L - S) {  // wave-uniform: the pair holds new tokens, whose rows come from LDS
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int ns = min(t0 + 16 * p + r, L - 1) - (L - S);  // keys past L re-read row L - 1
          if (ns >= 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) cur.k[p][i] = s_newk[hs][ns][4 * i + g];  // dims 32i + 8g
#pragma unroll
            for (int c = 0; c < 4; ++c) cur.v[p][c] = s_newv[hs][ns][4 * c + g];  // dims 32c + 8g
          }
        }
      }
    }
    u32x4 pb[NT];
    if constexpr (kQinLds) __asm__ __volatile__("" ::: "memory");  // keep the q reads below in the loop
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // Raw scores of keys t0 + 16p + 4g + j for query row 16t + r (rows past R
      // hold zeros in s_q and are fully masked).
      float sv[8];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc = mfma_16x16x32(cur.k[p][i], kQinLds ? s_q[hs][16 * t + r][4 * i + g] : qf[t][i], acc);
#pragma unroll
        for (int j = 0; j < 4; ++j) sv[4 * p + j] = acc[j];
      }
      if (t0 + 31 > L - S) {  // wave-uniform: only pairs at the causal frontier need the mask
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (t0 + 16 * (e >> 2) + 4 * g + (e & 3) > qpos[t]) sv[e] = -INFINITY;
      }
      float mx =
          fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
      mx = xor32_max(xor16_max(mx));
      // Probabilities exp2(s * c - m * c) against the running row maximum m;
      // the accumulators are rescaled only when some row's maximum moved (when
      // it did not, the factor is exactly 1).
      const bool moved = mx > m_run[t];
      if (__builtin_amdgcn_ballot_w64(moved)) {
        const float m_new = moved ? mx : m_run[t];
        const float mc_new = m_new == -INFINITY ? 0.f : m_new * scale_log2;
        // (Nothing is accumulated while the maximum is -inf: factor 0, never inf.)
        const float alpha =
            !moved ? 1.0f : (m_run[t] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc_run[t] - mc_new));
        l_run[t] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[t][dt] *= alpha;
        m_run[t] = m_new;
        mc_run[t] = mc_new;
      }
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = __builtin_amdgcn_exp2f(fmaf(sv[e], scale_log2, -mc_run[t]));
        l_run[t] += pv[e];
      }
      pb[t] = u32x4{pack_bf_hw(pv[0], pv[1]), pack_bf_hw(pv[2], pv[3]), pack_bf_hw(pv[4], pv[5]),
                    pack_bf_hw(pv[6], pv[7])};
    }

    // V^T fragments: dims 32c + [0, 16) and 32c + [16, 32) of both key tiles,
    // each multiplied into every row tile.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const u32x4 sel = half ? sel_hi : sel_lo;
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        const f32x4 v0 = mfma_16x16x32(cur.v[0][c], sel, z);
        const f32x4 v1 = mfma_16x16x32(cur.v[1][c], sel, z);
        const u32x4 a = {pack_hi16(v0[0], v0[1]), pack_hi16(v0[2], v0[3]), pack_hi16(v1[0], v1[1]),
                         pack_hi16(v1[2], v1[3])};
        const int dt = 2 * c + half;
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t][dt] = mfma_16x16x32(a, pb[t], o[t][dt]);
      }
    }
  };

  // Two register sets, A and B, alternate without copies.  Every prefetch is
  // issued unconditionally (past the wave's last pair it re-reads that pair,
  // an L2 hit), so the only branch skips a compute step and the vmcnt wait
  // before each step counts exactly the 16 loads issued after its own.
  if (n > 0) {
    const int t_last = t_first + (n - 1) * stride;
    for (int i = 0; i < n; i += 2) {
      const int ta = t_first + i * stride;
      int64_t blk0, blk1;
      pair_pages(s_pages, page0, min(ta + stride, t_last), L, log2_bs, num_blocks, blk0, blk1);
      load_pair(kv_b, k_cache, v_cache, blk0, blk1, min(ta + stride, t_last), L, kvh, KV, log2_bs, lane);
      __builtin_amdgcn_sched_barrier(0);
      step(kv_a, ta);
      pair_pages(s_pages, page0, min(ta + 2 * stride, t_last), L, log2_bs, num_blocks, blk0, blk1);
      load_pair(kv_a, k_cache, v_cache, blk0, blk1, min(ta + 2 * stride, t_last), L, kvh, KV, log2_bs, lane);
      __builtin_amdgcn_sched_barrier(0);
      if (i + 1 < n) step(kv_b, ta + stride);
    }
  }
  __asm__ __volatile__("" ::: "memory");  // the exchange buffer's last reads stay before the merge's s_o writes

  // Merge each head's kStreams waves on chip, one row tile at a time.
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float l_tot = xor32_sum(xor16_sum(l_run[t]));
    if (t > 0) __syncthreads();  // the previous tile's merge has read s_o, s_m, s_l
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)  // real rows only: the merge below reads rows < R
      if (16 * t + r < R) *reinterpret_cast<f32x4*>(&s_o[wave][r][dt * 16 + 4 * g]) = o[t][dt];
    if (g == 0) {
      s_m[wave][r] = m_run[t] == -INFINITY ? -INFINITY : mc_run[t];
      s_l[wave][r] = l_tot;
    }
    __syncthreads();
    const int rows = min(16, R - 16 * t);
    for (int idx = tid; idx < HPW * rows * (kD / 4); idx += 64 * kWaves) {
      const int ho = idx / (rows * (kD / 4)), rl = (idx / (kD / 4)) % rows, d0 = (idx % (kD / 4)) * 4;
      const int rr = 16 * t + rl;
      const int kvh_o = (int)blockIdx.y * HPW + ho;
      // Even: the (sequence, piece) unit; planned: this workgroup's own slot (the plan maps pieces to slots).
      const int64_t unit = use_plan ? ((int64_t)blockIdx.z * KV + kvh_o) * splits + blockIdx.x
                                    : ((int64_t)b * KV + kvh_o) * splits + split;
      float mmax = -INFINITY;
#pragma unroll
      for (int k = 0; k < kStreams; ++k) mmax = fmaxf(mmax, s_m[ho + HPW * k][rl]);
      const float mu = (mmax == -INFINITY) ? 0.f : mmax;
      float l = 0.f;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < kStreams; ++k) {
        const int w = ho + HPW * k;
        const float wt = exp2f(s_m[w][rl] - mu);
        l += s_l[w][rl] * wt;
        acc += *reinterpret_cast<const f32x4*>(&s_o[w][rl][d0]) * wt;
      }
      if (single) {
        const float inv = uncovered ? __builtin_nanf("") : l > 0.f ? 1.0f / l : 0.f;
        const int s = rr / G, hh = rr % G;
        uint32_t* dst = out_vec(out, (int64_t)b * S + s, (kvh_o * G + hh) * kD + d0, H * kD, out_packed);
        dst[0] = pack_bf(acc[0] * inv, acc[1] * inv);
        dst[1] = pack_bf(acc[2] * inv, acc[3] * inv);
      } else {
        f32x4* const po = reinterpret_cast<f32x4*>(part_o + (unit * kPartRows + rr) * kD + d0);
        *po = acc;
        if (d0 == 0) *reinterpret_cast<f32x2*>(part_ml + (unit * kPartRows + rr) * 2) = f32x2{mmax, l};
      }
    }
  }
}

// The merge for a planned launch: the sequence's context is in `pieces` pieces, piece j's partial at the
// unit of the workgroup slot piece_slots[j] (z << 8 | x) names (each written by this launch, possibly
// empty: max -inf, sum 0); one piece was stored by the main kernel.  All of a chunk's partials are
// requested before the first use.
// `uncovered`: the plan's pieces do not reach the context's end (a plan built from other lengths);
// the rows are then written as NaN.  A piece entry outside the launch (-1, or a slot past the batch or
// the split count) is read from the sequence's own first slot with weight 0 and also makes the rows NaN.
__device__ __forceinline__ void merge_planned(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                              int pieces, const int32_t* __restrict__ piece_slots, int b,
                                              int batch, int KV, int kvh, int splits, bool uncovered, int rr,
                                              int d0, uint32_t* dst) {
  constexpr int kChunk = 8;
  if (pieces <= 1) return;
  float m = -INFINITY, l = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  bool bad = uncovered;
  for (int c0 = 0; c0 < pieces; c0 += kChunk) {
    f32x2 ml[kChunk];
    f32x4 v[kChunk];
    int64_t unit[kChunk];
    bool ok[kChunk];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {  // past the last piece: the last, weight 0 below
      const int jj = min(c0 + j, pieces - 1);
      // The first `splits` pieces sit in the sequence's own slots; later ones in the slots that took them.
      int e = jj < splits ? (b << 8) | jj : piece_slots[jj];
      ok[j] = e >= 0 && (e >> 8) < batch && (e & 255) < splits;
      if (!ok[j]) e = b << 8;
      unit[j] = ((int64_t)(e >> 8) * KV + kvh) * splits + (e & 255);
    }
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const int64_t u = unit[j];
      ml[j] = *reinterpret_cast<const f32x2*>(part_ml + (u * kPartRows + rr) * 2);
      v[j] = *reinterpret_cast<const f32x4*>(part_o + (u * kPartRows + rr) * kD + d0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      bad |= c0 + j < pieces && !ok[j];
      const float mj = c0 + j < pieces && ok[j] ? ml[j][0] : -INFINITY;
      const float mn = fmaxf(m, mj);
      const float mu = (mn == -INFINITY) ? 0.f : mn;
      const float a = exp2f(m - mu), w = exp2f(mj - mu);
      l = l * a + ml[j][1] * w;
      acc = acc * a + v[j] * w;
      m = mn;
    }
  }
  const float inv = bad ? __builtin_nanf("") : l > 0.f ? 1.0f / l : 0.f;
  dst[0] = pack_bf(acc[0] * inv, acc[1] * inv);
  dst[1] = pack_bf(acc[2] * inv, acc[3] * inv);
}

// Merge of the context splits of every (sequence, kv head): one workgroup per
// pair, one thread per 4 output dims of a row.  Sequences whose context fitted
// one split were already stored by the main kernel.
// The merge's workgroups split each row's kD dims into 4 slices when a (sequence, kv head) has 8 or
// more rows, 2 from 4 rows, else 1, so that every workgroup still fills a wave: at B = 8, S = 4 the
// launch is 256 one-wave workgroups, each reading a quarter of a (sequence, kv head)'s partials.
// Measured against one slice: verify step 2151.5 vs 2157 us; one token per sequence (2 rows) with 4
// slices made the decode step 3 us slower, hence the row threshold.
int merge_dim_slices(int rows) { return rows >= 8 ? 4 : rows >= 4 ? 2 : 1; }

template <bool kPlanned>
__global__ __launch_bounds__(kPartRows * kD / 4) void paged_extend_merge_kernel(const float* __restrict__ part_o,
                                                                              const float* __restrict__ part_ml,
                                                                              const int32_t* __restrict__ seq_lens,
                                                                              int S, int H, int KV, int max_seq_len,
                                                                              int splits,
                                                                              const int32_t* __restrict__ plan,
                                                                              bf16_t* __restrict__ out,
                                                                              int out_packed) {
  constexpr int kChunk = 8;  // splits whose partials are requested together
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int G = H / KV;
  // One thread per 4 output dims of a row; with gridDim.z = 1, 2 or 4 dim slices, workgroup z takes
  // dims [z, z + 1) * kD / gridDim.z of every row (blockDim = rows * kD / 4 / gridDim.z).
  const int shift = __builtin_ctz(gridDim.z);
  const int per_row = (kD / 4) >> shift;
  const int rr = threadIdx.x / per_row;
  const int d0 = (int)blockIdx.z * (kD >> shift) + (threadIdx.x & (per_row - 1)) * 4;
  // A plan written for another launch (header: batch, splits) is ignored, as the main kernel ignores it.
  if (kPlanned && plan[0] == (int)gridDim.y && plan[1] == splits) {
    const int pieces = min(max(plan[kPlanHead + b], 1), 2 * splits);
    const int L = min(seq_lens[b], max_seq_len);
    const int span = min(((L + pieces - 1) / pieces + 31) / 32 * 32, ((max_seq_len + splits - 1) / splits + 31) / 32 * 32);
    merge_planned(part_o, part_ml, pieces, plan + kPlanHead + (int)gridDim.y * (1 + splits) + b * 2 * splits, b,
                  (int)gridDim.y, KV, kvh, splits, (int64_t)pieces * span < L, rr, d0,
                  out_vec(out, (int64_t)b * S + rr / G, (kvh * G + rr % G) * kD + d0, H * kD, out_packed));
    return;
  }
  const int64_t unit0 = ((int64_t)b * KV + kvh) * splits;
  // The context length is only needed at the end, but it is requested first so that its
  // latency overlaps the partials' instead of following it.  (As inline asm: the compiler
  // would sink an ordinary load of it to its use.  Being older than every load below, it
  // leaves the compiler's own counted waits exact; the explicit wait before its use covers it.)
  int seq_len_b;
  asm volatile("global_load_dword %0, %1, off" : "=v"(seq_len_b) : "v"(seq_lens + b) : "memory");
  float m = -INFINITY, l = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < splits; c0 += kChunk) {
    // The chunk's partials are requested together; entries past the last
    // split re-read it and enter with weight 0 (max -inf), exactly neutral.
    f32x2 ml[kChunk];
    f32x4 v[kChunk];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const int64_t u = unit0 + min(c0 + j, splits - 1);
      ml[j] = *reinterpret_cast<const f32x2*>(part_ml + (u * kPartRows + rr) * 2);
      v[j] = *reinterpret_cast<const f32x4*>(part_o + (u * kPartRows + rr) * kD + d0);
    }
    __builtin_amdgcn_sched_barrier(0);  // all of the chunk's loads go out before the first use
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const float mj = c0 + j < splits ? ml[j][0] : -INFINITY;
      const float mn = fmaxf(m, mj);
      const float mu = (mn == -INFINITY) ? 0.f : mn;
      const float a = exp2f(m - mu), w = exp2f(mj - mu);
      l = l * a + ml[j][1] * w;
      acc = acc * a + v[j] * w;
      m = mn;
    }
  }
  // Sequences whose context fitted one split were stored by the main kernel
  // (checked only now, so the partials above were requested without waiting).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the length load has landed
  const int L = min(seq_len_b, max_seq_len);
  const int span = ((L + splits - 1) / splits + 31) / 32 * 32;
  if (L <= span) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  const int s = rr / G, hh = rr % G;
  uint32_t* dst = out_vec(out, (int64_t)b * S + s, (kvh * G + hh) * kD + d0, H * kD, out_packed);
  dst[0] = pack_bf(acc[0] * inv, acc[1] * inv);
  dst[1] = pack_bf(acc[2] * inv, acc[3] * inv);
}

// A plan of context pieces for one launch (oxr_paged_extend_plan), so that contexts of different
// lengths take workgroups in proportion.  Without one, every context is cut into the launch's
// `splits` pieces and the longest bounds the launch.  One piece length serves the whole batch:
// the smallest multiple of 32 keys, from its total context over the B * splits workgroup slots up,
// for which the pieces fit the slots (each context at least one piece, at most 2 * splits).
// Slot (sequence z, x) takes piece x of context z while z has that many; the slots a short
// context leaves spare take, in order, the pieces past `splits` of the long ones; any left over
// stay idle.  Layout: [batch, splits, pieces of each sequence (B), slot entries (B * splits): sequence << 8 |
// piece, or -1 for idle; then per sequence 2 * splits piece entries: the slot z << 8 | x that takes the
// piece (-1 past the sequence's pieces)], where the header [batch, splits] names the launch the plan is
// for (the attention kernels ignore a plan whose header differs).  A workgroup writes its partial at its own slot's unit, so
// the workspace is that of an even launch.
constexpr int kPlanMaxBatch = 256;
constexpr int kPlanThreads = 256;
__global__ __launch_bounds__(kPlanThreads) void paged_extend_plan_kernel(const int32_t* __restrict__ seq_lens,
                                                                         int batch, int max_seq_len, int splits,
                                                                         int32_t* __restrict__ plan) {
  __shared__ int s_n[kPlanMaxBatch];
  __shared__ int s_spare[kPlanMaxBatch + 1], s_over[kPlanMaxBatch + 1];  // exclusive prefix sums
  __shared__ unsigned long long s_total;
  __shared__ int s_count;
  const int t = threadIdx.x;
  const int len = t < batch ? max(0, min(seq_lens[t], max_seq_len)) : 0;
  if (t == 0) s_total = 0ull;
  __syncthreads();
  if (len > 0) atomicAdd(&s_total, (unsigned long long)len);
  __syncthreads();
  const long long slots = (long long)batch * splits;
  const long long total = (long long)s_total;
  int span = (int)((total + slots - 1) / slots);
  span = max(32, (span + 31) / 32 * 32);
  const int span_max = max(32, (max_seq_len + 31) / 32 * 32);  // one piece per context: always fits
  for (int it = 0; it < 1 << 16; ++it) {
    if (t == 0) s_count = 0;
    __syncthreads();
    if (t < batch) atomicAdd(&s_count, min(max((len + span - 1) / span, 1), 2 * splits));
    __syncthreads();
    const int count = s_count;
    __syncthreads();  // every thread has read the count before the next pass clears it
    if (count <= slots || span >= span_max) break;
    span += 32;
  }
  if (t < batch) s_n[t] = min(max((len + span - 1) / span, 1), 2 * splits);
  __syncthreads();
  if (t == 0) {
    int sp = 0, ov = 0;
    for (int b = 0; b < batch; ++b) {
      s_spare[b] = sp;
      s_over[b] = ov;
      sp += splits - min(s_n[b], splits);
      ov += max(s_n[b] - splits, 0);
    }
    s_spare[batch] = sp;
    s_over[batch] = ov;
    plan[0] = batch;
    plan[1] = splits;
  }
  __syncthreads();
  if (t < batch) plan[kPlanHead + t] = s_n[t];
  for (long long w = t; w < slots; w += kPlanThreads) {
    const int z = (int)(w / splits), x = (int)(w % splits);
    int entry = -1;
    if (x < s_n[z]) {
      entry = (z << 8) | x;
    } else {
      const int r = s_spare[z] + (x - s_n[z]);  // rank among the spare slots
      if (r < s_over[batch]) {                  // the overflow piece of that rank
        int lo = 0, hi = batch;                 // s_over[lo] <= r < s_over[lo + 1]
        while (hi - lo > 1) {
          const int mid = (lo + hi) / 2;
          if (s_over[mid] <= r) lo = mid;
          else hi = mid;
        }
        entry = (lo << 8) | (splits + (r - s_over[lo]));
      }
    }
    plan[kPlanHead + batch + w] = entry;
    if (entry >= 0) plan[kPlanHead + batch + slots + (entry >> 8) * 2 * splits + (entry & 255)] = (z << 8) | x;
  }
  // Piece entries past each sequence's pieces.
  for (long long e = t; e < (long long)batch * 2 * splits; e += kPlanThreads)
    if ((int)(e % (2 * splits)) >= s_n[e / (2 * splits)]) plan[kPlanHead + batch + slots + e] = -1;
}

// Context splits per (sequence, group of `hpw` kv heads): about one 8-wave
// workgroup per CU over the whole batch, but at least kMinSplitKeys keys of
// the longest context per split.  (At B = 1, 256 workgroups would leave 64
// keys each: the launch is then fixed cost, and the merge walks 64 partials.)
constexpr int kMinSplitKeys = 256;
int splits_for(int32_t batch, int32_t num_kv_heads, int hpw, int32_t max_seq_len) {
  const int64_t units = (int64_t)batch * (num_kv_heads / hpw);
  int64_t splits = (256 + units - 1) / units;
  const int64_t by_keys = ((int64_t)max_seq_len + kMinSplitKeys - 1) / kMinSplitKeys;
  splits = splits < by_keys ? splits : by_keys;
  return (int)(splits < 1 ? 1 : (splits > 64 ? 64 : splits));
}

// kv heads per workgroup: two heads read 512-byte slices of each token row
// together (the heads of a row are adjacent) -- measured 1 us faster per
// launch than one head at the verify shape; four heads (16 splits) were 3 us
// slower.  Two heads only when the fused kernel's row jobs then fit one round
// of 32 16-lane groups; the unfused kernel makes the same choice, so that both
// split the context the same way and give the same bits.
int pick_hpw(int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads) {
  const int jobs_per_head = tokens_per_seq * (num_heads / num_kv_heads + 2);
  for (int hpw : {2, 1}) {
    if (num_kv_heads % hpw != 0 || hpw * jobs_per_head > kJobSlots) continue;
    return hpw;
  }
  return 1;
}

// Rounds of 32 row jobs the fused prologue needs (at most 2).
int job_rounds(int hpw, int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads) {
  const int jobs = hpw * tokens_per_seq * (num_heads / num_kv_heads + 2);
  return (jobs + kJobSlots - 1) / kJobSlots;
}

}  // namespace
}  // namespace oxr

namespace oxr {
namespace {

// Bytes of split partials a launch needs: the largest (batch' * KV * splits) over any head grouping and
// any batch' <= batch (smaller batches split their contexts further, so a workspace sized for a batch
// serves every smaller one).  A planned launch writes one partial per workgroup slot too.  (A launch
// with one split stores its output directly and needs none.)
size_t partial_bytes(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len) {
  if (batch <= 0 || num_kv_heads <= 0 || max_seq_len <= 0) return 0;
  size_t units = 0;
  for (int32_t bb = 1; bb <= batch; ++bb)
    for (int hpw : {1, 2})
      if (num_kv_heads % hpw == 0) {
        const int splits = splits_for(bb, num_kv_heads, hpw, max_seq_len);
        if (splits > 1) units = std::max(units, (size_t)bb * num_kv_heads * splits);
      }
  return units * kPartRows * (kD + 2) * sizeof(float);
}

}  // namespace
}  // namespace oxr

extern "C" size_t oxr_paged_extend_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len) {
  return oxr::partial_bytes(batch, num_kv_heads, max_seq_len);
}

namespace oxr {
namespace {

// Checks, split count and the two launches shared by both entry points; `ra`
// is null for the unfused one.
int launch_paged_extend(const oxr_bf16* q, const oxr_bf16* k_cache, const oxr_bf16* v_cache, const int32_t* seq_lens,
                        const int32_t* block_table, int64_t table_stride, int32_t batch, int32_t tokens_per_seq,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        int64_t num_blocks, int32_t max_seq_len, float scale, oxr_bf16* out, int out_packed,
                        void* workspace, size_t workspace_bytes, const RopeArgs* ra, const int32_t* plan,
                        hipStream_t s) {
  OXR_RETURN_IF(batch < 0 || tokens_per_seq <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_blocks <= 0 ||
                    table_stride < 0 || max_seq_len <= 0,
                OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(head_dim != kD || num_heads % num_kv_heads != 0, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(tokens_per_seq * (num_heads / num_kv_heads) > kPartRows, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(block_size < 16 || (block_size & (block_size - 1)) != 0, OXR_ERR_UNSUPPORTED);
  // Contexts are clamped to max_seq_len, so every key visited maps to a table entry.
  OXR_RETURN_IF((int64_t)max_seq_len > table_stride * block_size, OXR_ERR_INVALID_ARG);
  if (batch == 0) return OXR_OK;
  OXR_RETURN_IF((!ra && !q) || !k_cache || !v_cache || !seq_lens || !block_table || !out, OXR_ERR_INVALID_ARG);
  const size_t need = partial_bytes(batch, num_kv_heads, max_seq_len);
  OXR_RETURN_IF((need > 0 && !workspace) || workspace_bytes < need, OXR_ERR_WORKSPACE);
  OXR_RETURN_IF(batch > 65535 || num_kv_heads > 65535 || num_blocks > 0x7fffffffLL, OXR_ERR_UNSUPPORTED);
  const int hpw = pick_hpw(tokens_per_seq, num_heads, num_kv_heads);
  const int splits = splits_for(batch, num_kv_heads, hpw, max_seq_len);
  {
    // One split's page-table range must fit the kernel's LDS copy.
    const int64_t span_max = ((max_seq_len + splits - 1) / splits + 31) / 32 * 32;
    OXR_RETURN_IF((span_max + block_size - 1) / block_size + 1 > kMaxSpanPages, OXR_ERR_UNSUPPORTED);
  }
  int log2_bs = 0;
  while ((1 << log2_bs) < block_size) ++log2_bs;
  float* part_o = static_cast<float*>(workspace);
  if (splits == 1) plan = nullptr;  // nothing to balance: every context is one piece
  float* part_ml = part_o + (size_t)batch * num_kv_heads * splits * kPartRows * kD;
  const float scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid(splits, num_kv_heads / hpw, batch), block(64 * kWaves);
  const RopeArgs rope = ra ? *ra : RopeArgs{};
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, block, 0, s, ra ? nullptr : q, k_cache, v_cache, seq_lens, block_table,
                       table_stride, tokens_per_seq, num_heads, num_kv_heads, log2_bs, num_blocks, scale_log2,
                       max_seq_len, splits, plan, part_o, part_ml, out, out_packed, rope);
  };  auto launch_k = [&](auto even, auto planned) {
    if (plan) launch(planned);
    else launch(even);
  };

  const int nt = tokens_per_seq * (num_heads / num_kv_heads) > 16 ? 2 : 1;
  if (ra) {
    const int jr = job_rounds(hpw, tokens_per_seq, num_heads, num_kv_heads);  // 1 or 2, checked by the caller
    switch ((hpw - 1) * 4 + (nt - 1) * 2 + (jr - 1)) {
      case 0: launch_k(paged_extend_kernel<true, 1, 1, 1, false>, paged_extend_kernel<true, 1, 1, 1, true>); break;
      case 1: launch_k(paged_extend_kernel<true, 1, 1, 2, false>, paged_extend_kernel<true, 1, 1, 2, true>); break;
      case 2: launch_k(paged_extend_kernel<true, 1, 2, 1, false>, paged_extend_kernel<true, 1, 2, 1, true>); break;
      case 3: launch_k(paged_extend_kernel<true, 1, 2, 2, false>, paged_extend_kernel<true, 1, 2, 2, true>); break;
      case 4: launch_k(paged_extend_kernel<true, 2, 1, 1, false>, paged_extend_kernel<true, 2, 1, 1, true>); break;
      case 6: launch_k(paged_extend_kernel<true, 2, 2, 1, false>, paged_extend_kernel<true, 2, 2, 1, true>); break;
      default: return OXR_ERR_UNSUPPORTED;  // two heads are only chosen when one round holds their jobs
    }
  } else {
    switch ((hpw - 1) * 2 + (nt - 1)) {
      case 0: launch_k(paged_extend_kernel<false, 1, 1, 1, false>, paged_extend_kernel<false, 1, 1, 1, true>); break;
      case 1: launch_k(paged_extend_kernel<false, 1, 2, 1, false>, paged_extend_kernel<false, 1, 2, 1, true>); break;
      case 2: launch_k(paged_extend_kernel<false, 2, 1, 1, false>, paged_extend_kernel<false, 2, 1, 1, true>); break;
      default: launch_k(paged_extend_kernel<false, 2, 2, 1, false>, paged_extend_kernel<false, 2, 2, 1, true>); break;
    }
  }
  int status = OXR_LAUNCH_STATUS();
  if (status || splits == 1) return status;
  const int rows = tokens_per_seq * (num_heads / num_kv_heads);
  hipLaunchKernelGGL(plan ? paged_extend_merge_kernel<true> : paged_extend_merge_kernel<false>,
                     dim3(num_kv_heads, batch, merge_dim_slices(rows)), dim3(rows * kD / 4 / merge_dim_slices(rows)), 0,
                     s, part_o, part_ml,
                     seq_lens, tokens_per_seq, num_heads, num_kv_heads, max_seq_len, splits, plan, out, out_packed);
  return OXR_LAUNCH_STATUS();
}

}  // namespace
}  // namespace oxr

extern "C" int oxr_paged_extend(const oxr_bf16* q, const oxr_bf16* k_cache, const oxr_bf16* v_cache,
                                const int32_t* seq_lens, const int32_t* block_table, int64_t table_stride,
                                int32_t batch, int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t max_seq_len,
                                float scale, oxr_bf16* out, void* workspace, size_t workspace_bytes,
                                oxr_stream_t stream) {
  return oxr::launch_paged_extend(q, k_cache, v_cache, seq_lens, block_table, table_stride, batch, tokens_per_seq,
                                  num_heads, num_kv_heads, head_dim, block_size, num_blocks, max_seq_len, scale, out,
                                  0, workspace, workspace_bytes, nullptr, nullptr, (hipStream_t)stream);
}

extern "C" int oxr_qk_norm_rope_paged_extend(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight,
                                             const oxr_bf16* cos_table, const oxr_bf16* sin_table,
                                             int64_t table_rows, const int64_t* positions, float eps,
                                             oxr_bf16* k_cache, oxr_bf16* v_cache, const int64_t* slots,
                                             int64_t num_slots, const int32_t* seq_lens, const int32_t* block_table,
                                             int64_t table_stride, int32_t batch, int32_t tokens_per_seq,
                                             int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                             int32_t block_size, int64_t num_blocks, int32_t max_seq_len, float scale,
                                             oxr_bf16* out, int32_t out_packed, void* workspace,
                                             size_t workspace_bytes, oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(num_slots < 0, OXR_ERR_INVALID_ARG);
  // One 16-lane job per q row and per new K and V row, in at most two rounds of 32.
  OXR_RETURN_IF(num_kv_heads > 0 && num_heads % num_kv_heads == 0 &&
                    (tokens_per_seq > kMaxNew || tokens_per_seq * (num_heads / num_kv_heads + 2) > 2 * kJobSlots),
                OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(batch > 0 && (!qkv || !q_weight || !k_weight || !cos_table || !sin_table || table_rows <= 0 ||
                              !positions || !slots),
                OXR_ERR_INVALID_ARG);
  const RopeArgs ra{qkv, q_weight, k_weight, cos_table, sin_table, table_rows, positions, slots, num_slots, eps,
                    k_cache, v_cache};
  return launch_paged_extend(nullptr, k_cache, v_cache, seq_lens, block_table, table_stride, batch, tokens_per_seq,
                             num_heads, num_kv_heads, head_dim, block_size, num_blocks, max_seq_len, scale, out,
                             out_packed ? 1 : 0, workspace, workspace_bytes, &ra, nullptr, (hipStream_t)stream);
}

extern "C" size_t oxr_paged_extend_plan_ints(int32_t batch, int32_t tokens_per_seq, int32_t num_heads,
                                             int32_t num_kv_heads, int32_t max_seq_len) {
  using namespace oxr;
  if (batch <= 0 || tokens_per_seq <= 0 || num_heads <= 0 || num_kv_heads <= 0 || max_seq_len <= 0 ||
      num_heads % num_kv_heads != 0)
    return 0;
  const int splits = splits_for(batch, num_kv_heads, pick_hpw(tokens_per_seq, num_heads, num_kv_heads), max_seq_len);
  return splits > 1 ? (size_t)kPlanHead + (size_t)batch + (size_t)batch * 3 * splits : 0;
}

extern "C" int oxr_paged_extend_plan(const int32_t* seq_lens, int32_t batch, int32_t tokens_per_seq,
                                     int32_t num_heads, int32_t num_kv_heads, int32_t max_seq_len, int32_t* plan,
                                     size_t plan_ints, oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(batch < 0 || tokens_per_seq <= 0 || num_heads <= 0 || num_kv_heads <= 0 || max_seq_len <= 0,
                OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(num_heads % num_kv_heads != 0, OXR_ERR_UNSUPPORTED);
  const size_t need = oxr_paged_extend_plan_ints(batch, tokens_per_seq, num_heads, num_kv_heads, max_seq_len);
  if (need == 0) return OXR_OK;  // one piece per context: a planned launch ignores the plan
  OXR_RETURN_IF(!seq_lens || !plan || plan_ints < need, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(batch > kPlanMaxBatch, OXR_ERR_UNSUPPORTED);  // not reached: contexts split only below 256 units
  const int splits = splits_for(batch, num_kv_heads, pick_hpw(tokens_per_seq, num_heads, num_kv_heads), max_seq_len);
  hipLaunchKernelGGL(paged_extend_plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, seq_lens, batch,
                     max_seq_len, splits, plan);
  return OXR_LAUNCH_STATUS();
}

extern "C" int oxr_paged_extend_planned(const oxr_bf16* q, const oxr_bf16* k_cache, const oxr_bf16* v_cache,
                                        const int32_t* seq_lens, const int32_t* block_table, int64_t table_stride,
                                        int32_t batch, int32_t tokens_per_seq, int32_t num_heads,
                                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                        int64_t num_blocks, int32_t max_seq_len, float scale, oxr_bf16* out,
                                        void* workspace, size_t workspace_bytes, const int32_t* plan,
                                        size_t plan_ints, oxr_stream_t stream) {
  OXR_RETURN_IF(!plan || plan_ints < oxr_paged_extend_plan_ints(batch, tokens_per_seq, num_heads, num_kv_heads,
                                                                max_seq_len),
                OXR_ERR_INVALID_ARG);
  return oxr::launch_paged_extend(q, k_cache, v_cache, seq_lens, block_table, table_stride, batch, tokens_per_seq,
                                  num_heads, num_kv_heads, head_dim, block_size, num_blocks, max_seq_len, scale, out,
                                  0, workspace, workspace_bytes, nullptr, plan, (hipStream_t)stream);
}

extern "C" int oxr_qk_norm_rope_paged_extend_planned(
    const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight, const oxr_bf16* cos_table,
    const oxr_bf16* sin_table, int64_t table_rows, const int64_t* positions, float eps, oxr_bf16* k_cache,
    oxr_bf16* v_cache, const int64_t* slots, int64_t num_slots, const int32_t* seq_lens, const int32_t* block_table,
    int64_t table_stride, int32_t batch, int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t max_seq_len, float scale, oxr_bf16* out,
    int32_t out_packed, void* workspace, size_t workspace_bytes, const int32_t* plan, size_t plan_ints,
    oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(num_slots < 0, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(!plan || plan_ints < oxr_paged_extend_plan_ints(batch, tokens_per_seq, num_heads, num_kv_heads,
                                                                max_seq_len),
                OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(num_kv_heads > 0 && num_heads % num_kv_heads == 0 &&
                    (tokens_per_seq > kMaxNew || tokens_per_seq * (num_heads / num_kv_heads + 2) > 2 * kJobSlots),
                OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(batch > 0 && (!qkv || !q_weight || !k_weight || !cos_table || !sin_table || table_rows <= 0 ||
                              !positions || !slots),
                OXR_ERR_INVALID_ARG);
  const RopeArgs ra{qkv, q_weight, k_weight, cos_table, sin_table, table_rows, positions, slots, num_slots, eps,
                    k_cache, v_cache};
  return launch_paged_extend(nullptr, k_cache, v_cache, seq_lens, block_table, table_stride, batch, tokens_per_seq,
                             num_heads, num_kv_heads, head_dim, block_size, num_blocks, max_seq_len, scale, out,
                             out_packed ? 1 : 0, workspace, workspace_bytes, &ra, plan, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// The same launch with no workspace argument, for callers that cannot allocate
// (code under HIP graph capture, serving loops that forbid allocation): the
// split partials live in `scratch`, a static device array each GPU holds until
// the process ends.  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in); the device address comes from
// hipGetSymbolAddress once per device, on the entry point's first call there.
// The partials need no initial contents, so nothing is cleared.  Calls on one
// GPU share the array: calls that overlap in time on one GPU race.
// ---------------------------------------------------------------------------
namespace oxr {
namespace {

// Every shape fits: a launch splits its contexts only while its workgroup units
// (batch * KV / HPW) number fewer than 256, into ceil(256 / units) splits, so
// the partials of any launch cover at most HPW * max_u(u * ceil(256 / u)) =
// 2 * 510 < 1024 (sequence, kv head, split) units of kPartRows x (kD + 2) fp32.
constexpr size_t kScratchBytes = (size_t)1024 * kPartRows * (kD + 2) * sizeof(float);  // 16.25 MiB
constexpr int kScratchMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex scratch_mutex;
void* scratch_ptr[kScratchMaxDevices] = {};

// The current device's address of `scratch` (set up on first use), or an error status.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kScratchMaxDevices) return OXR_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return OXR_ERR_INVALID_ARG;
    scratch_ptr[dev] = ptr;
  }
  *out = scratch_ptr[dev];
  return OXR_OK;
}

}  // namespace
}  // namespace oxr

extern "C" size_t oxr_static_scratch_bytes(void) { return oxr::kScratchBytes; }

extern "C" int oxr_qk_norm_rope_paged_extend_static(
    const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight, const oxr_bf16* cos_table,
    const oxr_bf16* sin_table, int64_t table_rows, const int64_t* positions, float eps, oxr_bf16* k_cache,
    oxr_bf16* v_cache, const int64_t* slots, int64_t num_slots, const int32_t* seq_lens, const int32_t* block_table,
    int64_t table_stride, int32_t batch, int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t max_seq_len, float scale, oxr_bf16* out,
    int32_t out_packed, oxr_stream_t stream) {
  using namespace oxr;
  if (batch > 0 && num_kv_heads > 0 && max_seq_len > 0 &&
      partial_bytes(batch, num_kv_heads, max_seq_len) > kScratchBytes)
    return OXR_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  const int st = scratch_address(&ws);
  if (st) return st;
  return oxr_qk_norm_rope_paged_extend(qkv, q_weight, k_weight, cos_table, sin_table, table_rows, positions, eps,
                                       k_cache, v_cache, slots, num_slots, seq_lens, block_table, table_stride, batch,
                                       tokens_per_seq, num_heads, num_kv_heads, head_dim, block_size, num_blocks,
                                       max_seq_len, scale, out, out_packed, ws, kScratchBytes, stream);
}
