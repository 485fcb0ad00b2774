// Variable-length (prefill) attention on gfx950: the drop-in for
// attention.varlen (oxr_runtime/attention.py:47-59).
//
// Several sequences are concatenated along the token axis: q [T, H, 128],
// k/v [T, KV, 128] bf16, cu_seqlens int32 [n + 1] (sequence i is tokens
// [cu[i], cu[i+1])).  Within each sequence, query token j of q head h attends
// keys [0, j] (causal) or all keys (bidirectional) of kv head h / (H / KV);
// scores q.k * scale, fp32 softmax, bf16 output [T, H, 128].
//
// Prefill attention is MFMA-bound (Θ(len²) work per sequence), so the keys are
// staged once per workgroup in LDS and shared by every query row of the
// workgroup, and the products use the 32x32x16 MFMA, which reads half the LDS
// bytes per flop of the 16x16x32 one (LDS read bandwidth is the next limit):
// * A workgroup is 4 waves covering 128 query rows: the G = H / KV q heads of
//   one kv head, 128 / G consecutive positions each; wave w owns rows
//   32w .. 32w + 31 (one per MFMA column; row rho is head slot rho / (128 / G),
//   position q0 + rho % (128 / G)).
// * Key tiles of 64 rows go from memory straight into LDS (gfx950's 16-byte
//   global_load_lds: no staging registers, no LDS store instructions),
//   double-buffered: tile t + 1 is in flight while tile t is multiplied.  Rows
//   are unpadded with rotated 16-byte chunks, which gives the fragment reads
//   the banks of 68-dword (K) and 80-dword (V) row pitches, measured free of
//   bank conflicts on gfx950 for exactly these patterns.
// * Per wave and tile: S^T = K Q^T (16 MFMAs: 2 key blocks x 8 dim steps;
//   lane (n, h) holds keys 32kb + 8(v/4) + 4h + v%4 for query n), an
//   exp2-domain online softmax, then O^T += V^T P^T (16 MFMAs: 4 dim blocks x
//   4 key steps; P^T is used as computed: k slot 8h + 4p + j of key step ks
//   stands for key 16ks + 8p + 4h + j).  The V^T fragments come from gfx950's
//   transposing LDS read (ds_read_b64_tr_b16) of the row-major V tile.  The
//   QK^T products of tile t + 1 are issued among tile t's exponentials (K is
//   staged one tile ahead of V), so the matrix cores and the vector unit of a
//   wave overlap.
// * Causal: key tiles above a wave's last row are skipped, tiles that cross a
//   row's diagonal are masked per element; keys past the sequence are masked.
// Causal prefill runs this 4-wave kernel as a persistent launch whose
// workgroups take query tiles from shared lists.  Bidirectional prefill runs
// the 8-wave ping-pong kernel further down (same tiles and products, its two
// wave groups alternating softmax and MFMA phases on each SIMD).
#include <algorithm>
#include <atomic>

#include "common.h"

namespace oxr {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kVD = 128;               // head dim
constexpr int kVWaves = 4;             // waves per workgroup
constexpr int kVRows = 32 * kVWaves;   // query rows per workgroup (all q heads of the kv head)
constexpr int kKeyTile = 64;           // keys per LDS stage
constexpr int kLoadsPerWave = kKeyTile * kVD * 2 / 1024 / kVWaves;  // 1 KiB direct-to-LDS loads per wave and tensor
constexpr int kPersistentSlots = 64;   // persistent causal launch: workgroups per XCD (two per CU)

// Work counters of the persistent causal launch, per launch slot (the host cycles through
// kSchedRing of them, so launches in flight at once on different streams use different counters):
// for each of the 8 XCD groups the next item of its list to hand out, then the workgroups that have
// finished.  The launch's last workgroup to finish zeroes them all, so every launch finds them at zero
// (they are zero when the module loads).  System-scope atomics: performed coherently for the whole
// device, so a workgroup may take items from any group's list.
constexpr int kSchedRing = 16;
constexpr int kSchedStride = 32;              // uint32 words per counter (a 128-byte line each)
constexpr int kSchedWords = 9 * kSchedStride;  // per launch slot
__device__ uint32_t g_varlen_sched[kSchedRing * kSchedWords];

__device__ __forceinline__ uint32_t sched_take(uint32_t* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ f32x16 mfma_32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16).  Within each group of 16 lanes,
// lane 4a + b receives element b of the 4 bf16 addressed by lanes a, a + 4,
// a + 8 and a + 12 of its group, in that order.
__device__ __forceinline__ u32x2 lds_read_tr16(const bf16_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (v4s __attribute__((address_space(3)))*)(const_cast<bf16_t*>(p)));
  return __builtin_bit_cast(u32x2, x);
}

// Maximum of the 32 scores of a lane, as three-input maxima (each a v_max3_f32).
__device__ __forceinline__ float row_max32(const f32x16 (&sv)[2]) {
  float a[11];
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const int x = 3 * i, y = 3 * i + 1, z = 3 * i + 2;
    a[i] = fmaxf(fmaxf(sv[x >> 4][x & 15], sv[y >> 4][y & 15]), sv[z >> 4][z & 15]);
  }
  a[10] = fmaxf(sv[1][14], sv[1][15]);
  const float b0 = fmaxf(fmaxf(a[0], a[1]), a[2]), b1 = fmaxf(fmaxf(a[3], a[4]), a[5]);
  const float b2 = fmaxf(fmaxf(a[6], a[7]), a[8]), b3 = fmaxf(a[9], a[10]);
  return fmaxf(fmaxf(b0, b1), fmaxf(b2, b3));
}

// One causal work item: query tile `qt` (128 / G positions of each of the G q heads) of (sequence, kv
// head) pair `pair`.  Every wave of the workgroup takes part (it ends with a workgroup barrier and touches
// no LDS after it, so the next item may start right away).  Thread 0 takes the next item number from
// the counter `ctr` into `next` when the item's last two key tiles begin (or at once if it has no
// work), late enough that the items are started in list order.
__device__ __forceinline__ void varlen_item(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                            const bf16_t* __restrict__ v, const int32_t* __restrict__ cu_seqlens,
                                            int H, int KV, float scale_log2, bf16_t* __restrict__ out, int pair,
                                            int qt, bf16_t* s_k0, bf16_t* s_k1, bf16_t* s_v0, bf16_t* s_v1,
                                            uint32_t* ctr, int* next) {
  const int seq = pair / KV, kvh = pair - seq * KV;
  const int start = cu_seqlens[seq], len = cu_seqlens[seq + 1] - start;
  const int G = H / KV, rph = kVRows / G;  // positions per head in this workgroup
  const int q0 = qt * rph;                 // first position, per head
  if (q0 >= len) {                         // whole workgroup: before any barrier
    if (threadIdx.x == 0) *next = (int)sched_take(ctr);
    return;
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, h = lane >> 5;
  const int rho = 32 * wave + n;
  const int head = kvh * G + rho / rph;
  const int qpos = q0 + rho % rph;  // query position of lane column n
  // The wave's positions: offsets first_off .. first_off + min(rph, 32) - 1 from q0.
  const int first_off = rph >= 32 ? (32 * wave) % rph : 0;
  const int wave_first = q0 + first_off;
  const int wave_last = min(wave_first + min(rph, 32) - 1, len - 1);

  // Q^T fragments (B operand): lane (n, h) holds Q[qpos][16i + 8h, +8) for dim step i.
  u32x4 qf[8];
  {
    const int qrow = min(qpos, len - 1);  // rows past the sequence compute and are never stored
    const bf16_t* src = q + ((int64_t)(start + qrow) * H + head) * kVD + 8 * h;
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[i] = ld128(src + 16 * i);
  }
  // Q lands here: otherwise the compiler sinks these loads past the first barrier and then, unable
  // to tell them from the key-tile prefetch, waits for every tile's prefetch before its first
  // product.
#pragma unroll
  for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(qf[i]));

  const int key_end = min(len, q0 + rph);  // keys this workgroup needs
  const int tiles = (key_end + kKeyTile - 1) / kKeyTile;

  // Key tiles go straight from memory to LDS (global_load_lds, 16 bytes per lane: lane i of an
  // instruction writes bytes [16i, 16i + 16) of a 1 KiB block, i.e. 4 rows of 256 bytes).  Rows
  // are stored without padding, their 16-byte chunks rotated instead: K row r holds chunk c at
  // position (c + r) mod 16, V row r at (c + 4r) mod 16.  That gives every fragment read below the
  // banks of a 68-dword (K) or 80-dword (V) row pitch, the ones measured free of conflicts for
  // these patterns.  Keys past the sequence re-read its last key (their scores are masked).
  auto dma = [&](const bf16_t* src, int t, bf16_t* dst, int rot) {
#pragma unroll
    for (int u = 0; u < kLoadsPerWave; ++u) {
      const int j = kLoadsPerWave * wave + u;  // 1 KiB block: rows 4j .. 4j + 3
      const int row = 4 * j + (lane >> 4), pos = lane & 15;
      const int key = min(t * kKeyTile + row, len - 1);
      const int64_t base = ((int64_t)(start + key) * KV + kvh) * kVD;
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(src + base + 8 * ((pos - rot * row) & 15)),
          (void __attribute__((address_space(3)))*)(dst + 512 * j), 16, 0, 0);
    }
  };

  float m_run = -INFINITY, mc_run = 0.f, l_run = 0.f;
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;

  // Transposing-read address of lane (n, h) for V^T fragment (dim block dt, key step ks, half p):
  // lane j of its 16-lane group addresses key 16ks + 8p + 4h + j / 4, dims 32dt + 16 (n / 16) + 4 (j % 4),
  // i.e. chunk 4dt + 2 (n / 16) + (j % 4) / 2 of its row, half (j % 2); the row's rotation is 4 tr_key
  // (mod 16) for every (ks, p).
  const int tr_key = 4 * h + ((lane & 15) >> 2);
  int tr_off[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
    tr_off[dt] = 8 * ((4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1) + 4 * tr_key) & 15) + 4 * (lane & 1);

  // Raw scores of one tile: sv[kb][v] is key 32kb + 8(v/4) + 4h + v%4 of the tile for query n.  The
  // two key blocks' chains alternate, so consecutive products are independent.
  auto qk = [&](const bf16_t* kb_, f32x16 (&sv)[2]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) sv[kb][e] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(kb_ + (32 * kb + n) * kVD + 8 * ((2 * i + h + n) & 15));
        sv[kb] = mfma_32x32x16(kf, qf[i], sv[kb]);
      }
  };

  // Tile t, software-pipelined by one tile: its scores `cur` were computed during tile t - 1; the
  // products for tile t + 1's scores `nxt` (K in kq) are issued among this tile's exponentials, so
  // the matrix cores work while the softmax runs on the vector unit.  K runs one tile ahead of V in
  // the double buffers: tile t prefetches K(t + 2) into kd and V(t + 1) into vd, the buffers read
  // during tile t - 1.  Past the last tile `nxt` is computed from a stale buffer and never used.
  auto step = [&](int t, f32x16 (&cur)[2], f32x16 (&nxt)[2], const bf16_t* kq, const bf16_t* vp_, bf16_t* kd,
                  bf16_t* vd) {
    if (t + 2 < tiles) dma(k, t + 2, kd, 1);
    if (t + 1 < tiles) dma(v, t + 1, vd, 4);
    const int kt0 = t * kKeyTile;
    if (kt0 <= wave_last) {  // wave-uniform: otherwise every key of this and later tiles is masked
      // wave-uniform: a tile crossing the diagonal of one of the wave's rows, or the sequence end
      const bool edge = kt0 + kKeyTile - 1 > wave_first || kt0 + kKeyTile > len;
      if (edge) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = kt0 + 32 * kb + 8 * (e >> 2) + 4 * h + (e & 3);
            if (key >= len || key > qpos) cur[kb][e] = -INFINITY;
          }
      }
      // Row maximum (exact in any order) as a tree of three-input maxima (v_max3_f32): 32 scores in
      // 16 instructions instead of 31.
      const float mx = xor32_max(row_max32(cur));
      const bool moved = mx > m_run;
      if (__builtin_amdgcn_ballot_w64(moved)) {
        const float m_new = moved ? mx : m_run;
        const float mc_new = m_new == -INFINITY ? 0.f : m_new * scale_log2;
        const float alpha = !moved ? 1.0f : (m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc_run - mc_new));
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        m_run = m_new;
        mc_run = mc_new;
      }
      qk(kq, nxt);
      // P^T for key step ks: accumulators 8 (ks % 2) .. +7 of key block ks / 2, in k-slot order.
      // The tile's probabilities are summed as a tree, then added to the running sum.
      u32x4 pb[4];
      float ps[16];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pv[e] = __builtin_amdgcn_exp2f(fmaf(cur[ks >> 1][8 * (ks & 1) + e], scale_log2, -mc_run));
#pragma unroll
        for (int e = 0; e < 4; ++e) ps[4 * ks + e] = pv[e] + pv[e + 4];
        pb[ks] = u32x4{pack_bf_hw(pv[0], pv[1]), pack_bf_hw(pv[2], pv[3]), pack_bf_hw(pv[4], pv[5]),
                       pack_bf_hw(pv[6], pv[7])};
      }
#pragma unroll
      for (int w2 = 8; w2 >= 1; w2 >>= 1)
#pragma unroll
        for (int e = 0; e < w2; ++e) ps[e] += ps[e + w2];
      l_run += ps[0];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16_t* vrow = vp_ + (16 * ks + tr_key) * kVD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const u32x2 lo = lds_read_tr16(vrow + tr_off[dt]);            // keys 16ks + 4h + (0..3)
          const u32x2 hi = lds_read_tr16(vrow + 8 * kVD + tr_off[dt]);  // keys 16ks + 8 + 4h + (0..3)
          o[dt] = mfma_32x32x16(u32x4{lo.x, lo.y, hi.x, hi.y}, pb[ks], o[dt]);
        }
      }
    }
    // This wave's prefetches have landed in LDS once its vector memory count drains; the barrier
    // publishes every wave's, and ends every read of the buffers the next tile prefetches into.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };

  f32x16 sa[2], sb[2];
  dma(k, 0, s_k0, 1);
  if (tiles > 1) dma(k, 1, s_k1, 1);
  dma(v, 0, s_v0, 4);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  qk(s_k0, sa);
  for (int t = 0; t < tiles; t += 2) {
    if (t + 2 >= tiles && threadIdx.x == 0) *next = (int)sched_take(ctr);
    step(t, sa, sb, s_k1, s_v0, s_k0, s_v1);
    if (t + 1 < tiles) step(t + 1, sb, sa, s_k0, s_v1, s_k1, s_v0);
  }

  // Normalise and store: lane (n, h) holds O^T[32dt + 8(e/4) + 4h + e%4][query n].
  const float l_tot = xor32_sum(l_run);
  if (qpos < len) {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    bf16_t* dst = out + ((int64_t)(start + qpos) * H + head) * kVD + 4 * h;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int m = 0; m < 4; ++m)
        *reinterpret_cast<u32x2*>(dst + 32 * dt + 8 * m) =
            u32x2{pack_bf(o[dt][4 * m] * inv, o[dt][4 * m + 1] * inv),
                  pack_bf(o[dt][4 * m + 2] * inv, o[dt][4 * m + 3] * inv)};
  }
}

// Causal prefill, persistent: 64 workgroups per XCD (two per CU) take items from lists through shared
// counters until every list runs out, so no CU waits for the dispatcher between items, and a workgroup
// that runs slower (measured: of two equal workgroups on one CU the younger one took 24% longer) takes
// fewer items.  XCD group x owns pairs [x n / 8, (x + 1) n / 8) of the n (sequence, kv head) pairs,
// listed two pairs at a time (their key tiles fit the XCD's L2), each two's query tiles latest first,
// so a list ends with its smallest items.  A workgroup starts on its own XCD's group (workgroup b runs
// on XCD b % 8, round-robin dispatch), asks for its next item near the end of its current one and
// reads the answer after the item's last barrier; once that list is done it takes the remaining items
// of the other groups' lists, in turn.  That balances the XCDs (measured: alone on their own lists,
// their mean end times spread from 646 to 694 us in a 705 us launch) and mixed sequence lengths, whose
// long sequences' pairs sit in few groups.
__global__ __launch_bounds__(64 * kVWaves, 2) void varlen_attention_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ cu_seqlens, int H, int KV, int num_qtiles, int num_pairs, int ring,
    float scale_log2, bf16_t* __restrict__ out) {
  // Two buffers per tensor, as separate arrays: the tile loop is unrolled by two, so each buffer is
  // named statically and the compiler can tell a prefetch into one from reads of the other (members
  // of one array or struct, addressed per wave, it cannot: it then waits for every prefetch before
  // each tile's first LDS read).
  __shared__ bf16_t s_k0[kKeyTile * kVD], s_k1[kKeyTile * kVD];
  __shared__ bf16_t s_v0[kKeyTile * kVD], s_v1[kKeyTile * kVD];
  // Item numbers pass through LDS, alternating between two words: a word is rewritten two numbers
  // later, after a barrier that every wave reaches only once it has read the word.
  __shared__ int s_item[2];
  const int total = (int)gridDim.x;
  uint32_t* const base = g_varlen_sched + ring * kSchedWords;
  int grp = (int)blockIdx.x & 7, tried = 0, r = 0;
  // Group grp's pairs [lo, lo + cnt) and list length.
  int lo = 0, cnt = 0, items = 0;
  auto group = [&]() {
    lo = (int)((int64_t)grp * num_pairs / 8);
    cnt = (int)((int64_t)(grp + 1) * num_pairs / 8) - lo;
    items = cnt * num_qtiles;
  };
  group();
  if (threadIdx.x == 0) s_item[0] = (int)sched_take(base + grp * kSchedStride);
  __syncthreads();
  int i = s_item[0];
  while (true) {
    if (i >= items) {
      // This group's list is done: take from the next group's.
      if (++tried == 8) break;
      grp = (grp + 1) & 7;
      group();
      ++r;
      if (threadIdx.x == 0) s_item[r & 1] = (int)sched_take(base + grp * kSchedStride);
      __syncthreads();
      i = s_item[r & 1];
      continue;
    }
    int next = 0;
    const int g = i / (2 * num_qtiles), gp = min(2, cnt - 2 * g), j = i - g * 2 * num_qtiles;
    varlen_item(q, k, v, cu_seqlens, H, KV, scale_log2, out, lo + 2 * g + j % gp,
                         num_qtiles - 1 - j / gp, s_k0, s_k1, s_v0, s_v1, base + grp * kSchedStride, &next);
    ++r;
    if (threadIdx.x == 0) s_item[r & 1] = next;
    __syncthreads();
    i = s_item[r & 1];
  }
  // Every workgroup of the launch has taken its last number once all have counted themselves out.
  if (threadIdx.x == 0 && sched_take(base + 8 * kSchedStride) == (uint32_t)(total - 1)) {
    for (int x = 0; x <= 8; ++x)
      __hip_atomic_exchange(base + x * kSchedStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Ping-pong form: a workgroup of 8 waves covers 256 query rows; waves w and w + 4 run on the same
// SIMD.  Group A (waves 0-3) and group B (waves 4-7) alternate between a vector phase (the online
// softmax of a tile's scores) and a matrix phase (PV of that tile, QK^T of the next), in opposite
// phases, with a workgroup barrier between phases, so each SIMD has one wave issuing exponentials
// while the other issues MFMAs.  Phases, for tile t:
//   phase 2t + 1: loads of V(t + 1) and K(t + 2) start; A: PV(t), QK(t + 1); B: softmax(t)
//   phase 2t + 2: A: softmax(t + 1); B: PV(t), QK(t + 1); then every wave waits for its loads
// so V(t) and K(t + 1) are read in phases 2t + 1 and 2t + 2 and their buffers are refilled at the
// start of phase 2t + 3, after both reads.
constexpr int kPWaves = 8;
constexpr int kPRows = 32 * kPWaves;  // query rows per workgroup
constexpr int kPLoadsPerWave = kKeyTile * kVD * 2 / 1024 / kPWaves;

template <bool kCausal>
__global__ __launch_bounds__(64 * kPWaves, 1) void varlen_attention_pp_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ cu_seqlens, int H, int KV, int num_qtiles, float scale_log2,
    bf16_t* __restrict__ out) {
  __shared__ bf16_t s_k0[kKeyTile * kVD], s_k1[kKeyTile * kVD];
  __shared__ bf16_t s_v0[kKeyTile * kVD], s_v1[kKeyTile * kVD];

  // Work item order as in varlen_attention_kernel (XCD-contiguous items, late query tiles first).
  const int total = (int)gridDim.x, xcd = (int)blockIdx.x & 7, slot = (int)blockIdx.x >> 3;
  const int w = xcd * (total >> 3) + min(xcd, total & 7) + slot;
  const int pair = w / num_qtiles;
  const int seq = pair / KV, kvh = pair - seq * KV;
  const int start = cu_seqlens[seq], len = cu_seqlens[seq + 1] - start;
  const int G = H / KV, rph = kPRows / G;
  const int q0 = (num_qtiles - 1 - (w - pair * num_qtiles)) * rph;
  if (q0 >= len) return;  // whole workgroup: before any barrier

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool group_a = wave < kPWaves / 2;
  const int n = lane & 31, h = lane >> 5;
  const int rho = 32 * wave + n;
  const int head = kvh * G + rho / rph;
  const int qpos = q0 + rho % rph;
  const int first_off = rph >= 32 ? (32 * wave) % rph : 0;
  const int wave_first = q0 + first_off;
  const int wave_last = kCausal ? min(wave_first + min(rph, 32) - 1, len - 1) : len - 1;

  u32x4 qf[8];
  {
    const int qrow = min(qpos, len - 1);
    const bf16_t* src = q + ((int64_t)(start + qrow) * H + head) * kVD + 8 * h;
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[i] = ld128(src + 16 * i);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(qf[i]));

  const int key_end = kCausal ? min(len, q0 + rph) : len;
  const int tiles = (key_end + kKeyTile - 1) / kKeyTile;

  // Direct-to-LDS tile loads, rotated rows as in varlen_attention_kernel; kPLoadsPerWave 1 KiB
  // blocks per wave and tensor.
  auto dma = [&](const bf16_t* src, int t, bf16_t* dst, int rot) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kPLoadsPerWave; ++u) {
      const int j = kPLoadsPerWave * wave + u;
      const int row = 4 * j + (lane >> 4), pos = lane & 15;
      const int key = min(t * kKeyTile + row, len - 1);
      const int64_t base = ((int64_t)(start + key) * KV + kvh) * kVD;
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(src + base + 8 * ((pos - rot * row) & 15)),
          (void __attribute__((address_space(3)))*)(dst + 512 * j), 16, 0, 0);
    }
  };

  float m_run = -INFINITY, mc_run = 0.f, l_run = 0.f;
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  const int tr_key = 4 * h + ((lane & 15) >> 2);
  int tr_off[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
    tr_off[dt] = 8 * ((4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1) + 4 * tr_key) & 15) + 4 * (lane & 1);

  f32x16 sv[2];  // scores of the tile whose softmax is next
  u32x4 pb[4];   // P^T of the tile whose PV is next
  // A tile is skipped by a wave when all of its keys are past the wave's last row (wave-uniform).
  auto live = [&](int t) __attribute__((always_inline)) { return t >= 0 && t < tiles && t * kKeyTile <= wave_last; };

  // Matrix phase of tile t: PV(t) from vb (V(t)), then QK^T of tile t + 1 from kb (K(t + 1)).  The
  // LDS fragments are read one step ahead of their products (one step: a V key step, a K dim step),
  // with a scheduling barrier per step: left alone, the compiler issues all 48 reads first and needs
  // 128 more registers than the wave has.
  auto vread = [&](const bf16_t* vb, int ks, u32x2 (&d)[4][2]) __attribute__((always_inline)) {
    const bf16_t* vrow = vb + (16 * ks + tr_key) * kVD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      d[dt][0] = lds_read_tr16(vrow + tr_off[dt]);            // keys 16ks + 4h + (0..3)
      d[dt][1] = lds_read_tr16(vrow + 8 * kVD + tr_off[dt]);  // keys 16ks + 8 + 4h + (0..3)
    }
  };
  auto kread = [&](const bf16_t* kb_, int i, u32x4 (&d)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      d[kb] = *reinterpret_cast<const u32x4*>(kb_ + (32 * kb + n) * kVD + 8 * ((2 * i + h + n) & 15));
  };
  auto matrix_phase = [&](int t, const bf16_t* kb, const bf16_t* vb) __attribute__((always_inline)) {
    const bool pv = live(t), next = live(t + 1);
    u32x4 kr[2][2];
    if (pv) {
      u32x2 vr[2][4][2];
      vread(vb, 0, vr[0]);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks < 3) vread(vb, ks + 1, vr[(ks + 1) & 1]);
        else if (next) {
          kread(kb, 0, kr[0]);
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const u32x2 lo = vr[ks & 1][dt][0], hi = vr[ks & 1][dt][1];
          o[dt] = mfma_32x32x16(u32x4{lo.x, lo.y, hi.x, hi.y}, pb[ks], o[dt]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if (next) {
      kread(kb, 0, kr[0]);
    }
    if (next) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int e = 0; e < 16; ++e) sv[kb2][e] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i + 1 < 8) kread(kb, i + 1, kr[(i + 1) & 1]);
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2) sv[kb2] = mfma_32x32x16(kr[i & 1][kb2], qf[i], sv[kb2]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // Vector phase of tile t: mask, online softmax, P^T packed for the next matrix phase.
  auto vector_phase = [&](int t) __attribute__((always_inline)) {
    if (!live(t)) return;
    const int kt0 = t * kKeyTile;
    const bool edge = (kCausal && kt0 + kKeyTile - 1 > wave_first) || kt0 + kKeyTile > len;
    if (edge) {
      // Key kt0 + 4h + c with c = 32kb + 8(e / 4) + e % 4 a constant: compared against two per-tile
      // limits, so no per-element lane offsets are kept in registers across tiles.
      const int lim_len = len - kt0 - 4 * h, lim_q = qpos - kt0 - 4 * h;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int c = 32 * kb + 8 * (e >> 2) + (e & 3);
          if (c >= lim_len || (kCausal && c > lim_q)) sv[kb][e] = -INFINITY;
        }
    }
    const float mx = xor32_max(row_max32(sv));
    const bool moved = mx > m_run;
    if (__builtin_amdgcn_ballot_w64(moved)) {
      const float m_new = moved ? mx : m_run;
      const float mc_new = m_new == -INFINITY ? 0.f : m_new * scale_log2;
      const float alpha = !moved ? 1.0f : (m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc_run - mc_new));
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
      m_run = m_new;
      mc_run = mc_new;
    }
    float ps[16];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pv[e] = __builtin_amdgcn_exp2f(fmaf(sv[ks >> 1][8 * (ks & 1) + e], scale_log2, -mc_run));
#pragma unroll
      for (int e = 0; e < 4; ++e) ps[4 * ks + e] = pv[e] + pv[e + 4];
      pb[ks] = u32x4{pack_bf_hw(pv[0], pv[1]), pack_bf_hw(pv[2], pv[3]), pack_bf_hw(pv[4], pv[5]),
                     pack_bf_hw(pv[6], pv[7])};
    }
#pragma unroll
    for (int w2 = 8; w2 >= 1; w2 >>= 1)
#pragma unroll
      for (int e = 0; e < w2; ++e) ps[e] += ps[e + w2];
    l_run += ps[0];
  };
  // The barrier between phases orders LDS reads before the refills of later phases; its memory
  // clobber keeps LDS accesses on their side.  Only the end of an even phase waits for this wave's
  // tile loads (a fence or __syncthreads would wait for them at every barrier).
  auto phase_end = [&](bool wait_loads) __attribute__((always_inline)) {
    if (wait_loads) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
  };
  // Phase 2t + 1 and phase 2t + 2, with the buffers named statically: K(t + 1) in kb, V(t) in vb,
  // and the loads of K(t + 2) into kd, V(t + 1) into vd.  Each group runs its own loop (its phases in
  // its own order), so the register allocator sees one straight sequence per group; both loops pass
  // the same barriers, two per tile.
  auto loads = [&](int t, bf16_t* kd, bf16_t* vd) __attribute__((always_inline)) {
    if (t + 1 < tiles) dma(v, t + 1, vd, 4);
    if (t + 2 < tiles) dma(k, t + 2, kd, 1);
  };
  auto iteration_a = [&](int t, const bf16_t* kb, const bf16_t* vb, bf16_t* kd, bf16_t* vd)
                         __attribute__((always_inline)) {
    loads(t, kd, vd);
    matrix_phase(t, kb, vb);
    phase_end(false);
    vector_phase(t + 1);
    phase_end(true);
  };
  auto iteration_b = [&](int t, const bf16_t* kb, const bf16_t* vb, bf16_t* kd, bf16_t* vd)
                         __attribute__((always_inline)) {
    loads(t, kd, vd);
    vector_phase(t);
    phase_end(false);
    matrix_phase(t, kb, vb);
    phase_end(true);
  };

  // Prologue: K(0) in; phase -1 (A: QK(0); V(0) and K(1) start loading); phase 0 (A: softmax(0);
  // B: QK(0)).
  dma(k, 0, s_k0, 1);
  phase_end(true);
  if (0 < tiles) dma(v, 0, s_v0, 4);
  if (1 < tiles) dma(k, 1, s_k1, 1);
  if (group_a) {
    matrix_phase(-1, s_k0, s_v0);  // QK(0) only
    phase_end(false);
    vector_phase(0);
    phase_end(true);
    for (int t = 0; t < tiles; t += 2) {
      iteration_a(t, s_k1, s_v0, s_k0, s_v1);
      if (t + 1 < tiles) iteration_a(t + 1, s_k0, s_v1, s_k1, s_v0);
    }
  } else {
    phase_end(false);
    matrix_phase(-1, s_k0, s_v0);
    phase_end(true);
    for (int t = 0; t < tiles; t += 2) {
      iteration_b(t, s_k1, s_v0, s_k0, s_v1);
      if (t + 1 < tiles) iteration_b(t + 1, s_k0, s_v1, s_k1, s_v0);
    }
  }

  const float l_tot = xor32_sum(l_run);
  if (qpos < len) {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    bf16_t* dst = out + ((int64_t)(start + qpos) * H + head) * kVD + 4 * h;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int m = 0; m < 4; ++m)
        *reinterpret_cast<u32x2*>(dst + 32 * dt + 8 * m) =
            u32x2{pack_bf(o[dt][4 * m] * inv, o[dt][4 * m + 1] * inv),
                  pack_bf(o[dt][4 * m + 2] * inv, o[dt][4 * m + 3] * inv)};
  }
}

}  // namespace
}  // namespace oxr

extern "C" int oxr_varlen_attention(const oxr_bf16* q, const oxr_bf16* k, const oxr_bf16* v,
                                    const int32_t* cu_seqlens, int32_t num_seqs, int32_t max_len,
                                    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t causal,
                                    float scale, oxr_bf16* out, oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(num_seqs < 0 || max_len < 0 || num_heads <= 0 || num_kv_heads <= 0, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(head_dim != kVD || num_heads % num_kv_heads != 0, OXR_ERR_UNSUPPORTED);
  const int G = num_heads / num_kv_heads;
  OXR_RETURN_IF(8 % G != 0, OXR_ERR_UNSUPPORTED);  // G in {1, 2, 4, 8}
  if (num_seqs == 0 || max_len == 0) return OXR_OK;
  OXR_RETURN_IF(!q || !k || !v || !cu_seqlens || !out, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 != 0 || (uintptr_t)out % 8 != 0,
                OXR_ERR_UNSUPPORTED);
  // Bidirectional prefill runs the ping-pong kernel; its causal form needs more registers than two
  // waves per SIMD have (it spills), so causal prefill runs the persistent 4-wave kernel.
  const int rows_per_head = (causal ? kVRows : kPRows) / G;
  const int num_qtiles = (max_len + rows_per_head - 1) / rows_per_head;
  // Item numbers are int: the counters run past a list's end by at most one number per workgroup and
  // group, so the lists keep that much headroom below INT32_MAX.
  OXR_RETURN_IF((int64_t)num_qtiles * num_kv_heads * num_seqs > INT32_MAX - 8 * 8 * kPersistentSlots,
                OXR_ERR_UNSUPPORTED);
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  const int num_pairs = num_seqs * num_kv_heads;
  if (!causal) {
    const dim3 grid((unsigned)(num_qtiles * num_pairs));
    hipLaunchKernelGGL(varlen_attention_pp_kernel<false>, grid, dim3(64 * kPWaves), 0, s, q, k, v, cu_seqlens,
                       num_heads, num_kv_heads, num_qtiles, scale_log2, out);
  } else {
    // Two workgroups per CU, or fewer when the largest XCD group has fewer items.
    static std::atomic<uint32_t> launches{0};
    const int ring = (int)(launches.fetch_add(1u, std::memory_order_relaxed) % kSchedRing);
    const int per_xcd = (int)std::min<int64_t>(kPersistentSlots, (int64_t)((num_pairs + 7) / 8) * num_qtiles);
    hipLaunchKernelGGL(varlen_attention_kernel, dim3(8 * per_xcd), dim3(64 * kVWaves), 0, s, q, k, v, cu_seqlens,
                       num_heads, num_kv_heads, num_qtiles, num_pairs, ring, scale_log2, out);
  }
  return OXR_LAUNCH_STATUS();
}
