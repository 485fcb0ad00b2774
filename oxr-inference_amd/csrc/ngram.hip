// Batched n-gram suffix-match drafting (gfx950).
//
// Replaces the per-sequence Python dict of oxr_runtime/speculative.py:15-39.
// The dict maps every n-gram (n = 1..max_n) ending just before position p to
// the latest such p, and propose() looks up the history's own suffix, longest
// n first.  That is the same as: over all candidates p in [1, L-1] let m(p) be
// how many tokens before p match the suffix (capped at min(max_n, p)); the
// answer is the largest m(p) and, among those, the largest p.  So the kernel
// maximises the key (m(p), p).
//
// One 256-thread workgroup per sequence scans candidates from the end of the
// history backwards in chunks of up to 4096.  A chunk's window of history
// (4096 + max_n tokens) is staged in LDS in one round of coalesced loads, so a
// typical history costs one memory latency.  Each wave then walks its own
// 64-candidate tiles of the chunk (tile w, w + 4, ... from the top, one
// candidate per lane): every lane computes m(p) from LDS, and a ballot per n
// (longest first, only lengths that beat the wave's best so far) plus
// find-last-set picks the latest p.  The four waves combine through LDS once
// per chunk.  A wave stops at a full-length match, and so does the scan:
// nothing earlier can beat it.
#include "common.h"

namespace oxr {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxN = 8;
constexpr int kMaxDraft = 64;
constexpr int kChunk = 4096;  // candidates per LDS-staged chunk (16 KiB)
constexpr int kStage = (kChunk + kMaxN + kThreads - 1) / kThreads;  // history tokens each thread stages

// Where the verify inputs go when drafting also assembles them (engine.py:700-710).
struct VerifyInputs {
  const int32_t* seq_len;      // [B] KV length before the step (the reference's seq.length)
  const int32_t* block_table;  // [B, table_stride]
  int64_t table_stride;
  int block_size;
  int tokens_per_seq;  // S = 1 + k
  int64_t* ids;        // [B * S]
  int64_t* positions;  // [B * S]
  int64_t* slots;      // [B * S]
  int32_t* attn_seq_lens;  // [B] seq_len + S
  const int32_t* max_tokens;  // optional [B]: generated-token limit of each sequence
  int max_positions;          // > 0: the position table's size
};

template <bool kAssemble>
__global__ __launch_bounds__(kThreads) void ngram_propose_kernel(const int32_t* __restrict__ history,
                                                                 int64_t stride, const int32_t* __restrict__ hist_len,
                                                                 const int32_t* __restrict__ index_len, int max_n,
                                                                 int k, const int32_t* __restrict__ k_limit,
                                                                 int32_t* __restrict__ draft,
                                                                 int32_t* __restrict__ draft_len, VerifyInputs vi) {
  __shared__ int32_t window[kChunk + kMaxN];
  __shared__ int32_t wave_n[kThreads / kWave];
  __shared__ int32_t wave_p[kThreads / kWave];

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int32_t* h = history + (int64_t)b * stride;
  const int L = (int)min((int64_t)max(hist_len[b], 0), stride);  // never read past the row
  const int nmax = min(max_n, L);
  // Candidates are positions 1..last; `index_len` (optional) limits them to
  // the prefix that has been indexed, as a proposer built on a shorter list.
  int last = L - 1;
  if (index_len) last = min(last, index_len[b] - 1);

  int suffix[kMaxN];
#pragma unroll
  for (int i = 0; i < kMaxN; ++i) suffix[i] = (i < nmax) ? h[L - 1 - i] : 0;

  // The verify row's positions and slots do not depend on the drafts: thread j < S
  // looks up its slot now, while the history loads are in flight.
  int base_len = 0;
  int64_t my_slot = -1;
  if constexpr (kAssemble) {
    base_len = vi.seq_len[b];
    if (tid < vi.tokens_per_seq) {
      const int64_t pos = (int64_t)base_len + tid;
      const int64_t blk = pos / vi.block_size;
      if (pos >= 0 && blk < vi.table_stride) {
        const int32_t page = vi.block_table[(int64_t)b * vi.table_stride + blk];
        if (page >= 0) my_slot = (int64_t)page * vi.block_size + pos % vi.block_size;
      }
    }
  }

  int best_n = 0, best_p = -1;
  for (int top = last; top >= 1 && nmax > 0; top -= kChunk) {
    const int base = top - (kChunk - 1);  // candidate at window index kMaxN (may be < 1)
    // Stage h[base - kMaxN, top) into LDS: every load is issued before any store.
    int32_t staged[kStage];
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int i = tid + u * kThreads;
      const int pos = base - kMaxN + i;
      staged[u] = (i < kChunk + kMaxN && pos >= 0 && pos < L) ? h[pos] : 0;
    }
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int i = tid + u * kThreads;
      if (i < kChunk + kMaxN) window[i] = staged[u];
    }
    __syncthreads();

    // This wave's tiles, from the top down.  Within a wave a lower tile only wins
    // with a strictly longer match, so the ballots test only such lengths.
    int wn = 0, wp = -1;
    for (int t = wave; t < kChunk / kWave; t += kThreads / kWave) {
      const int p0 = top - kWave * t - (kWave - 1);  // candidate of lane 0
      if (p0 + kWave - 1 < 1) break;                // wave-uniform: below candidate 1
      const int p = p0 + lane;
      int m = 0;
      if (p >= 1) {
        const int cap = min(nmax, p);
#pragma unroll
        for (int i = 0; i < kMaxN; ++i) {
          if (i >= cap || m != i) break;
          // h[p - 1 - i] sits at window index (p - 1 - i) - (base - kMaxN).
          if (window[p - 1 - i - base + kMaxN] == suffix[i]) m = i + 1;
        }
      }
      for (int n = nmax; n > wn; --n) {
        const unsigned long long mask = __ballot(m >= n);
        if (mask) {
          wn = n;
          wp = p0 + (63 - __clzll(mask));
          break;
        }
      }
      if (wn == nmax) break;  // nothing lower in this wave beats a full-length match
    }
    if (lane == 0) {
      wave_n[wave] = wn;
      wave_p[wave] = wp;
    }
    __syncthreads();
    int tn = 0, tp = -1;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) {
      if (wave_n[w] > tn || (wave_n[w] == tn && wave_n[w] > 0 && wave_p[w] > tp)) {
        tn = wave_n[w];
        tp = wave_p[w];
      }
    }
    // Later chunks already hold the latest p for any length they matched, so an
    // earlier chunk only wins with a strictly longer match.
    if (tn > best_n) {
      best_n = tn;
      best_p = tp;
    }
    __syncthreads();  // window / wave_* are rewritten by the next chunk
    if (best_n == nmax) break;
  }

  int kb = k;
  if (k_limit) kb = max(0, min(k, k_limit[b]));
  if constexpr (kAssemble) {
    // Room left for drafts (engine.py:683-684): the accepted drafts plus the model's own token
    // must stay within max_tokens, and the step's positions within max_positions.
    if (vi.max_tokens) kb = max(0, min(kb, vi.max_tokens[b] - L - 1));
    if (vi.max_positions > 0) kb = max(0, min(kb, vi.max_positions - vi.seq_len[b] - 1));
  }
  int len = 0;
  if (best_n > 0) len = min(kb, L - best_p);
  for (int j = tid; j < k; j += kThreads) draft[(int64_t)b * k + j] = (j < len) ? h[best_p + j] : 0;
  if (tid == 0) draft_len[b] = len;

  if constexpr (kAssemble) {
    // Row b of the verify batch: [pending token, *draft, 0-padding], each at
    // position seq_len + j and slot slot_of(blocks, seq_len + j)
    // (engine.py:700-710, language.py:320-322).  A position past the block
    // table, or on a negative (unallocated) table entry, gets slot -1, which
    // the KV write skips.
    const int S = vi.tokens_per_seq;  // <= kThreads (checked on the host)
    if (tid < S) {
      const int j = tid;
      int64_t id = 0;
      if (j == 0) id = (L > 0) ? h[L - 1] : 0;
      else if (j - 1 < len) id = h[best_p + j - 1];
      const int64_t row = (int64_t)b * S + j;
      vi.ids[row] = id;
      vi.positions[row] = (int64_t)base_len + j;
      vi.slots[row] = my_slot;
    }
    if (tid == 0) vi.attn_seq_lens[b] = base_len + S;
  }
}

}  // namespace
}  // namespace oxr

extern "C" int oxr_ngram_propose(const int32_t* history, int64_t history_stride, const int32_t* history_len,
                                 const int32_t* index_len, int32_t batch, int32_t max_n, int32_t k,
                                 const int32_t* k_limit, int32_t* draft, int32_t* draft_len, oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(batch < 0 || k < 0 || history_stride < 0, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(max_n < 1 || max_n > kMaxN || k > kMaxDraft, OXR_ERR_UNSUPPORTED);
  if (batch == 0) return OXR_OK;
  OXR_RETURN_IF(!history || !history_len || !draft_len || (k > 0 && !draft), OXR_ERR_INVALID_ARG);
  hipLaunchKernelGGL(ngram_propose_kernel<false>, dim3(batch), dim3(kThreads), 0, (hipStream_t)stream, history,
                     history_stride, history_len, index_len, max_n, k, k_limit, draft, draft_len, VerifyInputs{});
  return OXR_LAUNCH_STATUS();
}

extern "C" int oxr_propose_verify_inputs(const int32_t* history, int64_t history_stride,
                                         const int32_t* history_len, int32_t batch, int32_t max_n, int32_t k,
                                         const int32_t* k_limit, const int32_t* seq_len, const int32_t* block_table,
                                         int64_t table_stride, int32_t block_size, int32_t tokens_per_seq,
                                         const int32_t* max_tokens, int32_t max_positions, int32_t* draft,
                                         int32_t* draft_len, int64_t* ids, int64_t* positions, int64_t* slots,
                                         int32_t* attn_seq_lens, oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(batch < 0 || k < 0 || history_stride < 0 || table_stride < 0 || block_size <= 0,
                OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(tokens_per_seq < k + 1, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(tokens_per_seq > kThreads, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(max_n < 1 || max_n > kMaxN || k > kMaxDraft, OXR_ERR_UNSUPPORTED);
  if (batch == 0) return OXR_OK;
  OXR_RETURN_IF(!history || !history_len || !draft_len || (k > 0 && !draft) || !seq_len || !block_table || !ids ||
                    !positions || !slots || !attn_seq_lens,
                OXR_ERR_INVALID_ARG);
  VerifyInputs vi{seq_len, block_table, table_stride, block_size, tokens_per_seq, ids, positions, slots,
                  attn_seq_lens, max_tokens, max_positions};
  hipLaunchKernelGGL(ngram_propose_kernel<true>, dim3(batch), dim3(kThreads), 0, (hipStream_t)stream, history,
                     history_stride, history_len, nullptr, max_n, k, k_limit, draft, draft_len, vi);
  return OXR_LAUNCH_STATUS();
}
