// Longest-prefix greedy acceptance and length rollback (gfx950).
//
// Replaces speculative.accept (oxr_runtime/speculative.py:42-48) and the
// bookkeeping after it in Engine._speculate / _take (engine.py:729-737,
// 647-664):
//   a        = longest j-prefix with draft[j] == predicted[j]   (j < draft_len)
//   taken    = draft[:a] + [predicted[a]] = predicted[0 .. a]
//   seq_len += a + 1                      (the KV "rollback": nothing is moved;
//                                          rejected slots keep the verify-step
//                                          K/V and are overwritten later)
//   history.append(t) for t in taken, stopping at EOS (not appended, finish
//   reason 1) or when the history reaches max_tokens (appended, reason 2).
// One lane per sequence: the work is a few dozen integer compares.
//
// argmax_accept_kernel does the same after finishing the LM head's argmax
// itself (the cross-workgroup reduction of argmax_reduce_kernel), so the
// verify step's greedy ids go from the LM head's per-workgroup keys to the
// accepted run in one launch.
#include <algorithm>

#include "common.h"
#include "lm_head_keys.h"

namespace oxr {
namespace {

constexpr int kPre = 8;             // drafts and predictions loaded before the first compare
constexpr int kMaxTokensPerSeq = 256;  // verify rows per sequence (the row assembly's limit)

// Everything after the loads: the accepted run, committed ids, length and history.  pv[j]
// (j <= kPre) are the first predictions, pred_at(j) gives any prediction (used past kPre).
template <class PredAt>
__device__ __forceinline__ void accept_sequence(int b, int32_t fin, int n_raw, const int32_t* d, const int32_t (&dv)[kPre],
                                                const int64_t (&pv)[kPre + 1], PredAt pred_at, int32_t len0,
                                                int32_t cap, int32_t sl, int k, int S, int eos_id,
                                                const int32_t* __restrict__ max_tokens, int32_t* __restrict__ accepted,
                                                int32_t* __restrict__ committed, int32_t* __restrict__ num_committed,
                                                int32_t* __restrict__ seq_len, int32_t* __restrict__ history,
                                                int64_t history_stride, int32_t* __restrict__ history_len,
                                                int32_t* __restrict__ finished) {
  if (fin != 0) {  // a finished sequence takes no tokens
    accepted[b] = 0;
    if (num_committed) num_committed[b] = 0;
    if (committed)
      for (int j = 0; j <= k; ++j) committed[(int64_t)b * (k + 1) + j] = -1;
    return;
  }
  const int n = min(max(n_raw, 0), min(k, S - 1));
  int a = 0;
#pragma unroll
  for (int j = 0; j < kPre; ++j)
    if (a == j && a < n && (int64_t)dv[j] == pv[j]) ++a;
  while (a >= kPre && a < n && (int64_t)d[a] == pred_at(a)) ++a;  // drafts beyond the preloaded ones
  accepted[b] = a;
  if (num_committed) num_committed[b] = a + 1;
  // Token j of the committed run is pv[j] for j <= kPre (static indices only: a dynamically
  // indexed register array would be placed in scratch memory), else pred_at(j).
  if (committed) {
    int32_t* const row = committed + (int64_t)b * (k + 1);
#pragma unroll
    for (int j = 0; j <= kPre; ++j)
      if (j <= k) row[j] = (j <= a) ? (int32_t)pv[j] : -1;
    for (int j = kPre + 1; j <= k; ++j) row[j] = (j <= a) ? (int32_t)pred_at(j) : -1;
  }
  if (seq_len) seq_len[b] = sl + a + 1;
  if (history) {
    int len = len0;
    int reason = 0;
    bool stop = false;
    auto take = [&](int32_t t) {  // history.append with the engine's stop rules
      if (t == eos_id) {
        reason = 1;
        stop = true;
        return;
      }
      if (len >= history_stride) {  // buffer full: stop as a length finish
        reason = 2;
        stop = true;
        return;
      }
      history[(int64_t)b * history_stride + len] = t;
      ++len;
      if (max_tokens && len >= cap) {
        reason = 2;
        stop = true;
      }
    };
#pragma unroll
    for (int j = 0; j <= kPre; ++j)
      if (!stop && j <= a) take((int32_t)pv[j]);
    for (int j = kPre + 1; !stop && j <= a; ++j) take((int32_t)pred_at(j));
    history_len[b] = len;
    if (finished) finished[b] = reason;
  }
}

__global__ __launch_bounds__(64) void accept_kernel(const int32_t* __restrict__ draft,
                                                    const int32_t* __restrict__ draft_len, int k,
                                                    const int64_t* __restrict__ predicted, int S, int batch,
                                                    int eos_id, const int32_t* __restrict__ max_tokens,
                                                    int32_t* __restrict__ accepted, int32_t* __restrict__ committed,
                                                    int32_t* __restrict__ num_committed,
                                                    int32_t* __restrict__ seq_len, int32_t* __restrict__ history,
                                                    int64_t history_stride, int32_t* __restrict__ history_len,
                                                    int32_t* __restrict__ finished) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  // Every input of this sequence is requested before any is used (one memory round trip):
  // the first kPre drafts and predictions, the lengths and the limits.
  // Loads are unconditional (a missing optional array reads draft_len[b] instead and the value is
  // discarded), so the compiler issues them together rather than one per branch.
  const int32_t* const any = draft_len + b;
  const int32_t fin_raw = *(finished ? finished + b : any);
  const int n_raw = draft_len[b];
  const int32_t* d = k > 0 ? draft + (int64_t)b * k : any;
  const int64_t* pred = predicted + (int64_t)b * S;
  int32_t dv[kPre];
  int64_t pv[kPre + 1];
#pragma unroll
  for (int j = 0; j < kPre; ++j) dv[j] = d[k > 0 ? min(j, k - 1) : 0];
#pragma unroll
  for (int j = 0; j <= kPre; ++j) pv[j] = pred[min(j, S - 1)];
  const int32_t len0_raw = *(history ? history_len + b : any);
  const int32_t cap_raw = *(max_tokens ? max_tokens + b : any);
  const int32_t sl_raw = *(seq_len ? seq_len + b : any);
  // Keep every load above ahead of the first use (the compiler would otherwise sink them past the
  // finished-sequence branch, one round trip each).
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::"v"(fin_raw), "v"(n_raw), "v"(len0_raw), "v"(cap_raw), "v"(sl_raw));
#pragma unroll
  for (int j = 0; j < kPre; ++j) asm volatile("" ::"v"(dv[j]));
#pragma unroll
  for (int j = 0; j <= kPre; ++j) asm volatile("" ::"v"(pv[j]));
  accept_sequence(b, finished ? fin_raw : 0, n_raw, d, dv, pv, [&](int j) { return pred[j]; },
                  history ? len0_raw : 0, max_tokens ? cap_raw : 0, seq_len ? sl_raw : 0, k, S, eos_id, max_tokens,
                  accepted, committed, num_committed, seq_len, history, history_stride, history_len, finished);
}

// One workgroup per sequence, one wave per verify row (rows w, w + W, ... for W = min(S, 16)
// waves).  A wave requests its row's keys (best[t * M + b * S + j], t < num_best: per LM-head
// workgroup the largest bf16 logit, then the lowest column, as argmax_key orders them), 4 per lane
// per round, while wave 0 requests the sequence's acceptance inputs; the row maximum is taken
// across the wave (the reduction of argmax_reduce_kernel, so the ids are the same), written to
// predicted and to LDS, and after one barrier thread 0 runs the acceptance on them.
constexpr int kMaxRowWaves = 16;
constexpr int kKeysPerLane = 4;  // 256 workgroups' keys per row in one round

__global__ __launch_bounds__(64 * kMaxRowWaves) void argmax_accept_kernel(
    const uint64_t* __restrict__ best, int num_best, int M, int64_t* __restrict__ predicted,
    const int32_t* __restrict__ draft, const int32_t* __restrict__ draft_len, int k, int S, int eos_id,
    const int32_t* __restrict__ max_tokens, int32_t* __restrict__ accepted, int32_t* __restrict__ committed,
    int32_t* __restrict__ num_committed, int32_t* __restrict__ seq_len, int32_t* __restrict__ history,
    int64_t history_stride, int32_t* __restrict__ history_len, int32_t* __restrict__ finished) {
  __shared__ int64_t s_pred[kMaxTokensPerSeq];
  const int b = blockIdx.x, lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int waves = (int)blockDim.x >> 6;
  const int32_t* const any = draft_len + b;
  // The acceptance inputs, requested by thread 0 (the only thread that uses them) before the keys.
  int32_t fin_raw = 0, n_raw = 0, len0_raw = 0, cap_raw = 0, sl_raw = 0;
  int32_t dv[kPre] = {};
  const int32_t* d = k > 0 ? draft + (int64_t)b * k : any;
  if (threadIdx.x == 0) {
    fin_raw = *(finished ? finished + b : any);
    n_raw = draft_len[b];
#pragma unroll
    for (int j = 0; j < kPre; ++j) dv[j] = d[k > 0 ? min(j, k - 1) : 0];
    len0_raw = *(history ? history_len + b : any);
    cap_raw = *(max_tokens ? max_tokens + b : any);
    sl_raw = *(seq_len ? seq_len + b : any);
  }
  const int64_t row0 = (int64_t)b * S;
  for (int j = wave; j < S; j += waves) {
    uint64_t mx = 0;
    for (int t0 = 0; t0 < num_best; t0 += 64 * kKeysPerLane) {
      uint64_t v[kKeysPerLane];
#pragma unroll
      for (int c = 0; c < kKeysPerLane; ++c) {
        const int t = min(t0 + 64 * c + lane, num_best - 1);  // past the end: a key already counted
        v[c] = best[(int64_t)t * M + row0 + j];
      }
#pragma unroll
      for (int c = 0; c < kKeysPerLane; ++c) mx = v[c] > mx ? v[c] : mx;
    }
#pragma unroll
    for (int mask = 1; mask < kWave; mask <<= 1) {
      const uint32_t lo = __shfl_xor((uint32_t)mx, mask, kWave);
      const uint32_t hi = __shfl_xor((uint32_t)(mx >> 32), mask, kWave);
      const uint64_t o = ((uint64_t)hi << 32) | lo;
      mx = o > mx ? o : mx;
    }
    if (lane == 0) {
      const int64_t id = (int64_t)(uint32_t)(~(uint32_t)mx);
      predicted[row0 + j] = id;
      s_pred[j] = id;
    }
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  int64_t pv[kPre + 1];
#pragma unroll
  for (int j = 0; j <= kPre; ++j) pv[j] = s_pred[min(j, S - 1)];
  accept_sequence(b, finished ? fin_raw : 0, n_raw, d, dv, pv, [&](int j) { return s_pred[j]; },
                  history ? len0_raw : 0, max_tokens ? cap_raw : 0, seq_len ? sl_raw : 0, k, S, eos_id, max_tokens,
                  accepted, committed, num_committed, seq_len, history, history_stride, history_len, finished);
}

int check_accept(const int32_t* draft, const int32_t* draft_len, int32_t k, int32_t tokens_per_seq, int32_t batch,
                 const int32_t* accepted, const int32_t* history, int64_t history_stride, const int32_t* history_len) {
  OXR_RETURN_IF(batch < 0 || k < 0 || tokens_per_seq < 1 || history_stride < 0, OXR_ERR_INVALID_ARG);
  if (batch == 0) return OXR_OK;
  OXR_RETURN_IF(!draft_len || !accepted || (k > 0 && !draft), OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(history && !history_len, OXR_ERR_INVALID_ARG);
  return OXR_OK;
}

}  // namespace
}  // namespace oxr

extern "C" int oxr_accept(const int32_t* draft, const int32_t* draft_len, int32_t k, const int64_t* predicted,
                          int32_t tokens_per_seq, int32_t batch, int32_t eos_id, const int32_t* max_tokens,
                          int32_t* accepted, int32_t* committed, int32_t* num_committed, int32_t* seq_len,
                          int32_t* history, int64_t history_stride, int32_t* history_len, int32_t* finished,
                          oxr_stream_t stream) {
  using namespace oxr;
  const int st = check_accept(draft, draft_len, k, tokens_per_seq, batch, accepted, history, history_stride,
                              history_len);
  if (st || batch == 0) return st;
  OXR_RETURN_IF(!predicted, OXR_ERR_INVALID_ARG);
  const int threads = 64;
  hipLaunchKernelGGL(accept_kernel, dim3((batch + threads - 1) / threads), dim3(threads), 0, (hipStream_t)stream,
                     draft, draft_len, k, predicted, tokens_per_seq, batch, eos_id, max_tokens, accepted, committed,
                     num_committed, seq_len, history, history_stride, history_len, finished);
  return OXR_LAUNCH_STATUS();
}

extern "C" int oxr_lm_head_accept_packed(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight_packed,
                                         int64_t hidden_size, int64_t vocab, void* workspace, size_t workspace_bytes,
                                         int64_t* predicted, const int32_t* draft, const int32_t* draft_len, int32_t k,
                                         int32_t tokens_per_seq, int32_t batch, int32_t eos_id,
                                         const int32_t* max_tokens, int32_t* accepted, int32_t* committed,
                                         int32_t* num_committed, int32_t* seq_len, int32_t* history,
                                         int64_t history_stride, int32_t* history_len, int32_t* finished,
                                         oxr_stream_t stream) {
  using namespace oxr;
  int st = check_accept(draft, draft_len, k, tokens_per_seq, batch, accepted, history, history_stride, history_len);
  if (st) return st;
  OXR_RETURN_IF(m != (int64_t)batch * tokens_per_seq || !predicted, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(tokens_per_seq > kMaxTokensPerSeq || m > 256, OXR_ERR_UNSUPPORTED);
  if (batch == 0) return OXR_OK;
  const uint64_t* best = nullptr;
  int num_best = 0;
  st = lm_head_keys(hidden, m, weight_packed, hidden_size, vocab, nullptr, workspace, workspace_bytes, true,
                    (hipStream_t)stream, &best, &num_best);
  if (st) return st;
  const int waves = std::min<int>(tokens_per_seq, kMaxRowWaves);
  hipLaunchKernelGGL(argmax_accept_kernel, dim3((unsigned)batch), dim3(64 * waves), 0, (hipStream_t)stream, best,
                     num_best, (int)m, predicted, draft, draft_len, k, tokens_per_seq, eos_id, max_tokens, accepted, committed,
                     num_committed, seq_len, history, history_stride, history_len, finished);
  return OXR_LAUNCH_STATUS();
}
