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
#include "common.h"

namespace oxr {
namespace {

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
  constexpr int kPre = 8;
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
  const int32_t fin = finished ? fin_raw : 0;
  const int32_t len0 = history ? len0_raw : 0;
  const int32_t cap = max_tokens ? cap_raw : 0;
  const int32_t sl = seq_len ? sl_raw : 0;

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
  while (a >= kPre && a < n && (int64_t)d[a] == pred[a]) ++a;  // drafts beyond the preloaded ones
  accepted[b] = a;
  if (num_committed) num_committed[b] = a + 1;
  // Token j of the committed run is pv[j] for j <= kPre (static indices only: a dynamically
  // indexed register array would be placed in scratch memory), else loaded again.
  if (committed) {
    int32_t* const row = committed + (int64_t)b * (k + 1);
#pragma unroll
    for (int j = 0; j <= kPre; ++j)
      if (j <= k) row[j] = (j <= a) ? (int32_t)pv[j] : -1;
    for (int j = kPre + 1; j <= k; ++j) row[j] = (j <= a) ? (int32_t)pred[j] : -1;
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
    for (int j = kPre + 1; !stop && j <= a; ++j) take((int32_t)pred[j]);
    history_len[b] = len;
    if (finished) finished[b] = reason;
  }
}

}  // namespace
}  // namespace oxr

extern "C" int oxr_accept(const int32_t* draft, const int32_t* draft_len, int32_t k, const int64_t* predicted,
                          int32_t tokens_per_seq, int32_t batch, int32_t eos_id, const int32_t* max_tokens,
                          int32_t* accepted, int32_t* committed, int32_t* num_committed, int32_t* seq_len,
                          int32_t* history, int64_t history_stride, int32_t* history_len, int32_t* finished,
                          oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(batch < 0 || k < 0 || tokens_per_seq < 1 || history_stride < 0, OXR_ERR_INVALID_ARG);
  if (batch == 0) return OXR_OK;
  OXR_RETURN_IF(!draft_len || !predicted || !accepted || (k > 0 && !draft), OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(history && !history_len, OXR_ERR_INVALID_ARG);
  const int threads = 64;
  hipLaunchKernelGGL(accept_kernel, dim3((batch + threads - 1) / threads), dim3(threads), 0, (hipStream_t)stream,
                     draft, draft_len, k, predicted, tokens_per_seq, batch, eos_id, max_tokens, accepted, committed,
                     num_committed, seq_len, history, history_stride, history_len, finished);
  return OXR_LAUNCH_STATUS();
}
