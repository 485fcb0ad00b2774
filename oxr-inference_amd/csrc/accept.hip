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
  if (finished && finished[b] != 0) {  // a finished sequence takes no tokens
    accepted[b] = 0;
    if (num_committed) num_committed[b] = 0;
    if (committed)
      for (int j = 0; j <= k; ++j) committed[(int64_t)b * (k + 1) + j] = -1;
    return;
  }
  const int n = min(max(draft_len[b], 0), min(k, S - 1));
  const int32_t* d = draft + (int64_t)b * k;
  const int64_t* pred = predicted + (int64_t)b * S;
  int a = 0;
  while (a < n && (int64_t)d[a] == pred[a]) ++a;
  accepted[b] = a;
  if (num_committed) num_committed[b] = a + 1;
  if (committed)
    for (int j = 0; j <= k; ++j) committed[(int64_t)b * (k + 1) + j] = (j <= a) ? (int32_t)pred[j] : -1;
  if (seq_len) seq_len[b] += a + 1;
  if (history) {
    int len = history_len[b];
    int reason = 0;
    for (int j = 0; j <= a; ++j) {
      const int32_t t = (int32_t)pred[j];
      if (t == eos_id) {
        reason = 1;
        break;
      }
      if (len >= history_stride) {  // buffer full: stop as a length finish
        reason = 2;
        break;
      }
      history[(int64_t)b * history_stride + len] = t;
      ++len;
      if (max_tokens && len >= max_tokens[b]) {
        reason = 2;
        break;
      }
    }
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
