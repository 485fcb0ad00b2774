// The LM head's argmax without its last step, for kernels that finish the argmax themselves.
#pragma once

#include "common.h"

namespace oxr {

// oxr_lm_head_argmax[_packed] up to, not including, the cross-workgroup reduction: the same
// checks and launches, leaving per-workgroup keys best[t * m + row] (t < num_best; the larger bf16
// logit, then the lower column, as one 64-bit key) at the start of the workspace.  m == 0 launches
// nothing and sets num_best = 0.
int lm_head_keys(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight, int64_t hidden_size, int64_t vocab,
                 oxr_bf16* logits, void* workspace, size_t workspace_bytes, bool packed, hipStream_t stream,
                 const uint64_t** best, int* num_best);

}  // namespace oxr
