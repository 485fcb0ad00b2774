// Expansion of one step's host-assembled inputs on the device (gfx950).
//
// The reference's graph runners (oxr_runtime/decode_graph.py:92-119, 176-205) pad each batch to
// its bucket on the host and copy five staging buffers, among them a dense [bucket, width] page
// table, per replay.  Here the host writes one compact int64 record -- the real sequences' rows
// and each sequence's page list back to back -- and issues one copy; this kernel, the first node
// of every captured graph, expands it into the bucket's static tensors:
//
//   record[0]                      n, the real sequences (<= capacity)
//   record[1]                      P, the pages listed
//   record[2 + 0T .. 2 + 1T)       ids        (T = capacity * S; rows of the n real sequences)
//   record[2 + 1T .. 2 + 2T)       positions
//   record[2 + 2T .. 2 + 3T)       slots
//   record[2 + 3T .. +capacity)    seq_lens
//   then capacity + 1 offsets      sequence b's pages are pages[off[b] .. off[b+1])
//   then P pages
//
// Rows of padded sequences (b >= n) are the scratch page's: token j of such a sequence has id 0,
// position j, slot scratch_block * block_size + j and seq_len S, so it writes and reads only the
// scratch page's first S slots (decode_graph.py:188-197).  Table entries past a sequence's pages,
// and whole rows of padded sequences, hold the scratch page.
#include "common.h"

namespace oxr {
namespace {

__global__ __launch_bounds__(256) void unpack_step_kernel(const int64_t* __restrict__ record, int capacity, int S,
                                                          int width, int scratch_block, int block_size,
                                                          int64_t* __restrict__ ids, int64_t* __restrict__ positions,
                                                          int64_t* __restrict__ slots, int32_t* __restrict__ seq_lens,
                                                          int32_t* __restrict__ table) {
  const int b = blockIdx.x;  // one workgroup per sequence of the bucket
  const int64_t T = (int64_t)capacity * S;
  const int64_t n = min(max(record[0], (int64_t)0), (int64_t)capacity);
  const int64_t* r_ids = record + 2;
  const int64_t* r_pos = r_ids + T;
  const int64_t* r_slots = r_pos + T;
  const int64_t* r_lens = r_slots + T;
  const int64_t* r_off = r_lens + capacity;
  const int64_t* r_pages = r_off + capacity + 1;
  const bool real = b < n;
  for (int j = threadIdx.x; j < S; j += blockDim.x) {
    const int64_t row = (int64_t)b * S + j;
    ids[row] = real ? r_ids[row] : 0;
    positions[row] = real ? r_pos[row] : j;
    slots[row] = real ? r_slots[row] : (int64_t)scratch_block * block_size + j;
  }
  if (threadIdx.x == 0) seq_lens[b] = real ? (int32_t)r_lens[b] : S;
  const int64_t first = real ? r_off[b] : 0;
  const int64_t count = real ? min(max(r_off[b + 1] - first, (int64_t)0), (int64_t)width) : 0;
  for (int c = threadIdx.x; c < width; c += blockDim.x)
    table[(int64_t)b * width + c] = c < count ? (int32_t)r_pages[first + c] : scratch_block;
}

}  // namespace
}  // namespace oxr

extern "C" size_t oxr_step_record_words(int32_t capacity, int32_t tokens_per_seq, int32_t width) {
  if (capacity <= 0 || tokens_per_seq <= 0 || width < 0) return 0;
  const size_t c = (size_t)capacity;
  return 2 + 3 * c * (size_t)tokens_per_seq + c + (c + 1) + c * (size_t)width;
}

extern "C" int oxr_unpack_step_inputs(const int64_t* record, int32_t capacity, int32_t bucket, int32_t tokens_per_seq,
                                      int32_t width, int32_t scratch_block, int32_t block_size, int64_t* ids,
                                      int64_t* positions, int64_t* slots, int32_t* seq_lens, int32_t* table,
                                      oxr_stream_t stream) {
  OXR_RETURN_IF(capacity <= 0 || bucket < 0 || bucket > capacity || tokens_per_seq <= 0 || width < 0 ||
                    scratch_block < 0 || block_size <= 0,
                OXR_ERR_INVALID_ARG);
  if (bucket == 0) return OXR_OK;
  OXR_RETURN_IF(!record || !ids || !positions || !slots || !seq_lens || (width > 0 && !table), OXR_ERR_INVALID_ARG);
  hipLaunchKernelGGL(oxr::unpack_step_kernel, dim3(bucket), dim3(256), 0, (hipStream_t)stream, record, capacity,
                     tokens_per_seq, width, scratch_block, block_size, ids, positions, slots, seq_lens, table);
  return OXR_LAUNCH_STATUS();
}
