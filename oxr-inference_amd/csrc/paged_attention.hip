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
// of thousands of tokens, so the context is split into chunks of kChunk
// tokens and every (chunk, kv head, sequence) is one single-wave workgroup.
// Each writes an unnormalised partial (running max m, sum l, O[R][128]) and
// counts itself on a per-(sequence, kv head) counter; the workgroup that
// arrives last merges the chunks with the usual log-sum-exp rescaling and
// resets the counter, so one launch does the whole op.  A context that fits
// in one chunk is normalised and stored directly.
//
// Per wave, 32 keys at a time (two 16-key MFMA tiles):
//   S^T tile = K[16 keys x 128] * Q^T        4 x v_mfma_f32_16x16x32_bf16 per tile
//     K comes straight from the paged cache: a lane reads 64 contiguous bytes
//     of one key row, which is exactly its MFMA A-operand fragment; Q^T is
//     held in registers.  Lane (r = l % 16, g = l / 16) gets the scores of
//     keys 4g..4g+3 for query row r.
//   online softmax per row in the exp2 domain (scale * log2 e folded in)
//   O^T += V^T[128 x 32 keys] * P^T             8 MFMAs (one per 16 dims)
//     P^T is the B operand as computed (bf16), with key slot 4p + j of lane
//     group g standing for key 16p + 4g + j; V^T goes through LDS: the 32 key
//     rows are loaded with 128-byte-per-lane reads and written transposed, so
//     each A fragment is two 8-byte LDS reads.
//     Accumulators hold O^T[d][r], so the per-row rescale is a per-lane scalar.
// The next 32 keys' K and V are loaded before the current ones are used.
#include "common.h"

namespace oxr {
namespace {

constexpr int kD = 128;
constexpr int kRows = 16;   // query rows per (sequence, kv head): one MFMA tile
constexpr int kVPitch = 36; // LDS row pitch of V^T in bf16 (32 keys + pad, 8-byte aligned)

struct PairRegs {
  u32x4 k[2][4];  // K fragments of the two 16-key tiles
  u32x4 v[8];     // 128 contiguous bytes of one key's V row
};

__device__ __forceinline__ int64_t row_of(const int32_t* __restrict__ table_row, int tok, int log2_bs,
                                          int64_t num_blocks) {
  int64_t blk = table_row[tok >> log2_bs];
  blk = blk < 0 ? 0 : (blk >= num_blocks ? num_blocks - 1 : blk);  // never leave the pool
  return (blk << log2_bs) + (tok & ((1 << log2_bs) - 1));
}

__device__ __forceinline__ void load_pair(PairRegs& pr, const bf16_t* __restrict__ k_cache,
                                          const bf16_t* __restrict__ v_cache, const int32_t* __restrict__ table_row,
                                          int t0, int L, int kvh, int KV, int log2_bs, int64_t num_blocks, int lane) {
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int tok = min(t0 + 16 * p + r, L - 1);
    const bf16_t* src = k_cache + (row_of(table_row, tok, log2_bs, num_blocks) * KV + kvh) * kD + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) pr.k[p][i] = ld128_nt(src + 8 * i);
  }
  const int tv = t0 + (lane >> 1);
  const bool valid = tv < L;
  const bf16_t* src = v_cache + (row_of(table_row, min(tv, L - 1), log2_bs, num_blocks) * KV + kvh) * kD + 64 * (lane & 1);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 x = ld128_nt(src + 8 * i);
    pr.v[i] = valid ? x : u32x4{0u, 0u, 0u, 0u};  // keys past L contribute 0 * 0, never 0 * garbage
  }
}

template <int kChunk>
__global__ __launch_bounds__(64) void paged_extend_partial_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache, const bf16_t* __restrict__ v_cache,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ block_table, int64_t table_stride, int S,
    int H, int KV, int log2_bs, int64_t num_blocks, float scale_log2, int max_seq_len, int max_chunks,
    float* __restrict__ part_o, float* __restrict__ part_ml, int32_t* __restrict__ counters,
    bf16_t* __restrict__ out) {
  __shared__ __align__(16) uint16_t vt[kD * kVPitch];

  const int chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int L = min(seq_lens[b], max_seq_len);  // max_seq_len <= table span, checked on the host
  const int t_begin = chunk * kChunk;
  if (t_begin >= L) return;  // the merge reads only chunks below ceil(L / kChunk)
  const int t_end = min(L, t_begin + kChunk);
  const int G = H / KV, R = S * G;
  const int lane = threadIdx.x;
  const int r = lane & 15, g = lane >> 4;
  const int32_t* table_row = block_table + (int64_t)b * table_stride;

  // Q^T fragments for row r: q[b, s, kvh * G + hh, 32g + 8i .. +7].
  u32x4 qf[4];
  int qpos = -1;  // absolute position of row r; keys after it are masked
  if (r < R) {
    const int s = r / G, hh = r % G;
    const bf16_t* src = q + (((int64_t)b * S + s) * H + kvh * G + hh) * kD + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[i] = ld128(src + 8 * i);
    qpos = L - S + s;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[i] = u32x4{0u, 0u, 0u, 0u};
  }

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  PairRegs cur, nxt;
  load_pair(cur, k_cache, v_cache, table_row, t_begin, L, kvh, KV, log2_bs, num_blocks, lane);
  for (int t0 = t_begin; t0 < t_end; t0 += 32) {
    const bool more = t0 + 32 < t_end;
    if (more) load_pair(nxt, k_cache, v_cache, table_row, t0 + 32, L, kvh, KV, log2_bs, num_blocks, lane);

    // Scores of keys t0 + 16p + 4g + j for query row r.
    float sv[8];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = mfma_16x16x32(cur.k[p][i], qf[i], acc);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = t0 + 16 * p + 4 * g + j;
        sv[4 * p + j] = (tok <= qpos) ? acc[j] * scale_log2 : -INFINITY;
      }
    }
    float mx = sv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
    mx = fmaxf(mx, shfl_xor_f(mx, 16));
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;  // fully masked so far: keep p = 0
    const float alpha = exp2f(m_run - m_use);
    float pv[8], psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pv[e] = exp2f(sv[e] - m_use);
      psum += pv[e];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
    const u32x4 pb = {pack_bf(pv[0], pv[1]), pack_bf(pv[2], pv[3]), pack_bf(pv[4], pv[5]), pack_bf(pv[6], pv[7])};

    // V^T into LDS: this lane holds dims 64 * (lane & 1) + [0, 64) of key lane >> 1.
    __syncthreads();
    {
      const int key = lane >> 1, d0 = 64 * (lane & 1);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w[4] = {cur.v[i].x, cur.v[i].y, cur.v[i].z, cur.v[i].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vt[(d0 + 8 * i + 2 * e) * kVPitch + key] = (uint16_t)(w[e] & 0xffffu);
          vt[(d0 + 8 * i + 2 * e + 1) * kVPitch + key] = (uint16_t)(w[e] >> 16);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint16_t* row = vt + (dt * 16 + r) * kVPitch;
      const u32x2 lo = *reinterpret_cast<const u32x2*>(row + 4 * g);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(row + 16 + 4 * g);
      const u32x4 a = {lo.x, lo.y, hi.x, hi.y};
      o[dt] = mfma_16x16x32(a, pb, o[dt]);
    }
    if (more) cur = nxt;
  }

  float l_tot = l_run + shfl_xor_f(l_run, 16);
  l_tot += shfl_xor_f(l_tot, 32);
  const int nc = (L + kChunk - 1) / kChunk;
  if (nc == 1) {
    // The whole context fits one chunk: normalise and store directly.
    if (r < R) {
      const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
      const int s = r / G, hh = r % G;
      bf16_t* dst = out + (((int64_t)b * S + s) * H + kvh * G + hh) * kD;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const f32x4 v = o[dt] * inv;
        *reinterpret_cast<u32x2*>(dst + dt * 16 + 4 * g) = u32x2{pack_bf(v[0], v[1]), pack_bf(v[2], v[3])};
      }
    }
    return;
  }
  const int64_t unit0 = ((int64_t)b * KV + kvh) * max_chunks;
  if (r < R) {
    float* dst = part_o + ((unit0 + chunk) * kRows + r) * kD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(dst + dt * 16 + 4 * g) = o[dt];
    if (g == 0) {
      part_ml[((unit0 + chunk) * kRows + r) * 2 + 0] = m_run;
      part_ml[((unit0 + chunk) * kRows + r) * 2 + 1] = l_tot;
    }
  }
  // The last chunk of this (sequence, kv head) to finish merges all of them:
  // release the partial, count it, and the workgroup that brings the count to
  // nc acquires every partial and resets the counter for the next launch.
  __threadfence();
  int arrived = 0;
  if (lane == 0) arrived = atomicAdd(counters + (int64_t)b * KV + kvh, 1);
  arrived = __shfl(arrived, 0, kWave);
  if (arrived != nc - 1) return;
  __threadfence();
  if (lane == 0) counters[(int64_t)b * KV + kvh] = 0;
  for (int idx = lane; idx < R * (kD / 4); idx += kWave) {
    const int rr = idx / (kD / 4), d0 = (idx % (kD / 4)) * 4;
    float mmax = -INFINITY;
    for (int c = 0; c < nc; ++c) mmax = fmaxf(mmax, __builtin_nontemporal_load(part_ml + ((unit0 + c) * kRows + rr) * 2));
    const float m_use = (mmax == -INFINITY) ? 0.f : mmax;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float lsum = 0.f;
    for (int c = 0; c < nc; ++c) {
      const float* ml = part_ml + ((unit0 + c) * kRows + rr) * 2;
      const float w = exp2f(__builtin_nontemporal_load(ml) - m_use);
      lsum += __builtin_nontemporal_load(ml + 1) * w;
      const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(part_o + ((unit0 + c) * kRows + rr) * kD + d0));
      acc += v * w;
    }
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    const int s = rr / G, hh = rr % G;
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + (((int64_t)b * S + s) * H + kvh * G + hh) * kD + d0);
    dst[0] = pack_bf(acc[0] * inv, acc[1] * inv);
    dst[1] = pack_bf(acc[2] * inv, acc[3] * inv);
  }
}

constexpr int kChunkTokens = 256;

int chunks_for(int32_t max_seq_len) { return (max_seq_len + kChunkTokens - 1) / kChunkTokens; }

}  // namespace
}  // namespace oxr

extern "C" size_t oxr_paged_extend_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len) {
  using namespace oxr;
  if (batch <= 0 || num_kv_heads <= 0 || max_seq_len <= 0) return 0;
  const size_t units = (size_t)batch * num_kv_heads * chunks_for(max_seq_len);
  return units * kRows * (kD + 2) * sizeof(float) + (size_t)batch * num_kv_heads * sizeof(int32_t);
}

extern "C" int oxr_paged_extend(const oxr_bf16* q, const oxr_bf16* k_cache, const oxr_bf16* v_cache,
                                const int32_t* seq_lens, const int32_t* block_table, int64_t table_stride,
                                int32_t batch, int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t max_seq_len,
                                float scale, oxr_bf16* out, void* workspace, size_t workspace_bytes,
                                oxr_stream_t stream) {
  using namespace oxr;
  OXR_RETURN_IF(batch < 0 || tokens_per_seq <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_blocks <= 0 ||
                    table_stride < 0 || max_seq_len <= 0,
                OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(head_dim != kD || num_heads % num_kv_heads != 0, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(tokens_per_seq * (num_heads / num_kv_heads) > kRows, OXR_ERR_UNSUPPORTED);
  OXR_RETURN_IF(block_size <= 0 || (block_size & (block_size - 1)) != 0, OXR_ERR_UNSUPPORTED);
  // Contexts are clamped to max_seq_len, so every key visited maps to a table entry.
  OXR_RETURN_IF((int64_t)max_seq_len > table_stride * block_size, OXR_ERR_INVALID_ARG);
  if (batch == 0) return OXR_OK;
  OXR_RETURN_IF(!q || !k_cache || !v_cache || !seq_lens || !block_table || !out, OXR_ERR_INVALID_ARG);
  const size_t need = oxr_paged_extend_workspace_bytes(batch, num_kv_heads, max_seq_len);
  OXR_RETURN_IF(!workspace || workspace_bytes < need, OXR_ERR_WORKSPACE);
  const int max_chunks = chunks_for(max_seq_len);
  OXR_RETURN_IF(max_chunks > 65535 || batch > 65535, OXR_ERR_UNSUPPORTED);
  int log2_bs = 0;
  while ((1 << log2_bs) < block_size) ++log2_bs;
  float* part_o = static_cast<float*>(workspace);
  float* part_ml = part_o + (size_t)batch * num_kv_heads * max_chunks * kRows * kD;
  int32_t* counters = reinterpret_cast<int32_t*>(part_ml + (size_t)batch * num_kv_heads * max_chunks * kRows * 2);
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(paged_extend_partial_kernel<kChunkTokens>, dim3(max_chunks, num_kv_heads, batch), dim3(64), 0,
                     (hipStream_t)stream, q, k_cache, v_cache, seq_lens, block_table, table_stride, tokens_per_seq,
                     num_heads, num_kv_heads, log2_bs, num_blocks, scale_log2, max_seq_len, max_chunks, part_o,
                     part_ml, counters, out);
  return OXR_LAUNCH_STATUS();
}
