// Variable-length (prefill) attention on gfx950: the drop-in for
// attention.varlen (oxr_runtime/attention.py:47-59).
//
// Several sequences are concatenated along the token axis: q [T, H, 128],
// k/v [T, KV, 128] bf16, cu_seqlens int32 [n + 1] (sequence i is tokens
// [cu[i], cu[i+1])).  Within each sequence, query token j of q head h attends
// keys [0, j] (causal) or all keys (bidirectional) of kv head h / (H / KV);
// scores q.k * scale, fp32 softmax, bf16 output [T, H, 128].
//
// Prefill attention is MFMA-bound (Θ(len²) work per sequence), so unlike the
// verify kernel the keys are staged once per workgroup in LDS and shared by
// every query row of the workgroup:
// * A workgroup is 8 waves covering 128 query rows: the G = H / KV q heads of
//   one kv head, 128 / G consecutive positions each (16 rows per wave).
// * Key tiles of 64 rows are loaded cooperatively (two 16-byte pieces of K and
//   of V per thread), written to LDS row-major with 16-byte stores and a
//   32-byte row pad (rows 72 dwords apart: conflict-free fragment reads),
//   double-buffered: tile t + 1 is in registers while tile t is multiplied.
//   The PV product needs 8 keys of one dim per lane; gfx950's transposing LDS
//   read (ds_read_b64_tr_b16) gathers them from the row-major V tile.
// * Per wave and tile: S^T = K Q^T (16 MFMAs 16x16x32: 4 key blocks x 4 dim
//   steps; lane (r, g) holds keys 4g..4g+3 of each key block for query r), an
//   exp2-domain online softmax, then O^T += V^T P^T (16 MFMAs; P^T is used as
//   computed: key slot 8g + 4p + j of a 32-key step stands for key 16p + 4g + j,
//   and the V^T fragments are gathered in the same order).
// * Causal: key tiles above a wave's last row are skipped, the diagonal tile
//   is masked per element; keys past the sequence are masked.
#include "common.h"

namespace oxr {
namespace {

constexpr int kVD = 128;           // head dim
constexpr int kVWaves = 8;         // waves per workgroup
constexpr int kVRows = 16 * kVWaves;  // query rows per workgroup (all q heads of the kv head)
constexpr int kKeyTile = 64;       // keys per LDS stage
constexpr int kKPitch = kVD + 16;  // bf16 per K row in LDS (32-byte pad: conflict-free fragment reads)
constexpr int kVPitch = kVD + 16;  // bf16 per V row in LDS (32-byte pad: conflict-free transposing reads)

// LDS transpose read (gfx950 ds_read_b64_tr_b16).  Within each group of 16 lanes,
// lane 4a + b receives element b of the 4 bf16 addressed by lanes a, a + 4,
// a + 8 and a + 12 of its group, in that order.
__device__ __forceinline__ u32x2 lds_read_tr16(const bf16_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (v4s __attribute__((address_space(3)))*)(const_cast<bf16_t*>(p)));
  return __builtin_bit_cast(u32x2, x);
}

template <bool kCausal>
__global__ __launch_bounds__(64 * kVWaves) void varlen_attention_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ cu_seqlens, int H, int KV, float scale_log2, bf16_t* __restrict__ out) {
  __shared__ bf16_t s_k[2][kKeyTile][kKPitch];
  __shared__ bf16_t s_v[2][kKeyTile][kVPitch];

  const int seq = blockIdx.z, kvh = blockIdx.y;
  const int start = cu_seqlens[seq], len = cu_seqlens[seq + 1] - start;
  const int G = H / KV, rows_per_head = kVRows / G;
  // Query tiles in reverse order: under the causal mask the late ones do the most work, so they
  // are dispatched first.
  const int q0 = (int)(gridDim.x - 1 - blockIdx.x) * rows_per_head;  // first position, per head
  if (q0 >= len) return;                            // whole workgroup: before any barrier

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int waves_per_head = kVWaves / G;
  const int head = kvh * G + wave / waves_per_head;
  const int w0 = q0 + 16 * (wave % waves_per_head);  // this wave's first query position
  const int qpos = w0 + r;                           // query position of lane row r

  // Q^T fragments (B operand): lane (r, g) holds Q[w0 + r][32i + 8g, +8) for dim step i.
  u32x4 qf[4];
  {
    const int qrow = min(qpos, len - 1);  // rows past the sequence compute and are never stored
    const bf16_t* src = q + ((int64_t)(start + qrow) * H + head) * kVD + 8 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[i] = ld128(src + 32 * i);
  }

  // Keys this workgroup needs, and the last key any of this wave's rows sees.
  const int key_end = kCausal ? min(len, q0 + rows_per_head) : len;
  const int wave_last = kCausal ? min(w0 + 15, len - 1) : len - 1;
  const int tiles = (key_end + kKeyTile - 1) / kKeyTile;

  // Cooperative staging: 16-byte piece p = t + 512h (h = 0, 1) of the tile is
  // dims [8 (p % 16), +8) of key p / 16, from K and from V (a wave covers 4
  // whole rows); keys past the sequence re-read its last key (their scores are
  // masked).  Both are stored row-major.
  const int st_key = tid >> 4, st_d = (tid & 15) * 8;
  u32x4 kr[2], vr[2];
  auto fetch = [&](int t) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int key = min(t * kKeyTile + st_key + 32 * h, len - 1);
      const int64_t row = ((int64_t)(start + key) * KV + kvh) * kVD + st_d;
      kr[h] = ld128(k + row);
      vr[h] = ld128(v + row);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      *reinterpret_cast<u32x4*>(&s_k[buf][st_key + 32 * h][st_d]) = kr[h];
      *reinterpret_cast<u32x4*>(&s_v[buf][st_key + 32 * h][st_d]) = vr[h];
    }
  };

  float m_run = -INFINITY, mc_run = 0.f, l_run = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  fetch(0);
  stash(0);
  __syncthreads();
  for (int t = 0; t < tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < tiles) fetch(t + 1);  // in flight during this tile's products
    const int kt0 = t * kKeyTile;
    if (kt0 <= wave_last) {  // wave-uniform: otherwise every key of the tile is masked for this wave
      // Raw scores of keys kt0 + 16kb + 4g + j for query row r.
      float sv[16];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 kf = *reinterpret_cast<const u32x4*>(&s_k[buf][16 * kb + r][32 * i + 8 * g]);
          acc = mfma_16x16x32(kf, qf[i], acc);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) sv[4 * kb + j] = acc[j];
      }
      const bool edge = kt0 + kKeyTile - 1 > (kCausal ? w0 : len - 1) || kt0 + kKeyTile > len;
      if (edge) {  // wave-uniform: the diagonal tile or the sequence's last tile
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kt0 + 16 * (e >> 2) + 4 * g + (e & 3);
          if (key >= len || (kCausal && key > qpos)) sv[e] = -INFINITY;
        }
      }
      float mx = sv[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mx = fmaxf(mx, sv[e]);
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      const bool moved = mx > m_run;
      if (__builtin_amdgcn_ballot_w64(moved)) {
        const float m_new = moved ? mx : m_run;
        const float mc_new = m_new == -INFINITY ? 0.f : m_new * scale_log2;
        const float alpha = !moved ? 1.0f : (m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc_run - mc_new));
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
        m_run = m_new;
        mc_run = mc_new;
      }
      float pv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        pv[e] = __builtin_amdgcn_exp2f(fmaf(sv[e], scale_log2, -mc_run));
        l_run += pv[e];
      }
      // Two 32-key steps; P^T slot 8g + 4p + j is key 16 (2s + p) + 4g + j.
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4 pb = {pack_bf_hw(pv[8 * s + 0], pv[8 * s + 1]), pack_bf_hw(pv[8 * s + 2], pv[8 * s + 3]),
                          pack_bf_hw(pv[8 * s + 4], pv[8 * s + 5]), pack_bf_hw(pv[8 * s + 6], pv[8 * s + 7])};
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          // A = V^T: lane (r, g) gets dim 16 dt + r of keys 32s + 16p + 4g + (0..3), p = 0, 1, from
          // two transposing reads in which lane j of the group addresses key 32s + 16p + 4g + j / 4,
          // dims 16 dt + 4 (j % 4) .. +3.
          const bf16_t* vp = &s_v[buf][32 * s + 4 * g + (r >> 2)][16 * dt + 4 * (r & 3)];
          const u32x2 lo = lds_read_tr16(vp);
          const u32x2 hi = lds_read_tr16(vp + 16 * kVPitch);
          o[dt] = mfma_16x16x32(u32x4{lo.x, lo.y, hi.x, hi.y}, pb, o[dt]);
        }
      }
    }
    if (t + 1 < tiles) stash(buf ^ 1);  // the other buffer was last read before the previous barrier
    __syncthreads();
  }

  // Normalise and store: lane (r, g) holds O^T[16 dt + 4g + j][query r].
  float l_tot = l_run + shfl_xor_f(l_run, 16);
  l_tot += shfl_xor_f(l_tot, 32);
  if (qpos < len) {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    bf16_t* dst = out + ((int64_t)(start + qpos) * H + head) * kVD + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<u32x2*>(dst + 16 * dt) =
          u32x2{pack_bf(o[dt][0] * inv, o[dt][1] * inv), pack_bf(o[dt][2] * inv, o[dt][3] * inv)};
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
  OXR_RETURN_IF(kVWaves % G != 0, OXR_ERR_UNSUPPORTED);  // G in {1, 2, 4, 8}
  OXR_RETURN_IF(num_seqs > 65535 || num_kv_heads > 65535, OXR_ERR_UNSUPPORTED);
  if (num_seqs == 0 || max_len == 0) return OXR_OK;
  OXR_RETURN_IF(!q || !k || !v || !cu_seqlens || !out, OXR_ERR_INVALID_ARG);
  OXR_RETURN_IF(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 != 0 || (uintptr_t)out % 8 != 0,
                OXR_ERR_UNSUPPORTED);
  const int rows_per_head = kVRows / G;
  const dim3 grid((unsigned)((max_len + rows_per_head - 1) / rows_per_head), (unsigned)num_kv_heads,
                  (unsigned)num_seqs);
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  if (causal)
    hipLaunchKernelGGL(varlen_attention_kernel<true>, grid, dim3(64 * kVWaves), 0, s, q, k, v, cu_seqlens,
                       num_heads, num_kv_heads, scale_log2, out);
  else
    hipLaunchKernelGGL(varlen_attention_kernel<false>, grid, dim3(64 * kVWaves), 0, s, q, k, v, cu_seqlens,
                       num_heads, num_kv_heads, scale_log2, out);
  return OXR_LAUNCH_STATUS();
}
