/*
 * oxr_verify.h -- C ABI of the MI355X (gfx950) speculative-decoding verify step.
 *
 * Every entry point takes device pointers that the caller owns, plain sizes and
 * a HIP stream (a `hipStream_t`, e.g. torch.cuda.current_stream().cuda_stream).
 * They allocate nothing, never synchronize the device, and are safe to record
 * into a HIP graph.  bf16 tensors are passed as `uint16_t` bit patterns.
 *
 * Return value: OXR_OK (0) on success; a negative OXR_ERR_* code when an
 * argument is rejected before any launch; a positive hipError_t when a launch
 * failed.  oxr_status_string() names each code.
 *
 * Reference interfaces each entry point replaces are cited as file:line in
 * NickWilde18/oxr-inference (oxr_runtime/...).
 */
#ifndef OXR_VERIFY_H
#define OXR_VERIFY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OXR_ABI_VERSION 1

#define OXR_OK 0
#define OXR_ERR_INVALID_ARG (-1)   /* null pointer, negative or inconsistent size */
#define OXR_ERR_UNSUPPORTED (-2)   /* shape outside what the kernels implement     */
#define OXR_ERR_WORKSPACE (-3)     /* workspace missing or smaller than required   */
#define OXR_ERR_SCRATCH_LIMIT (-4) /* shape needs more than the static scratch holds */

typedef void* oxr_stream_t; /* hipStream_t */
typedef uint16_t oxr_bf16;  /* raw bfloat16 bits */

/* Library identity and status strings (no reference counterpart). */
int oxr_abi_version(void);
const char* oxr_status_string(int status);

/*
 * Self-test of the MFMA 16x16x32 bf16 operand layout the kernels assume (no
 * reference counterpart): c[16x16] = a[16x32] @ b[32x16], bf16 in, fp32 out.
 */
int oxr_selftest_mfma_layout(const uint16_t* a, const uint16_t* b, float* c, oxr_stream_t stream);

/*
 * (1) Batched n-gram suffix-match drafting.
 * Replaces NgramProposer.__init__/_add/extend/propose (oxr_runtime/speculative.py:15-39):
 * for each sequence b with history h = history[b, :history_len[b]] and
 * L = history_len[b], try n = min(max_n, L) .. 1 and take the largest p in
 * [n, L-1] with h[p-n:p] == h[L-n:L]; the draft is h[p : min(p+k_b, L)] with
 * k_b = k_limit ? max(0, min(k, k_limit[b])) : k.  No match -> empty draft.
 * history is int32 [batch, history_stride]; draft is int32 [batch, k] (unused
 * entries set to 0); draft_len is int32 [batch].  index_len (optional, int32
 * [batch]) limits the candidates to p <= index_len[b] - 1: the positions a
 * proposer has indexed so far (NgramProposer built on a prefix, not extended).
 * max_n must be in [1, 8] and k in [0, 64].
 */
int oxr_ngram_propose(const int32_t* history, int64_t history_stride, const int32_t* history_len,
                      const int32_t* index_len, int32_t batch, int32_t max_n, int32_t k, const int32_t* k_limit,
                      int32_t* draft, int32_t* draft_len, oxr_stream_t stream);

/*
 * (1b) Drafting fused with verify-input assembly.
 * Replaces Engine._speculate's draft loop and row assembly
 * (oxr_runtime/engine.py:674-684, 700-710; slot_of at language.py:320-322):
 * drafts as oxr_ngram_propose, then for row j < tokens_per_seq of sequence b
 *   ids[b*S + j]       = j == 0 ? history[b, L-1] : (j-1 < draft_len ? draft[j-1] : 0)
 *   positions[b*S + j] = seq_len[b] + j
 *   slots[b*S + j]     = block_table[b, pos / block_size] * block_size + pos % block_size
 *                        (-1 when pos / block_size >= table_stride or the table entry is negative)
 *   attn_seq_lens[b]   = seq_len[b] + S
 * seq_len is the KV length before the step (the reference's seq.length).
 * Drafts are further capped by the room engine.py:683-684 leaves:
 * k_b <= max_tokens[b] - L - 1 (when max_tokens is non-null) and
 * k_b <= max_positions - seq_len[b] - 1 (when max_positions > 0).
 * tokens_per_seq (S) must be >= k + 1 and at most 256 (OXR_ERR_UNSUPPORTED beyond).
 * ids/positions/slots are int64 [B*S].
 */
int oxr_propose_verify_inputs(const int32_t* history, int64_t history_stride, const int32_t* history_len,
                              int32_t batch, int32_t max_n, int32_t k, const int32_t* k_limit,
                              const int32_t* seq_len, const int32_t* block_table, int64_t table_stride,
                              int32_t block_size, int32_t tokens_per_seq, const int32_t* max_tokens,
                              int32_t max_positions, int32_t* draft, int32_t* draft_len, int64_t* ids,
                              int64_t* positions, int64_t* slots, int32_t* attn_seq_lens, oxr_stream_t stream);

/*
 * Step inputs of the list-interface graph runners, expanded on the device.
 * Replaces the host-side padding, scratch-page filling and pack_page_table of
 * DecodeGraphs.run / ExtendGraphs.run (oxr_runtime/decode_graph.py:92-119,
 * 176-205; kv_cache.py:60-72): the host writes one int64 record for up to
 * `capacity` sequences of tokens_per_seq (S) rows each --
 *   [n, P, ids[capacity*S], positions[capacity*S], slots[capacity*S],
 *    seq_lens[capacity], page offsets[capacity + 1], pages[P]]
 * (rows of the n real sequences; sequence b's pages are
 * pages[off[b] .. off[b+1])) -- copies it in one transfer, and this kernel
 * fills the bucket's tensors: ids / positions / slots int64 [bucket*S],
 * seq_lens int32 [bucket], table int32 [bucket, width].  Sequences b >= n
 * become scratch rows (id 0, position j, slot scratch_block*block_size + j,
 * seq_len S); table entries past a sequence's pages hold scratch_block.
 * oxr_step_record_words gives the record's size in int64 words.
 */
size_t oxr_step_record_words(int32_t capacity, int32_t tokens_per_seq, int32_t width);
int oxr_unpack_step_inputs(const int64_t* record, int32_t capacity, int32_t bucket, int32_t tokens_per_seq,
                           int32_t width, int32_t scratch_block, int32_t block_size, int64_t* ids,
                           int64_t* positions, int64_t* slots, int32_t* seq_lens, int32_t* table,
                           oxr_stream_t stream);

/*
 * (4c) Longest-prefix greedy acceptance + length rollback.
 * Replaces speculative.accept (oxr_runtime/speculative.py:42-48) and the
 * per-sequence bookkeeping of Engine._speculate/_take (engine.py:729-737,
 * 647-664): a = longest prefix with draft[b, j] == predicted[b, j]
 * (j < draft_len[b]); committed[b, :a+1] = predicted[b, :a+1] (rest -1);
 * seq_len[b] += a + 1 (no KV data moves); the committed ids are appended to
 * history[b] (history_len += appended) stopping at eos_id (not appended,
 * finished = 1) or at max_tokens[b] (finished = 2).  Sequences with
 * finished[b] != 0 on entry are left unchanged.  predicted is int64 [B, S]
 * (the greedy ids of the verify step); committed is int32 [B, k+1].
 * Optional (nullable): max_tokens, committed, num_committed, seq_len,
 * history (+ history_len), finished.  eos_id < 0 disables the EOS stop.
 */
int oxr_accept(const int32_t* draft, const int32_t* draft_len, int32_t k, const int64_t* predicted,
               int32_t tokens_per_seq, int32_t batch, int32_t eos_id, const int32_t* max_tokens, int32_t* accepted,
               int32_t* committed, int32_t* num_committed, int32_t* seq_len, int32_t* history,
               int64_t history_stride, int32_t* history_len, int32_t* finished, oxr_stream_t stream);

/*
 * (2) Fused q/k RMSNorm + NeoX RoPE + paged KV-cache write.
 * Replaces kernels.qk_norm_rope_store / _launch (oxr_runtime/kernels.py:102-130):
 * qkv bf16 [n, (H + 2*KV) * 128]; q_weight, k_weight bf16 [128]; cos, sin bf16
 * [n, 64]; slots int64 [n]; k_cache, v_cache bf16 [num_slots, KV, 128] (the
 * reference's [blocks, block_size, KV, 128] viewed flat).  Writes q_out bf16
 * [n, H, 128] and, when k_out / v_out are non-null (need_kv=True), contiguous
 * k_out / v_out bf16 [n, KV, 128].  num_slots = blocks * block_size; a slot
 * outside [0, num_slots) is skipped instead of written out of bounds.  Rounding chain and the sum-of-squares
 * addition tree follow kernels.py:31-63 and 133-165; rsqrt is 1/sqrt with
 * both operations correctly rounded.  head_dim must be 128.
 */
int oxr_qk_norm_rope_store(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight,
                           const oxr_bf16* cos, const oxr_bf16* sin, float eps, oxr_bf16* k_cache,
                           oxr_bf16* v_cache, const int64_t* slots, int64_t num_slots, int64_t n, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, oxr_bf16* q_out, oxr_bf16* k_out,
                           oxr_bf16* v_out, oxr_stream_t stream);

/*
 * (2b) The same kernel reading cos/sin straight from the model's RoPE tables:
 * row positions[i] of cos_table / sin_table (bf16 [table_rows, 64]), i.e. the
 * gather rope_cos[positions] of LanguageModel.extend (language.py:204) fused
 * into the kernel.  Positions outside the table are clamped to it.
 */
int oxr_qk_norm_rope_store_at(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight,
                              const oxr_bf16* cos_table, const oxr_bf16* sin_table, int64_t table_rows,
                              const int64_t* positions, float eps, oxr_bf16* k_cache, oxr_bf16* v_cache,
                              const int64_t* slots, int64_t num_slots, int64_t n, int32_t num_heads,
                              int32_t num_kv_heads, int32_t head_dim, oxr_bf16* q_out, oxr_bf16* k_out,
                              oxr_bf16* v_out, oxr_stream_t stream);

/*
 * RMSNorm of rows (language.py:69-72): out = bf16(w * bf16(x * 1/sqrt(mean(x^2) + eps))),
 * fp32 statistics.  x bf16 [rows, ldx]; hidden a multiple of 512 up to 4096.
 * Used for the decoder norms after the residual add has been fused into the
 * preceding GEMM (OXR_EPI_ADD_RESIDUAL).  out is [rows, ldo], or, with
 * out_packed != 0, in the packed layout of (4c) (16-row tiles, row length
 * hidden, room for the rows rounded up to 16; ldo unused) -- the X operand of
 * oxr_gemm_bf16_packed with OXR_GEMM_X_PACKED.  The same holds for the two
 * norms below.
 */
int oxr_rms_norm(const oxr_bf16* x, int64_t ldx, int64_t rows, int64_t hidden, const oxr_bf16* weight, float eps,
                 oxr_bf16* out, int64_t ldo, int32_t out_packed, oxr_stream_t stream);

/*
 * Embedding gather + first RMSNorm of the verify forward: residual[i] =
 * table[ids[i]] (decode_graph.py:164 embed_tokens(ids)), out[i] =
 * rms_norm(residual[i]) (language.py:253-255, layer 0's input norm).  Ids
 * outside [0, vocab) are clamped.  residual and out are bf16 [rows, hidden].
 */
int oxr_embed_rms_norm(const int64_t* ids, int64_t rows, const oxr_bf16* table, int64_t vocab, int64_t hidden,
                       const oxr_bf16* weight, float eps, oxr_bf16* residual, oxr_bf16* out, int32_t out_packed,
                       oxr_stream_t stream);

/*
 * Embedding lookup (the reference's nn.Embedding embed_tokens, language.py:155),
 * as the eager decode and verify paths call it before building a DecodeBatch /
 * ExtendBatch (engine.py:595, 717; decode_graph.py:75, 164): out[i] =
 * table[ids[i]], bf16 [rows, ldo].  Ids outside [0, vocab) are clamped (the
 * reference callers pass ids.clamp(min=0), model.py:32).
 */
int oxr_embed_gather(const int64_t* ids, int64_t rows, const oxr_bf16* table, int64_t vocab, int64_t hidden,
                     oxr_bf16* out, int64_t ldo, oxr_stream_t stream);

/*
 * Residual add + RMSNorm from GEMM partials (_add_rms_norm, language.py:94-99):
 * residual = bf16(bf16(sum_s partials[s]) + residual) in place, then out =
 * rms_norm(residual) as oxr_rms_norm.  partials fp32 [k_splits, rows, hidden]
 * (from oxr_gemm_bf16_partial), summed in split order.
 */
int oxr_add_partials_rms_norm(const float* partials, int32_t k_splits, int64_t rows, int64_t hidden,
                              oxr_bf16* residual, const oxr_bf16* weight, float eps, oxr_bf16* out,
                              int32_t out_packed, oxr_stream_t stream);

/*
 * The same with the residual read from residual_in and the sum stored to residual (the two may be
 * the same buffer): the norm after oxr_mlp_block, which leaves the new residual in a second buffer.
 */
int oxr_add_partials_rms_norm_from(const float* partials, int32_t k_splits, int64_t rows, int64_t hidden,
                                   const oxr_bf16* residual_in, oxr_bf16* residual, const oxr_bf16* weight,
                                   float eps, oxr_bf16* out, int32_t out_packed, oxr_stream_t stream);

/*
 * A decoder layer's MLP block in one launch (DecoderLayer._mlp, language.py:266-269, with
 * _add_rms_norm 94-99 and _silu_mul 102-104), for 1..32 token rows of the config-5 decoder
 * (hidden 2048, intermediate 6144) on an MI355X in its single-partition mode (256 CUs, 8 XCDs):
 *   residual_out = bf16(bf16(sum_s o_partials[s]) + residual_in)      (o_splits = 4 or 8 slices)
 *   h = rms_norm(residual_out) * post_norm, as oxr_add_partials_rms_norm (same bits)
 *   act = bf16(bf16(silu(bf16(h gate^T))) * bf16(h up^T))
 *   partials_out[x] = act[:, 768 x : 768 x + 768] @ down[:, 768 x : 768 x + 768]^T, x = 0..7 (fp32
 *   [8, rows, 2048], summed in slice order by the next oxr_add_partials_rms_norm[_from]).
 * gate_up_interleaved: the fused gate_up weight [2 * 6144, 2048] with its rows interleaved by 8
 * (row 16 j + i is gate row 8 j + i for i < 8, up row 8 j + i - 8 otherwise), then packed
 * (oxr_pack_weight_bf16); down: down_proj [2048, 6144] packed.  residual_out must not be
 * residual_in (every XCD reads each input row while one writes the output row).
 * workspace: oxr_mlp_block_workspace_bytes() bytes, 256-byte aligned, zero before the first call;
 * each call leaves its control words zero again, so one workspace serves every later call on its
 * stream (calls that overlap on one GPU race).  Word 512 (uint32) of the workspace is an error
 * word the kernel ORs into when workgroup placement or a wait inside the launch fails (the
 * launch then ends with undefined outputs); it stays set until the caller clears it.
 * OXR_ERR_UNSUPPORTED for other shapes or devices (oxr_mlp_block_supported says which).
 */
size_t oxr_mlp_block_workspace_bytes(void);
int oxr_mlp_block_supported(int64_t rows, int64_t hidden, int64_t intermediate, int32_t o_splits);
int oxr_mlp_block(const float* o_partials, int32_t o_splits, const oxr_bf16* residual_in, int64_t rows,
                  int64_t hidden, int64_t intermediate, const oxr_bf16* post_norm, float eps,
                  const oxr_bf16* gate_up_interleaved, const oxr_bf16* down, oxr_bf16* residual_out,
                  float* partials_out, void* workspace, size_t workspace_bytes, oxr_stream_t stream);

/*
 * (3) Multi-query causal paged attention of the verify step.
 * Replaces attention.paged_extend (oxr_runtime/attention.py:96-109); math as
 * the reference test stub (tests/test_language_fused.py:19-28, 50-57):
 * q bf16 [B, S, H, 128]; k_cache, v_cache bf16 [num_blocks, block_size, KV,
 * 128]; seq_lens int32 [B] (including the S new tokens, whose K/V are already
 * in the cache); block_table int32 [B, table_stride].  Token s of sequence b
 * attends keys [0, seq_lens[b] - S + s] of kv head h / (H / KV) with scores
 * q.k * scale and an fp32 softmax; out bf16 [B, S, H, 128].
 * Requires H % KV == 0, S * (H / KV) <= 32, block_size a power of two >= 16,
 * max_seq_len <= table_stride * block_size; contexts longer than max_seq_len
 * are clamped to it.  workspace: at least
 * oxr_paged_extend_workspace_bytes(batch, KV, max_seq_len) bytes of device
 * memory for the context split's partials (no initial contents needed; calls
 * that overlap in time must not share a workspace).  A workspace sized for a
 * batch serves every smaller batch (smaller batches split their contexts
 * further; the size is the largest need up to `batch`).
 */
size_t oxr_paged_extend_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len);
int oxr_paged_extend(const oxr_bf16* q, const oxr_bf16* k_cache, const oxr_bf16* v_cache, const int32_t* seq_lens,
                     const int32_t* block_table, int64_t table_stride, int32_t batch, int32_t tokens_per_seq,
                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     int64_t num_blocks, int32_t max_seq_len, float scale, oxr_bf16* out, void* workspace,
                     size_t workspace_bytes, oxr_stream_t stream);

/*
 * (3b) (2b) followed by (3) in one launch: the attention block of the decoder
 * layer's extend (oxr_runtime/language.py:311-316: kernels.qk_norm_rope_store
 * from _attention_inputs, language.py:260-263, then attention.paged_extend)
 * without the q round trip through memory.  Takes the qkv
 * projection bf16 [B * S, H + 2 KV, 128] of the S new tokens of each sequence
 * (token b * S + s) with the arguments of (2b) (no k_out / v_out) and of (3)
 * (no q).  Each new token's K (normed, rotated) and V are stored at its slot
 * exactly as (2b) stores them, by the workgroup whose keys contain its position
 * seq_lens[b] - S + s, before that workgroup reads them; slots must hold the
 * cache locations of those positions under block_table (as the verify step
 * assembles them).  A slot outside [0, num_slots) is not stored, as in
 * (2b), but the token's computed K/V still take part in the attention.
 * Same requirements and workspace as (3), and also
 * tokens_per_seq <= 16 with tokens_per_seq * (H / KV + 2) <= 64; bit-identical
 * q, cache rows and output to (2b) then (3).
 */
int oxr_qk_norm_rope_paged_extend(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight,
                                  const oxr_bf16* cos_table, const oxr_bf16* sin_table, int64_t table_rows,
                                  const int64_t* positions, float eps, oxr_bf16* k_cache, oxr_bf16* v_cache,
                                  const int64_t* slots, int64_t num_slots, const int32_t* seq_lens,
                                  const int32_t* block_table, int64_t table_stride, int32_t batch,
                                  int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t block_size, int64_t num_blocks, int32_t max_seq_len, float scale,
                                  oxr_bf16* out, int32_t out_packed, void* workspace, size_t workspace_bytes,
                                  oxr_stream_t stream);

/*
 * (3c) Balanced context pieces for (3) and (3b).  No counterpart in the
 * reference (its flash-attn kernel schedules work itself); for batches whose
 * contexts differ in length, where (3) and (3b) cut every context into the
 * same number of pieces and the longest context bounds the launch.
 * oxr_paged_extend_plan writes, on the stream, a plan of
 * oxr_paged_extend_plan_ints(...) int32 entries from the device seq_lens (the
 * arguments are those of the launch the plan is for; 0 entries: the launch
 * keeps every context in one piece and needs no plan).  The planned launches
 * take the plan written for the same seq_lens, batch, tokens_per_seq, heads
 * and max_seq_len: every context is cut into pieces of about the batch's mean
 * share, long contexts taking the workgroups short ones leave spare (each
 * workgroup keeps its partials in its own slot of the same workspace).  The
 * planned calls take the plan's length (plan_ints) and refuse a shorter one.
 * The plan's header records the batch and split count it was written for; a
 * launch whose batch or split count differs (another max_seq_len or
 * tokens_per_seq) ignores it and runs on even pieces, bit-identical to (3) /
 * (3b).  A plan written from other seq_lens whose pieces do not reach a
 * context's end, or that names pieces outside the launch, makes that
 * sequence's output rows NaN; nothing is addressed outside the launch's
 * arrays.  Same
 * arguments, requirements and workspace as (3) and (3b) otherwise; outputs
 * within the same tolerance (the pieces differ, so the fp32 merge order does),
 * and the planned (3b) is bit-identical to the planned (3).
 */
size_t oxr_paged_extend_plan_ints(int32_t batch, int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads,
                                  int32_t max_seq_len);
int oxr_paged_extend_plan(const int32_t* seq_lens, int32_t batch, int32_t tokens_per_seq, int32_t num_heads,
                          int32_t num_kv_heads, int32_t max_seq_len, int32_t* plan, size_t plan_ints,
                          oxr_stream_t stream);
int oxr_paged_extend_planned(const oxr_bf16* q, const oxr_bf16* k_cache, const oxr_bf16* v_cache,
                             const int32_t* seq_lens, const int32_t* block_table, int64_t table_stride, int32_t batch,
                             int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t block_size, int64_t num_blocks, int32_t max_seq_len, float scale, oxr_bf16* out,
                             void* workspace, size_t workspace_bytes, const int32_t* plan, size_t plan_ints,
                             oxr_stream_t stream);
int oxr_qk_norm_rope_paged_extend_planned(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight,
                                          const oxr_bf16* cos_table, const oxr_bf16* sin_table, int64_t table_rows,
                                          const int64_t* positions, float eps, oxr_bf16* k_cache, oxr_bf16* v_cache,
                                          const int64_t* slots, int64_t num_slots, const int32_t* seq_lens,
                                          const int32_t* block_table, int64_t table_stride, int32_t batch,
                                          int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads,
                                          int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                          int32_t max_seq_len, float scale, oxr_bf16* out, int32_t out_packed,
                                          void* workspace, size_t workspace_bytes, const int32_t* plan,
                                          size_t plan_ints, oxr_stream_t stream);

/*
 * (3b') (3b) without a workspace argument, allocating nothing.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops or harnesses that forbid allocation).
 * The split partials live in a static device array of
 * oxr_static_scratch_bytes() bytes (16.25 MiB) that each GPU the library runs
 * on holds until the process ends.  Every shape (3b) accepts fits it (a launch
 * splits contexts into at most 1020 partial units); a shape whose partials
 * exceeded it would return
 * OXR_ERR_SCRATCH_LIMIT.  The array's device address is looked
 * up on the first call on each device, which must therefore not be inside a
 * stream capture.  All calls on one GPU share the array: calls that overlap in
 * time on one GPU race.  Arguments and results otherwise as (3b).
 */
size_t oxr_static_scratch_bytes(void);
int oxr_qk_norm_rope_paged_extend_static(const oxr_bf16* qkv, const oxr_bf16* q_weight, const oxr_bf16* k_weight,
                                         const oxr_bf16* cos_table, const oxr_bf16* sin_table, int64_t table_rows,
                                         const int64_t* positions, float eps, oxr_bf16* k_cache, oxr_bf16* v_cache,
                                         const int64_t* slots, int64_t num_slots, const int32_t* seq_lens,
                                         const int32_t* block_table, int64_t table_stride, int32_t batch,
                                         int32_t tokens_per_seq, int32_t num_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                         int32_t max_seq_len, float scale, oxr_bf16* out, int32_t out_packed,
                                         oxr_stream_t stream);

/*
 * (4a) Weight-streaming bf16 GEMM Y = X * W^T with a fused epilogue.
 * Replaces the nn.Linear projections of the verify forward (language.py:261
 * qkv_proj, 268 o_proj, 269 gate_up_proj/down_proj) together with the
 * elementwise op that follows each:
 *   OXR_EPI_STORE        y = bf16(x @ w^T)                          y [m, n]
 *   OXR_EPI_SILU_MUL     w holds 2n rows (gate then up, language.py:238);
 *                        y = bf16(bf16(silu(bf16(g))) * bf16(u))      y [m, n]
 *                        (_silu_mul, language.py:102-104)
 *   OXR_EPI_ADD_RESIDUAL y = bf16(bf16(x @ w^T) + y), in place: the residual
 *                        add of _add_rms_norm (language.py:94-99)
 * x bf16 [m, ldx] (first k columns used), w bf16 [rows, k] row-major, fp32
 * accumulation.  m <= 256 (one launch per 64 rows over the same weight), k a
 * multiple of 128, x and w 16-byte aligned.
 */
#define OXR_EPI_STORE 0
#define OXR_EPI_SILU_MUL 1
#define OXR_EPI_ADD_RESIDUAL 3
int oxr_gemm_bf16(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w, int64_t k, int64_t n,
                  int32_t epilogue, oxr_bf16* y, int64_t ldy, oxr_stream_t stream);

/*
 * (4a') The same GEMM for weights too narrow to fill the chip with whole-K
 * tiles (o_proj, down_proj): k is split across workgroups and each split's
 * fp32 sums are written to partials [k_splits, m, n]; nothing else is stored.
 * k_splits must equal oxr_gemm_bf16_partial_splits(n, k).  The residual add
 * + RMSNorm that follows consumes them (oxr_add_partials_rms_norm).
 */
int32_t oxr_gemm_bf16_partial_splits(int64_t n, int64_t k);
int oxr_gemm_bf16_partial(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w, int64_t k, int64_t n,
                          float* partials, int32_t k_splits, oxr_stream_t stream);

/*
 * (4b) LM head GEMM with fused vocab-wide argmax.
 * Replaces LanguageModel.logits (language.py:213-214) followed by
 * argmax(dim=-1) (decode_graph.py:167, engine.py:726): logits = hidden @
 * weight^T in fp32, rounded to bf16, and predicted[i] = the first index of
 * the largest bf16 logit of row i (NaN counts as largest, -0 == +0).
 * hidden bf16 [m, hidden_size]; weight bf16 [vocab, hidden_size]; predicted
 * int64 [m].  logits (optional, bf16 [m, vocab]) receives the bf16 logits.
 * m <= 64 (up to 256 with oxr_lm_head_argmax_packed and hidden_size 512,
 * 1024 or 2048: one launch then reads the weight once for all rows);
 * hidden_size a multiple of 128.  workspace: at least
 * oxr_lm_head_workspace_bytes(m, vocab) bytes (per-tile maxima; for more
 * than 32 rows also room for the rows repacked).
 */
size_t oxr_lm_head_workspace_bytes(int64_t m, int64_t vocab);
int oxr_lm_head_argmax(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight, int64_t hidden_size, int64_t vocab,
                       oxr_bf16* logits, int64_t* predicted, void* workspace, size_t workspace_bytes,
                       oxr_stream_t stream);

/*
 * (4d) Argmax of logits the caller holds: logits.argmax(dim=-1) of the eager
 * verify path (engine.py:726) and of the acceptance workload's fp32 logits.
 * logits [rows, ld] of dtype OXR_DTYPE_F32 or OXR_DTYPE_BF16 (the first
 * `vocab` columns of each row are compared); predicted int64 [rows] = the
 * first index of the largest value (NaN counts as largest, -0 == +0), as
 * torch.argmax.  workspace: oxr_argmax_workspace_bytes(rows, vocab) bytes
 * (per-chunk maxima; no initial contents needed).  rows <= 65535.
 */
#define OXR_DTYPE_F32 0
#define OXR_DTYPE_BF16 1
size_t oxr_argmax_workspace_bytes(int64_t rows, int64_t vocab);
int oxr_argmax(const void* logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t ld, int64_t* predicted,
               void* workspace, size_t workspace_bytes, oxr_stream_t stream);

/*
 * (3c) Variable-length (prefill) attention.  Replaces attention.varlen
 * (oxr_runtime/attention.py:47-59): sequences concatenated along the token
 * axis, q bf16 [T, num_heads, 128], k and v bf16 [T, num_kv_heads, 128],
 * cu_seqlens int32 [num_seqs + 1] (sequence i is tokens [cu[i], cu[i+1]),
 * every length <= max_len).  Within each sequence, query token j of head h
 * attends keys [0, j] when causal != 0, else all keys, of kv head
 * h / (num_heads / num_kv_heads); scores q.k * scale, fp32 softmax, output
 * bf16 [T, num_heads, 128].  num_heads / num_kv_heads must be 1, 2, 4 or 8.
 * Causal launches hand out work through counters in the library's static
 * device memory, one of 16 sets per launch in turn: at most 16 causal launches
 * may run at once on one device.
 */
int oxr_varlen_attention(const oxr_bf16* q, const oxr_bf16* k, const oxr_bf16* v, const int32_t* cu_seqlens,
                         int32_t num_seqs, int32_t max_len, int32_t num_heads, int32_t num_kv_heads,
                         int32_t head_dim, int32_t causal, float scale, oxr_bf16* out, oxr_stream_t stream);

/*
 * (4c) Packed weights and token rows.  The reference keeps nn.Linear weights row-major
 * ([rows, k], language.py:234-245 and the LM head of :213-214); these entry
 * points take the same weights re-ordered once, at load time, into the order
 * the GEMM kernels consume them: for each 16-row tile t and 128-column step q,
 * four contiguous 1 KiB blocks, block i holding, for lane l = 16g + r,
 * w[16t + r][128q + 32i + 8g .. +8).  Every load instruction of the kernels
 * then reads 1 KiB of contiguous memory.  The last tile is zero-padded, so a
 * packed weight holds oxr_packed_weight_elems(rows, k) bf16 elements.
 * The *_packed GEMM entries behave exactly like their row-major versions
 * (same requirements, bit-identical results) given oxr_pack_weight_bf16 of
 * the same weight; OXR_EPI_SILU_MUL additionally needs n % 16 == 0.
 */
size_t oxr_packed_weight_elems(int64_t rows, int64_t k);
int oxr_pack_weight_bf16(const oxr_bf16* w, int64_t rows, int64_t k, oxr_bf16* packed, oxr_stream_t stream);
/*
 * Token rows may travel between kernels in the same layout (16-token tiles,
 * row length k, rows past m padding): flags OXR_GEMM_X_PACKED (x packed; ldx
 * unused) and OXR_GEMM_Y_PACKED (y packed with row length n, a multiple of
 * 128; ldy unused; OXR_EPI_STORE and OXR_EPI_SILU_MUL).  Producers of packed
 * rows: the norms' out_packed, oxr_qk_norm_rope_paged_extend's out_packed
 * and OXR_GEMM_Y_PACKED.  A packed [m, k] buffer holds ceil(m / 16) * 16 * k
 * elements.
 */
#define OXR_GEMM_X_PACKED 1
#define OXR_GEMM_Y_PACKED 2
int oxr_gemm_bf16_packed(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w_packed, int64_t k, int64_t n,
                         int32_t epilogue, oxr_bf16* y, int64_t ldy, int32_t flags, oxr_stream_t stream);
int oxr_gemm_bf16_partial_packed(const oxr_bf16* x, int64_t ldx, int64_t m, const oxr_bf16* w_packed, int64_t k,
                                 int64_t n, float* partials, int32_t k_splits, int32_t flags, oxr_stream_t stream);
int oxr_lm_head_argmax_packed(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight_packed, int64_t hidden_size,
                              int64_t vocab, oxr_bf16* logits, int64_t* predicted, void* workspace,
                              size_t workspace_bytes, oxr_stream_t stream);

/*
 * LM head + greedy argmax + acceptance in two launches: oxr_lm_head_argmax_packed followed by
 * oxr_accept, with the argmax's cross-workgroup reduction done by the acceptance launch.
 * Replaces LanguageModel.logits + argmax (language.py:213-214, decode_graph.py:167) and
 * speculative.accept with the engine's rollback (speculative.py:42-48, engine.py:729-737).
 * m = batch * tokens_per_seq token rows (at most 256; tokens_per_seq at most 256), sequence b's
 * rows b * tokens_per_seq .. + tokens_per_seq - 1.  predicted (int64 [m]) receives the greedy
 * ids; every other argument and output is that of oxr_lm_head_argmax_packed (logits are not
 * written) or oxr_accept, with the same results bit for bit.
 */
int oxr_lm_head_accept_packed(const oxr_bf16* hidden, int64_t m, const oxr_bf16* weight_packed, int64_t hidden_size,
                              int64_t vocab, void* workspace, size_t workspace_bytes, int64_t* predicted,
                              const int32_t* draft, const int32_t* draft_len, int32_t k, int32_t tokens_per_seq,
                              int32_t batch, int32_t eos_id, const int32_t* max_tokens, int32_t* accepted,
                              int32_t* committed, int32_t* num_committed, int32_t* seq_len, int32_t* history,
                              int64_t history_stride, int32_t* history_len, int32_t* finished, oxr_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OXR_VERIFY_H */
