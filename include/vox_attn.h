/* libvoxattn: MI355X (gfx950) paged-KV attention for the VoxCPM2 engine, C ABI.
 *
 * The three launch entry points replace the GPU calls that the reference's Attention.forward makes
 * (reference: nanovllm_voxcpm/model/layers.py:326-362). All device buffers are owned by the caller; the library
 * never allocates, frees or synchronizes, so every call is stream-ordered on `stream` (a hipStream_t, NULL = the
 * null stream) and may be captured into a HIP graph. Element types: bf16 tensors are passed as raw pointers to
 * 16-bit words, index tensors are int32. Strides are in elements.
 *
 * Every function returns VOX_OK or an error code; vox_last_error() returns the calling thread's message for the
 * last failure. No function throws.
 */
#ifndef VOX_ATTN_H_
#define VOX_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VOX_ABI_VERSION 13

#define VOX_OK 0
#define VOX_EINVAL 1 /* bad argument: shape, stride, alignment or null pointer (reference: the asserts of
                        nanovllm_voxcpm/model/layers.py:299-302 and kernels/prefill_attn.py:107-108) */
#define VOX_EHIP 2   /* the HIP runtime reported an error at launch */

/* Plan modes of the decode calls (the `plan` argument). The decode layout (how the sequences' tokens are dealt to the
 * workgroups, and the block id of every tile) depends only on the lengths, the block tables and, in store mode, the
 * slots, which every layer of one decode step shares. No reference counterpart: the reference likewise builds
 * per-step metadata once per forward context for all layers (nanovllm_voxcpm/engine/utils.py:53-57).
 *   VOX_PLAN_NONE    every workgroup scans the lengths and stages the table itself
 *   VOX_PLAN_RECORD  the same, and the layout is recorded in the workspace
 *   VOX_PLAN_REUSE   the layout is read from the workspace, where the last VOX_PLAN_RECORD call on it recorded it;
 *                    the caller guarantees that call had the same batch, context lengths (varlen: cu_seqlens), block
 *                    tables, slots (store mode: reuse only after a store-mode record) and workgroup count. Parts of
 *                    the layout a record cannot hold are scanned again. Batches above 512 sequences run unplanned. */
#define VOX_PLAN_NONE 0
#define VOX_PLAN_RECORD 1
#define VOX_PLAN_REUSE 2

const char* vox_last_error(void);
int vox_abi_version(void);

/* KV slot scatter. Replaces store_kvcache / store_kvcache_kernel (reference: nanovllm_voxcpm/model/layers.py:266-305).
 * For each token i < num_tokens with slot = slot_mapping[i] in [0, num_slots): copies the num_kv_heads*head_dim
 * contiguous elements of key row i (rows key_row_stride apart) to k_cache + slot*num_kv_heads*head_dim, and
 * likewise value -> v_cache. slot -1 (padding) is skipped, as in the reference; other out-of-range slots are skipped
 * too instead of writing outside the cache. Bit-exact. */
int vox_store_kvcache(const void* key, const void* value, int64_t key_row_stride, int64_t value_row_stride,
                      void* k_cache, void* v_cache, int64_t num_slots, const int32_t* slot_mapping,
                      int64_t num_tokens, int num_kv_heads, int head_dim, void* stream);

/* Paged decode attention, one query token per sequence. Replaces the decode branch's
 * flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache, cache_seqlens=context_lens, block_table=block_tables,
 * softmax_scale, causal=True) (reference: nanovllm_voxcpm/model/layers.py:349-358).
 *   q            bf16 [batch, num_heads, head_dim], sequence rows q_row_stride apart, heads head_dim apart
 *   k/v_cache    bf16 [num_blocks, block_size, num_kv_heads, head_dim], contiguous
 *   block_tables int32 [batch, bt_stride]; the first max_blocks columns of every row must be readable (the
 *                kernel may stage them all), but entries past ceil(context_lens[b] / block_size) are never used;
 *                an entry inside the context outside [0, num_blocks) masks that block's keys (no weight)
 *   context_lens int32 [batch]; 0 = padded row, whose output is written as zeros
 *   plan         VOX_PLAN_NONE, VOX_PLAN_RECORD or VOX_PLAN_REUSE (above)
 *   workspace    >= vox_decode_workspace_bytes(batch) bytes of scratch, 16-byte aligned: the split-KV partials and
 *                the step layout the two kernels of the call (launched in order on `stream`) pass on, and the plan
 *                records. VOX_PLAN_REUSE reads what the recording call left there, so the workspace must be the
 *                same and untouched by other calls in between; no other contents need to survive a call.
 *   out          bf16 [batch, num_heads, head_dim], contiguous
 * Supported: head_dim 128, num_kv_heads 1 or 2, num_heads <= 16, block_size a multiple of 32. */
int vox_decode_attn(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                    int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                    int max_blocks, const int32_t* context_lens, int batch, int num_heads, int num_kv_heads,
                    int head_dim, float softmax_scale, int plan, void* workspace, size_t workspace_bytes,
                    void* out, void* stream);

/* The decode step's KV store and decode attention in one call: vox_store_kvcache(key, value, key_row_stride,
 * value_row_stride, k_cache, v_cache, num_blocks * block_size, slot_mapping, batch, ...) followed by
 * vox_decode_attn(...) (reference: the decode branch of nanovllm_voxcpm/model/layers.py:326-358, store_kvcache then
 * flash_attn_with_kvcache), without the store's own launch: the split kernel reads each sequence's new token from
 * key / value where the tile it loads holds that token's slot, and writes the rows into the caches. Same results as
 * the two calls when no slot_mapping[b] lies inside another sequence's context (the engine's sequences each write
 * only their own last block); slot -1 and slots outside the cache store nothing.
 *   key / value    bf16 [batch, num_kv_heads, head_dim], heads contiguous, rows *_row_stride elements apart
 *                  (multiples of 8), 16-byte aligned
 *   slot_mapping   int32 [batch]
 * Other arguments as vox_decode_attn. */
int vox_decode_attn_store(const void* q, int64_t q_row_stride, const void* key, const void* value,
                          int64_t key_row_stride, int64_t value_row_stride, const int32_t* slot_mapping,
                          void* k_cache, void* v_cache, int64_t num_blocks, int block_size,
                          const int32_t* block_tables, int64_t bt_stride, int max_blocks, const int32_t* context_lens,
                          int batch, int num_heads, int num_kv_heads, int head_dim, float softmax_scale, int plan,
                          void* workspace, size_t workspace_bytes, void* out, void* stream);

/* vox_decode_attn without the workspace argument: the split-KV scratch is a static device array of 16 MiB
 * (16777216 bytes) that each GPU the library runs on holds until the process ends, so the
 * call allocates nothing (no hipMalloc, no allocator call of any kind). No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture that must not touch an allocator, tight serving loops).
 * Returns VOX_EINVAL when vox_decode_workspace_bytes(batch) exceeds the array (not for any batch at the default
 * workgroup count: batches are launched 512 sequences at a time). Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams, or host threads) race and must be serialized by the caller.
 * The array needs no clearing: each call writes every scratch value it reads. Runs with VOX_PLAN_NONE. Other
 * arguments as vox_decode_attn. */
int vox_decode_attn_noalloc(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                            int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                            int max_blocks, const int32_t* context_lens, int batch, int num_heads, int num_kv_heads,
                            int head_dim, float softmax_scale, void* out, void* stream);

/* Workspace bytes vox_decode_attn needs for `batch` sequences on the current device. No reference
 * counterpart: flash-attn sizes its split-KV buffers internally (reference call site: nanovllm_voxcpm/model/layers.py:350). */
size_t vox_decode_workspace_bytes(int batch);

/* Workgroups the decode split kernel runs on the current device (one per CU), and a process-wide override for tuning
 * and tests (0 restores the built-in choice; change it only between calls, the workspace size depends on it). No
 * reference counterpart. */
int vox_decode_workgroups(void);
void vox_set_decode_workgroups(int workgroups);

/* Varlen attention for prefill steps. Replaces flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q,
 * max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True, block_table) (reference: nanovllm_voxcpm/model/layers.py:
 * 337-348), the Triton paged_prefill_attention / short_causal_attention in bf16 mode (reference:
 * nanovllm_voxcpm/kernels/prefill_attn.py:98-124, kernels/short_attn.py:156-179), and, with causal = 0 and uniform
 * lengths, flash_attn_func(q, k, v, softmax_scale, causal=False) (reference: nanovllm_voxcpm/model/layers.py:361).
 *   q              bf16 [T, num_heads, head_dim], token rows q_row_stride apart
 *   key/value      packed bf16 [Tk, num_kv_heads, head_dim] rows (used when block_tables is NULL)
 *   k/v_cache      paged bf16 [num_blocks, block_size, num_kv_heads, head_dim] (used when block_tables != NULL)
 *   cu_seqlens_q/k int32 [batch + 1]; both NULL selects uniform lengths uniform_seqlen_q / uniform_seqlen_k
 *   causal         bottom-right aligned: query i of a sequence with nq queries and nk keys sees keys j <= nk-nq+i
 *   out            bf16 [T, num_heads, head_dim], token rows out_row_stride apart
 *   plan, workspace
 *                  NULL, or a decode workspace (>= vox_prefill_workspace_bytes(batch) bytes, under vox_decode_attn's
 *                  contract) and its plan mode: with block tables and cu_seqlens, sequences with exactly one query (the
 *                  decode rows of a mixed prefill + decode step) then run on the split-KV decode kernel, which spreads
 *                  long contexts over every CU (needs num_heads <= 16, num_kv_heads 1 or 2, block_size a multiple of
 *                  32, out 16-byte aligned with out_row_stride a multiple of 8; otherwise, or with NULL, the prefill
 *                  kernel takes every row). Calls of up to 256 sequences over blocks of a multiple of 64 tokens run
 *                  both kinds of rows in one launch, sharing every CU. Results within the same tolerance either way.
 * Supported: head_dim 128, num_heads / num_kv_heads dividing 128. */
int vox_prefill_attn(const void* q, int64_t q_row_stride, const void* key, const void* value,
                     int64_t key_row_stride, int64_t value_row_stride, const void* k_cache, const void* v_cache,
                     int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                     int max_blocks, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch,
                     int max_seqlen_q, int uniform_seqlen_q, int uniform_seqlen_k, int num_heads, int num_kv_heads,
                     int head_dim, float softmax_scale, int causal, void* out, int64_t out_row_stride, int plan,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Scratch bytes vox_prefill_attn's one-query rows need for `batch` sequences on the current device. No reference
 * counterpart (flash-attn sizes its buffers internally; reference call site: nanovllm_voxcpm/model/layers.py:337). */
size_t vox_prefill_workspace_bytes(int batch);

/* A packed prefill step's KV store and its attention in one call: vox_store_kvcache(key, value, key_row_stride,
 * value_row_stride, k_cache, v_cache, num_slots, slot_mapping, num_tokens, num_kv_heads, head_dim) followed by
 * vox_prefill_attn over the packed rows key / value (no block table) (reference: the prefill branch of
 * nanovllm_voxcpm/model/layers.py:326-348 without a block table, store_kvcache then flash_attn_varlen_func over the
 * step's own k and v). The attention reads the packed rows, not the cache, so the copy rides in the attention launch
 * (the last workgroups copy the rows after their own work) instead of a launch of its own. Outputs and caches are
 * identical to the two calls. Rows the 16-byte copy cannot move (16-byte aligned rows, strides multiples of 8) take
 * the two calls. Arguments as in those two functions; num_tokens = the rows of key / value and slot_mapping. */
int vox_prefill_attn_store(const void* q, int64_t q_row_stride, const void* key, const void* value,
                           int64_t key_row_stride, int64_t value_row_stride, const int32_t* slot_mapping,
                           void* k_cache, void* v_cache, int64_t num_slots, int64_t num_tokens,
                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int max_seqlen_q,
                           int num_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal, void* out,
                           int64_t out_row_stride, void* stream);

/* A paged prefill step's KV store and its attention in one call: vox_store_kvcache(key, value, key_row_stride,
 * value_row_stride, k_cache, v_cache, num_blocks * block_size, slot_mapping, num_tokens, num_kv_heads, head_dim)
 * followed by vox_prefill_attn over the caches through block_tables (reference: the prefill branch of
 * nanovllm_voxcpm/model/layers.py:326-348 with a block table, store_kvcache then flash_attn_varlen_func over
 * k_cache / v_cache; the mixed steps of nanovllm_voxcpm/engine/scheduler.py:340 (_ride) take this branch).
 * With blocks of a multiple of 64 tokens and rows 16-byte aligned with strides multiples of 8 (below 2^24 elements),
 * the store rides in the attention launch: each sequence's new keys (its last nq key positions) are read from the
 * rows key / value (row cu_seqlens_q[b] + i for the i-th) instead of the cache, and the rows are written into the
 * caches after the reads: by the merge kernel when the call runs as one mixed launch (vox_prefill_attn's conditions:
 * workspace, up to 256 sequences, some sequence with more than one query), else, when it runs on the prefill kernel
 * alone (no workspace), by the launch's last workgroups. That equals the two calls when, as the engine's scheduler
 * guarantees, slot_mapping holds for each sequence's new tokens the slots its block table gives their positions, and
 * no sequence's new slots lie inside another sequence's context. Otherwise (a workspace whose call is not one mixed
 * launch, other block sizes, other rows) the two calls run. Outputs and caches are identical to the two calls;
 * num_tokens = the rows of key / value and slot_mapping; plan as vox_prefill_attn's, except that a REUSE call needs a
 * record made by this function (records hold the new tokens' slots). */
int vox_prefill_attn_store_paged(const void* q, int64_t q_row_stride, const void* key, const void* value,
                                 int64_t key_row_stride, int64_t value_row_stride, const int32_t* slot_mapping,
                                 int64_t num_tokens, void* k_cache, void* v_cache, int64_t num_blocks, int block_size,
                                 const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int max_seqlen_q,
                                 int num_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal,
                                 void* out, int64_t out_row_stride, int plan, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* vox_prefill_attn with the int8 output epilogue the W8A8 o_proj consumes. Replaces the quant=True modes of the
 * Triton paged_prefill_attention, short_causal_attention and short_attention (reference:
 * nanovllm_voxcpm/kernels/prefill_attn.py:84-92 and :98-124, kernels/short_attn.py:55-64, :70-90, :137-146, :156-179;
 * caller kernels/fused_layer.py:698-730). Per token t, with o the fp32 attention output over all heads:
 *   x = o * inv_smooth (inv_smooth fp32 [num_heads * head_dim], NULL = 1), amax = max(max_c |x[c]|, 1e-6),
 *   out_scale[t] = amax / 127,   out_q[t, c] = rint(x[c] / out_scale[t])  (round half to even, int8).
 *   out_q      int8 [T, num_heads * head_dim], token rows out_q_row_stride apart (multiple of 4, 4-byte aligned)
 *   out_scale  fp32 [T]
 *   num_tokens T, the query rows (cu_seqlens_q[batch], or batch * uniform_seqlen_q) that out_q, out_scale and
 *              the workspace hold; rows at or past it are neither read nor written, so a cu_seqlens_q reaching past
 *              it truncates the output instead of writing out of bounds (0: nothing to do)
 *   workspace  NULL, or >= vox_prefill_int8_workspace_bytes(...) bytes of scratch (16-byte aligned): where that is
 *              nonzero the call runs as two passes (the bf16 kernel into the workspace, then a per-token
 *              quantization of its rows), which is faster for long sequences whose work items outnumber the CUs;
 *              the codes then come from the bf16-rounded o (as the reference's flash-attn + quantize path computes
 *              them) instead of the fp32 accumulators, within one code step of each other
 * Other arguments as vox_prefill_attn. Supported: num_kv_heads 1 or 2 (one workgroup holds all heads of its tokens). */
int vox_prefill_attn_int8(const void* q, int64_t q_row_stride, const void* key, const void* value,
                          int64_t key_row_stride, int64_t value_row_stride, const void* k_cache, const void* v_cache,
                          int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                          int max_blocks, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch,
                          int max_seqlen_q, int uniform_seqlen_q, int uniform_seqlen_k, int num_heads,
                          int num_kv_heads, int head_dim, float softmax_scale, int causal, const float* inv_smooth,
                          void* out_q, int64_t out_q_row_stride, float* out_scale, int64_t num_tokens,
                          void* workspace, size_t workspace_bytes, void* stream);

/* A prefill step's KV store and its int8-output attention in one call: vox_store_kvcache(key, value, key_row_stride,
 * value_row_stride, k_cache, v_cache, num_blocks * block_size, slot_mapping, store_rows, num_kv_heads, head_dim)
 * followed by vox_prefill_attn_int8, over the packed rows key / value (block_tables NULL) or over the caches through
 * block_tables. Replaces the W8A8 layer's store_kvcache + short_causal_attention(quant=True) pair (the head-start step
 * of a burst) and its store_kvcache + paged_prefill_attention(quant=True) pair (eager prefix-cache steps) (reference:
 * nanovllm_voxcpm/kernels/fused_layer.py:643-667 and :619-641). The copy rides in the int8 launch (the last
 * workgroups copy the rows after their own work; in the two-pass form, in the bf16 pass); with block tables the launch
 * reads each sequence's new keys (its last nq key positions) from the rows instead of the cache, which equals the two
 * calls when, as the engine guarantees, slot_mapping holds the slots the tables give those positions and no sequence's
 * new slots lie inside another sequence's context. Outputs and caches identical to the two calls; rows the 16-byte
 * copy cannot move, and block sizes other than multiples of 64 with block tables, take the two calls. Arguments as in
 * those two functions (k_cache / v_cache [num_blocks, block_size, HK, head_dim]; store_rows = the rows of key / value
 * and slot_mapping, num_tokens = the query rows). */
int vox_prefill_attn_int8_store(const void* q, int64_t q_row_stride, const void* key, const void* value,
                                int64_t key_row_stride, int64_t value_row_stride, const int32_t* slot_mapping,
                                int64_t store_rows, void* k_cache, void* v_cache, int64_t num_blocks, int block_size,
                                const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int max_seqlen_q,
                                int num_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal,
                                const float* inv_smooth, void* out_q, int64_t out_q_row_stride, float* out_scale,
                                int64_t num_tokens, void* workspace, size_t workspace_bytes, void* stream);

/* Scratch bytes for vox_prefill_attn_int8's two-pass form for a call of this shape: num_tokens * num_heads *
 * head_dim * 2 where the two passes are the faster form, 0 where the fused epilogue is (then pass NULL). No
 * reference counterpart (the reference's quant kernels allocate their outputs only). */
size_t vox_prefill_int8_workspace_bytes(int64_t num_tokens, int batch, int max_seqlen_q, int num_heads,
                                        int num_kv_heads, int head_dim, int causal);

/* Copy the first n token slots of KV-cache blocks in every (layer, K/V) plane, in one launch. Replaces
 * copy_kv_block_prefix (reference: nanovllm_voxcpm/kernels/kv_copy.py:17-41; callers model/runner.py:232-248,
 * model/engine.py:383-452).
 *   kv          2-byte elements [num_planes, num_blocks, block_size, per_token], contiguous (the engine's
 *               [layers, 2, blocks, block_size, kv_heads, head_dim] tensor: num_planes = layers * 2,
 *               per_token = kv_heads * head_dim)
 *   entries     device int32 [num_entries, 3]: (src block, dst block, n tokens); n is clipped to block_size and
 *               n <= 0 does nothing; entries with a block outside [0, num_blocks) are skipped
 *   max_tokens  an upper bound of the entries' n (sizes the launch; host-known, as the reference's grid)
 * Bit-exact. Entries that write a block another entry of the same call reads race, as in the reference. */
int vox_copy_kv_block_prefix(void* kv, int64_t num_planes, int64_t num_blocks, int block_size, int64_t per_token,
                             int elem_bytes, const int32_t* entries, int num_entries, int max_tokens, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VOX_ATTN_H_ */
