// Launch descriptors shared by the kernels and the C-ABI layer (host and device visible, plain data only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vox {

// One decode partial: O[16 heads][128] unnormalized, then m[16] and l[16] (log2 domain).
constexpr int kPartialFloats = 16 * 128 + 16 + 16;
// Sequences one decode launch takes (their step layout lives in LDS); larger batches are launched in slices.
constexpr int kMaxSeqPerLaunch = 512;
// Block-table entries (batch x max_blocks) a decode launch keeps in LDS; wider tables are read from global memory.
constexpr int kBtLds = 3584;
// Decode plan records (int32 per workgroup) and the plan modes of a decode launch: none (the layout from a scan in
// every workgroup), record (the same, and each workgroup writes its record), reuse (each workgroup loads the record
// an earlier launch over the same lengths, tables and slots wrote; a record that does not fit falls back to the scan)
constexpr int kPlanRecInts = 1024;
constexpr int kPlanNone = 0, kPlanRecord = 1, kPlanReuse = 2;

struct DecodeArgs {
  const uint16_t* q;          // bf16 [B, H, 128]; sequence rows q_row_stride apart, heads 128 apart
  int64_t q_row_stride;
  const uint16_t* k_cache;    // bf16 [num_blocks, block_size, HK, 128], contiguous
  const uint16_t* v_cache;
  int64_t num_blocks;
  int block_size;
  const int32_t* block_tables;  // int32 [B, bt_stride], first max_blocks columns used
  int64_t bt_stride;
  int max_blocks;
  const int32_t* context_lens;  // int32 [B]
  int batch;
  int num_heads;
  int group;                  // H / HK
  float scale_log2;           // softmax_scale * log2(e)
  int grid;                   // workgroups of the split kernel (persistent, balanced ranges)
  float* partials;            // [B + grid, kPartialFloats]
  int32_t* steps;             // [B + 2]: first step of every sequence, the total, the active workgroups
  int32_t* plan;              // [grid, kPlanRecInts]: one record per workgroup
  int plan_mode;              // kPlanNone, kPlanRecord (write the records and the steps), kPlanReuse (read them)
  uint16_t* out;              // bf16 [B, H, 128]: sequence rows out_row_stride apart, heads 128 apart
  int64_t out_row_stride;
  // Varlen mode (cu_q != nullptr; context_lens unused): the one-query rows of a varlen call. Sequence b is handled
  // when it has exactly one query (cu_q[b + 1] - cu_q[b] == 1): its keys are the first cu_k[b + 1] - cu_k[b] tokens
  // of its table row, and its q and output row is cu_q[b]. Every other sequence is left alone: no keys, no output.
  const int32_t* cu_q;
  const int32_t* cu_k;
  // Store mode (slot_mapping != nullptr): this step's K/V row of every sequence, bf16 with heads contiguous and rows
  // new_*_stride elements apart, belongs at cache slot slot_mapping[row] (-1 = none), row = b ([B, HK, 128] rows), or
  // in varlen mode row = cu_q[b], the sequence's query row. The split kernel reads the new token from the row instead
  // of the cache: the tile holding slot_mapping[b] takes the row's K and V there, or in varlen mode the tile holding
  // the sequence's last key (the caller's slots being those its tables give the new tokens' positions). The cache
  // writes come after every read: without cu_q the merge kernel writes each sequence's row; in varlen mode merge
  // workgroups [B, B + copy_wgs) copy rows [0, copy_rows) (every row of the step, the prefill rows' too) to their
  // slots. The result is that of storing first and then attending, as long as no sequence's new slot lies inside
  // another sequence's context.
  const int32_t* slot_mapping;
  const uint16_t* new_k;
  const uint16_t* new_v;
  int64_t new_k_stride;
  int64_t new_v_stride;
  int64_t copy_rows;
  int copy_wgs;
};

struct PrefillArgs {
  const uint16_t* q;          // bf16 [T, H, 128]; token rows q_row_stride apart
  int64_t q_row_stride;
  // packed K/V (block_tables == nullptr): bf16 [Tk, HK, 128], token rows *_row_stride apart
  const uint16_t* k_src;
  const uint16_t* v_src;
  int64_t k_row_stride;
  int64_t v_row_stride;
  // paged K/V (block_tables != nullptr): bf16 [num_blocks, block_size, HK, 128], contiguous
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t num_blocks;
  int block_size;
  const int32_t* block_tables;
  int64_t bt_stride;
  int max_blocks;
  // sequences: cu_seqlens (int32 [B + 1]) or, when null, uniform lengths
  const int32_t* cu_q;
  const int32_t* cu_k;
  int uniform_q;
  int uniform_k;
  int batch;
  int num_heads;
  int num_kv_heads;
  int group;                  // H / HK; 128 % group == 0
  float scale_log2;
  int causal;                 // bottom-right aligned: query i of nq sees keys j <= nk - nq + i
  uint16_t* out;              // bf16 [T, H, 128]; token rows out_row_stride apart
  int64_t out_row_stride;
  // int8 output (launch_prefill_int8): per token, o * inv_smooth (inv_smooth fp32 [H * 128] or null) over all
  // heads -> amax; out_q = rint(o * inv_smooth / scale) with scale = max(amax, 1e-6) / 127, out_scale[token] = scale
  const float* inv_smooth;
  int8_t* out_q;              // int8 [T, H * 128]; token rows out_row_stride apart
  float* out_scale;           // fp32 [T]
  int xcd_order;              // set by the launcher: run contiguous (q tile, sequence, kv head) ranges per XCD
  int skip_single;            // sequences with exactly one query are left to the decode kernel (varlen mode)
  int persistent;             // set by the launcher: a fixed grid loops over the (q tile, kv head) items of the
                              // sequences, found by a scan of cu_q (at most kMaxSeqPerLaunch sequences per launch)
  int64_t row_limit;          // > 0: output rows at or past it are neither read (q) nor written (the rows the caller's
                              // output holds; a cu_seqlens_q reaching past it truncates instead of writing out of bounds)
  // KV store riding in a packed launch (vox_prefill_attn_store): rows i < store_rows of k_src / v_src go to cache slot
  // store_slots[i] of store_k_cache / store_v_cache (rows of num_kv_heads * 128; -1 and slots outside
  // [0, store_num_slots) skipped), copied by workgroups [store_first, store_first + store_wgs) (launch order) after
  // their work item
  const int32_t* store_slots;
  uint16_t* store_k_cache;
  uint16_t* store_v_cache;
  int64_t store_rows;         // 0: no store
  int64_t store_num_slots;
  int store_first;
  int store_wgs;
  // paged keys with the step's new keys in rows (launch_mixed with a riding store): sequence b's keys at positions
  // nk - nq and later (its nq new tokens, stored by this launch's merge kernel) come from k_src / v_src rows
  // cu_q[b] + (position - (nk - nq)) instead of the cache; the earlier keys through the block table as usual
  int new_from_rows;
};

struct CopyArgs {
  void* kv;                   // [num_planes][num_blocks][block_size][per_token] elements, contiguous
  int64_t num_planes;         // layers x 2 (K, V)
  int64_t num_blocks;
  int block_size;
  int64_t per_token;          // elements per token slot (kv_heads x head_dim)
  const int32_t* entries;     // int32 [num_entries][3]: src block, dst block, tokens
  int num_entries;
};

hipError_t launch_store_kvcache(const void* k, const void* v, int64_t k_row_stride, int64_t v_row_stride,
                                void* k_cache, void* v_cache, int64_t num_slots, const int32_t* slot_mapping,
                                int64_t n, int row_elems, bool vec16, hipStream_t stream);

hipError_t launch_decode(const DecodeArgs& a, int num_kv_heads, hipStream_t stream);
// The merge kernel alone (after a mixed launch whose decode workgroups left partials).
hipError_t launch_decode_merge(const DecodeArgs& a, hipStream_t stream);

hipError_t launch_prefill(const PrefillArgs& a, int max_seqlen_q, hipStream_t stream);

// A mixed prefill + decode step as one launch: the one-query rows on decode workgroups (d, its workspace set up),
// the other rows on persistent prefill workgroups (a, persistent with skip_single) sharing the CUs, then the merge
// kernel. For the shapes mixed_launch_fits accepts (paged tiles, at most 256 sequences).
bool mixed_launch_fits(const PrefillArgs& a, int num_kv_heads);
hipError_t launch_mixed(const PrefillArgs& a, int max_seqlen_q, const DecodeArgs& d, int num_kv_heads,
                        hipStream_t stream);

hipError_t launch_copy_block_prefix(const CopyArgs& a, int max_tokens, bool vec16, hipStream_t stream);

// The same attention with the int8 epilogue; one workgroup covers every KV group of its tokens (num_kv_heads <= 2).
hipError_t launch_prefill_int8(const PrefillArgs& a, int max_seqlen_q, hipStream_t stream);

// Whether the int8 output is faster as two passes (the bf16 attention kernel into a scratch buffer, then
// launch_quantize_rows) than with the fused epilogue, for a call of this shape.
bool prefill_int8_two_pass(int batch, int max_seqlen_q, int num_heads, int num_kv_heads, int causal);

// Per-token int8 quantization of `rows` bf16 rows of `row_elems` values (contiguous, row_elems a multiple of 8,
// at most 2048): out_q[t] = rint(x[t] * inv_smooth / scale_t), out_scale[t] = scale_t = max(amax_t, 1e-6) / 127.
hipError_t launch_quantize_rows(const uint16_t* x, int64_t rows, int row_elems, const float* inv_smooth, int8_t* out_q,
                                int64_t out_row_stride, float* out_scale, hipStream_t stream);

}  // namespace vox
