// Kernel 3: paged decode attention (one query token per sequence) over a block-table KV cache: the split kernel
// (decode_kernel, the work of decode_body.h's decode_split over its own LDS) and the merge of the sequences it cut
// (decode_merge_kernel). The algorithm and its gfx950 mapping are described in decode_body.h.
#include "decode_body.h"

namespace vox {

namespace {

using namespace dec;

template <int HK, bool BTL>
__global__ __launch_bounds__(kThreads, 2) void decode_kernel(DecodeArgs p) {
  using LDS = LdsOwn<HK, BTL>;
  __shared__ __attribute__((aligned(16))) uint16_t s_vt[kWaves * kTile * Tile<HK>::VROW];  // per-wave V tiles
  __shared__ __attribute__((aligned(16))) float s_slot[LDS::kSlots * kPartialFloats];     // (wave, segment) partials
  __shared__ int s_ctx[kMaxSeqPerLaunch];        // context per sequence, cut to the table's reach
  __shared__ int s_row[kMaxSeqPerLaunch];        // q / output row per sequence
  __shared__ int s_snew[kMaxSeqPerLaunch];       // store mode: the cache slot of each sequence's new token
  __shared__ int s_start[kMaxSeqPerLaunch + 1];  // first step per sequence; s_start[batch] = total steps
  __shared__ int s_wtot[kWaves];
  __shared__ int s_wmax[kWaves];  // most steps of one sequence, per wave
  // the block table, when it fits (no block-id round trips at segment starts); in reuse mode the plan record
  __shared__ __attribute__((aligned(16))) int s_bt[LDS::kBtInts];
  __shared__ int s_rtiles[kRecTiles];  // record mode: the block id of every tile of the range, for the record
  const LDS L{s_vt, s_slot, s_ctx, s_row, s_snew, s_start, s_wtot, s_wmax, s_bt, s_rtiles};
  decode_split<HK>(p, (int)blockIdx.x, (int)gridDim.x, L);
}

// Varlen store mode: merge workgroup B + wid copies rows wid, wid + copy_wgs, ... of new_k / new_v (below copy_rows)
// into the caches at their slots (-1 and slots outside the cache skipped), 16 bytes per lane, each batch's loads
// issued before its stores. It runs after the split's reads, as the per-sequence copy of the non-varlen store does.
// Non-temporal stores: nothing in the step reads the rows back from the cache, and written through L2 the 2.9 MB of a
// config-5 step was still draining when the next launch started (its attention 1.4 us slower; step 47.9 -> 46.8 us).
__device__ __forceinline__ void copy_new_rows(const DecodeArgs& p, int wid) {
  const int row_elems = p.num_heads / p.group * kD;  // HK x 128
  const int pieces = row_elems / 8;                  // 16-byte pieces of a K (or V) row
  const int per_row = 2 * pieces;
  const int64_t nslots = p.num_blocks * p.block_size;
  const int64_t rows = (p.copy_rows - wid + p.copy_wgs - 1) / p.copy_wgs;
  const int64_t total = rows * per_row;
  const int nth = (int)blockDim.x;
  constexpr int kBatch = 4;
  for (int64_t base = threadIdx.x; base < total; base += (int64_t)kBatch * nth) {
    u32x4 val[kBatch];
    int64_t slot[kBatch];
    uint16_t* dst[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t idx = base + (int64_t)u * nth;
      const bool in = idx < total;
      const int64_t r_local = in ? idx / per_row : 0;
      const int rem = (int)(idx - r_local * per_row);
      const int which = rem >= pieces;  // 0: key, 1: value
      const int piece = rem - which * pieces;
      const int64_t row = wid + r_local * p.copy_wgs;
      const uint16_t* src = (which ? p.new_v + row * p.new_v_stride : p.new_k + row * p.new_k_stride) + piece * 8;
      val[u] = in ? ld_g16(src) : zero4();
      slot[u] = in ? (int64_t)p.slot_mapping[row] : -1;
      dst[u] = const_cast<uint16_t*>(which ? p.v_cache : p.k_cache) + piece * 8;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (slot[u] >= 0 && slot[u] < nslots)
        __builtin_nontemporal_store(val[u], reinterpret_cast<u32x4*>(dst[u] + slot[u] * row_elems));
  }
}

// Writes the sequences that decode_kernel left as partials, and the zeros of empty rows (in varlen mode only those of
// one-query sequences; the others belong to the prefill kernel). One workgroup per sequence, thread = (head, 8 dims).
// Sequence b covers steps [sb, eb) of the layout decode_kernel published in `steps`, with the number G of workgroups
// it used; workgroup g of G covers [floor(g S / G), floor((g + 1) S / G)) (at least one step, as G <= S), and the
// workgroups touching b, g_first..g_last in merge_row, each left a partial at slot b + g. Online rescale over the
// partials (fp32), the loads of kMergeBatch partials in flight together. Runs after decode_kernel on the same stream,
// which makes the partials visible. In varlen store mode workgroups past the sequences copy the step's new rows into
// the caches (copy_new_rows).
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs p) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  if (b >= p.batch) {  // (workgroup-uniform) a copy workgroup of the varlen store mode
    copy_new_rows(p, b - p.batch);
    return;
  }
  int s_tot = p.steps[p.batch], s_b = p.steps[b], s_e = p.steps[b + 1], s_g = p.steps[p.batch + 1];
  int c0 = b, c1 = b + 1, slot32 = -1;
  if (p.cu_q) {
    c0 = p.cu_q[b];
    c1 = p.cu_q[b + 1];
  }
  const bool own_row = p.slot_mapping && !p.cu_q;  // store mode: this sequence's row (varlen: the copy workgroups)
  if (own_row) slot32 = p.slot_mapping[b];
  // every value in registers here: the loads go out together, one round trip (left to itself the compiler sinks
  // each load to its first use, behind the branches, one round trip apiece)
  asm volatile("" ::"s"(s_tot), "s"(s_b), "s"(s_e), "s"(s_g), "s"(c0), "s"(c1), "s"(slot32));
  // store mode: the new K / V row goes into the cache, now that every read of the split is done; its load is issued
  // before the merge's and its store made last, so the copy shares the merge's round trip instead of adding its own
  // (a non-temporal store: no later read of this step wants the row in L2)
  u32x4 kv_chunk = zero4();
  uint16_t* kv_dst = nullptr;
  if (own_row) {
    const int row_elems = p.group ? p.num_heads / p.group * kD : 0;  // HK x 128
    const int64_t slot = slot32;
    const int chunk = tid & 127;  // 16-byte chunk of the row: threads 0-127 K, 128-255 V
    if (slot >= 0 && slot < p.num_blocks * p.block_size && chunk * 8 < row_elems) {
      const bool is_v = tid >= 128;
      const uint16_t* src = (is_v ? p.new_v + (int64_t)b * p.new_v_stride : p.new_k + (int64_t)b * p.new_k_stride);
      kv_dst = const_cast<uint16_t*>(is_v ? p.v_cache : p.k_cache) + slot * row_elems + chunk * 8;
      kv_chunk = ld_g16(src + chunk * 8);
    }
  }
  merge_row(p, b, tid, s_tot, s_b, s_e, s_g, c0, c1);
  if (kv_dst) __builtin_nontemporal_store(kv_chunk, reinterpret_cast<u32x4*>(kv_dst));
}

}  // namespace

hipError_t launch_decode_merge(const DecodeArgs& a, hipStream_t stream) {
  const int64_t wgs = (int64_t)a.batch + (a.slot_mapping && a.cu_q && a.copy_rows > 0 ? a.copy_wgs : 0);
  decode_merge_kernel<<<dim3((unsigned)wgs), dim3(256), 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a, int num_kv_heads, hipStream_t stream) {
  const dim3 grid((unsigned)a.grid);
  const bool btl = (int64_t)a.batch * a.max_blocks <= kBtLds;
  if (num_kv_heads == 1 && btl)
    decode_kernel<1, true><<<grid, dim3(kThreads), 0, stream>>>(a);
  else if (num_kv_heads == 1)
    decode_kernel<1, false><<<grid, dim3(kThreads), 0, stream>>>(a);
  else if (btl)
    decode_kernel<2, true><<<grid, dim3(kThreads), 0, stream>>>(a);
  else
    decode_kernel<2, false><<<grid, dim3(kThreads), 0, stream>>>(a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_decode_merge(a, stream);
}

}  // namespace vox
