// The split-KV decode work of one workgroup (decode_split) and the merge of one sequence's partials (merge_row), as
// device functions: decode_attn.hip wraps them in the decode kernels, and the mixed prefill + decode kernel
// (prefill_attn.hip) runs decode_split in the workgroups that take the decode rows of a mixed step.
//
// Semantics (reference call: nanovllm_voxcpm/model/layers.py:350-358, flash_attn_with_kvcache with cache_seqlens and
// block_table, causal, softmax_scale): for every sequence b and query head h,
//   o[b, h] = softmax_j(scale * q[b, h] . K[b, j, h // G]) V[b, j, h // G],   j < context_lens[b],
// where token j lives in cache block block_tables[b, j // block_size] at slot j % block_size, G = H / HK. The same
// code also serves the one-query rows of a paged varlen call (the decode rows of a mixed prefill + decode step,
// reference: nanovllm_voxcpm/model/layers.py:337-348 with block_table): there a sequence's context is its key count
// when it has exactly one query, and its q / output row is cu_seqlens_q[b].
//
// gfx950 mapping.
//  * Work split (persistent, balanced): the tokens of all sequences are cut into 16-token steps, laid end to end in
//    sequence order, and a fixed grid of workgroups (one per CU by default) takes equal contiguous ranges of steps.
//    Every workgroup streams the same number of bytes; it walks its range sequence by sequence. The step layout
//    comes from a scan of context_lens inside the kernel, so the launch shape depends only on host-known sizes
//    (graph capture). The block table is staged in LDS when it fits, so block lookups never wait on memory.
//  * Plan records: the layout depends only on the lengths and block tables, which every layer of a decode step
//    shares. A launch in record mode writes each workgroup's part of it (its range, the sequences it touches, the
//    block id of every tile it walks) into a 4 KiB record of the workspace; a later launch in reuse mode loads its
//    record (one 16-byte load per thread) instead of staging the lengths and the table and scanning them, so its
//    first tile loads go out one round trip after it starts.
//  * A workgroup (4 waves) computes all query heads (<= 16) of a sequence at once. A cache slot row [HK][D] is
//    contiguous (HK * 256 bytes), so the score GEMM contracts over the whole row c = (kv head, d) with a
//    block-diagonal query operand B[c, h] = q[h, d] if c's kv head is h's group else 0: the 16 MFMA columns are 16
//    real heads instead of 8 heads padded to 16, and each K slot row feeds the MFMA A operand straight from global
//    memory (lane = token, 16 contiguous bytes per k-step).
//  * Each wave walks 16-token tiles, issuing all of a tile's loads before waiting on any: S^T[16 tok x 16 heads] = K Q^T
//    (HK*4 MFMA 16x16x32), online softmax in fp32 with exp2, then O^T[c, h] += V^T P^T (MFMA 16x16x16 per 16 output
//    dims and kv head). V is written row-major into a private LDS tile with 16-byte stores and read back transposed
//    by ds_read_b64_tr_b16, which hands each lane four tokens of one column: exactly the A operand. P^T is already in
//    the B layout, no shuffles.
//  * Merging: the four waves of a workgroup merge in LDS. A sequence inside one workgroup's range is written
//    directly; a sequence cut by range boundaries leaves one fp32 partial (O, m, l) per workgroup that touched it,
//    at slot b + g (unique: the (sequence, workgroup) pairs form a monotone staircase), and decode_merge_kernel, next
//    on the stream, combines them. (Merging in the split kernel itself, by the last workgroup to arrive, was measured
//    slower: the arrival atomic and the device-coherent reads of the other pieces, issued after the slowest
//    workgroup's last tile, cost more than this launch's gap and two round trips.)
#pragma once

#include "vox_common.h"
#include "vox_kernels.h"

namespace vox {

namespace {

namespace dec {

constexpr int kD = 128;
constexpr int kTile = 16;              // tokens per wave iteration
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
// The work is balanced in units of one wave tile: with 64-token units a config-4 launch (2700 units over 256
// workgroups) gave some workgroups 11 units and others 10, and the 11-unit ones (10 % more bytes) ended the launch.
constexpr int kMaxHeads = 16;
#ifndef VOX_MAX_PIECES
#define VOX_MAX_PIECES 32
#endif
#ifndef VOX_MERGE_BATCH
#define VOX_MERGE_BATCH 8
#endif
// Most partials one sequence is cut into. A sequence of n steps meets at most about n G / S + 2 of G equal ranges of
// S steps, so a launch uses G' = min(grid, (kMaxPieces - 2) S / n_max) workgroups (the others leave after the layout
// scan): a long sequence among few is not cut into one-step pieces, each a partial for the merge kernel to load.
constexpr int kMaxPieces = VOX_MAX_PIECES;
constexpr int kMergeBatch = VOX_MERGE_BATCH;  // partials whose loads the merge kernel keeps in flight together
constexpr int kMOff = kMaxHeads * kD;          // inside a partial: O [16 heads][128], then m[16], l[16] (log2 domain)
constexpr int kLOff = kMOff + kMaxHeads;

__device__ __forceinline__ f32x4 mfma_16x16x16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// Plan record of one workgroup (int32 offsets). The window holds up to 64 consecutive sequences from wb on: their
// first and end steps, context, q / output row and new-token slot; then the block id of every tile of the range.
constexpr int kRecValid = 0, kRecR = 1, kRecR1 = 2, kRecS = 3, kRecG = 4, kRecWb = 5, kRecBatch = 6, kRecGrid = 7;
constexpr int kRecWin = 16;                       // [kRecWin + 64 a + k]: a = 0 st, 1 en, 2 ctx, 3 row, 4 snew
constexpr int kRecTileOff = kRecWin + 5 * kWave;  // block id of range tile r + i
constexpr int kRecTiles = kPlanRecInts - kRecTileOff;
static_assert(kPlanRecInts == 4 * kThreads, "one 16-byte load per thread loads a record");

template <int HK>
struct Tile {
  static constexpr int ROW = HK * kD;              // elements per cache slot row
  static constexpr int KC = ROW / 32;              // score MFMA k-steps
  static constexpr int VP = kTile * ROW / 8 / 64;  // 16-byte V pieces per lane per tile
  static constexpr int PPR = ROW / 8;              // 16-byte pieces per slot row
  static constexpr int VROW = ROW + 16;            // padded LDS row: the 16 rows a transposed read touches hit distinct banks
  static constexpr int VT_BYTES = kTile * VROW * 2;  // one wave's V tile in LDS
  u32x4 k[KC];
  u32x4 v[VP];
  bool ok;  // the tile's cache block is mapped
};

// Issues the loads of the 16-token tile whose first token sits at cache slot slot0 (a tile never straddles a cache
// block). Every load is unconditional and in bounds, so the compiler can count outstanding loads exactly: the caller
// maps an unmapped block to block 0 and masks what it read. K rows land in MFMA A layout (lane = token r16), V
// pieces coalesced (16 bytes per lane, whole slot rows per instruction; streaming loads, as every tile is read once
// per launch). slot0 is wave-uniform: each load is a
// uniform base plus a per-lane 32-bit byte offset that is the same for every tile (koff, voff) plus an immediate.
template <int HK>
__device__ __forceinline__ void load_tile(Tile<HK>& T, const DecodeArgs& p, int64_t slot0, uint32_t koff,
                                          uint32_t voff) {
  using TT = Tile<HK>;
  const char* kb = reinterpret_cast<const char*>(p.k_cache + slot0 * TT::ROW) + koff;
  const char* vb = reinterpret_cast<const char*>(p.v_cache + slot0 * TT::ROW) + voff;
#pragma unroll
  for (int kc = 0; kc < TT::KC; ++kc) T.k[kc] = ld_g16_stream(kb + kc * 64);
  // V piece i covers 64 / PPR slot rows starting at row i * 64 / PPR: i * 1024 bytes past piece 0 for any HK
#pragma unroll
  for (int i = 0; i < TT::VP; ++i) T.v[i] = ld_g16_stream(vb + i * 1024);
}

// load_tile in store mode: tile row r_new (-1: none) is the step's new token, read from its K / V rows nk / nv
// instead of the cache (the same loads, with the lanes of that row pointed at the new row: no extra load).
template <int HK>
__device__ __forceinline__ void load_tile_new(Tile<HK>& T, const DecodeArgs& p, int64_t slot0, uint32_t koff,
                                              uint32_t voff, int r_new, const uint16_t* nk, const uint16_t* nv) {
  using TT = Tile<HK>;
  const int lane = threadIdx.x & 63;
  const char* kb = reinterpret_cast<const char*>(p.k_cache + slot0 * TT::ROW) + koff;
  const char* vb = reinterpret_cast<const char*>(p.v_cache + slot0 * TT::ROW) + voff;
  // K: lane (row r16, dims jq * 8 + ...): the new row's same dims, at koff less the row offset
  if ((lane & 15) == r_new) kb = reinterpret_cast<const char*>(nk) + (koff - (uint32_t)(r_new * TT::ROW) * 2u);
#pragma unroll
  for (int kc = 0; kc < TT::KC; ++kc) T.k[kc] = ld_g16_stream(kb + kc * 64);
  // V piece i holds slot row i * 64 / PPR + lane / PPR, dims (lane % PPR) * 8
  const char* nvb = reinterpret_cast<const char*>(nv) + (uint32_t)((lane % TT::PPR) * 8) * 2u;
#pragma unroll
  for (int i = 0; i < TT::VP; ++i) {
    const bool mine = i * (64 / TT::PPR) + lane / TT::PPR == r_new;
    T.v[i] = ld_g16_stream(mine ? nvb : vb + i * 1024);
  }
}

// floor((a * b + c) / d) for the step-range bounds (all operands >= 0, d > 0): one 32-bit division when the
// numerator fits in 32 bits, as it does for every real step, instead of the long 64-bit sequence.
__device__ __forceinline__ int64_t muldiv(int64_t a, int64_t b, int64_t c, int64_t d) {
  const uint64_t num = (uint64_t)a * (uint64_t)b + (uint64_t)c;
  if (num <= 0xffffffffull && d <= 0xffffffffll) return (uint32_t)num / (uint32_t)d;
  return (int64_t)(num / (uint64_t)d);
}

// G' of a launch over `steps` steps whose longest sequence has `max_seq_steps`; at most `steps`, so no range is empty
__device__ __forceinline__ int active_workgroups(int grid, int64_t steps, int max_seq_steps) {
  if (max_seq_steps <= 0) return 1;
  const int64_t cap = min(steps, muldiv(kMaxPieces - 2, steps, 0, max_seq_steps));
  return (int)max((int64_t)1, min((int64_t)grid, cap));
}

// A value every lane of the wave holds, moved to a scalar register (LDS reads land in vector registers).
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Where decode_split keeps its LDS state. A workgroup's range is worked in rounds of up to kRoundSegs segments (a
// segment = the part of one sequence inside the range). In a round each wave takes an equal contiguous share of the
// round's tiles, across segment boundaries, and leaves one partial per segment it touched in a slot; one barrier,
// then the workgroup merges the round's segments. Wave w's share follows wave w - 1's, so the (wave, segment) pairs
// of a round form a staircase and pair (w, k) can use slot w + k: kRoundSegs + 3 slots. (With the waves taking a
// segment's tiles in turn instead, every segment ended in a barrier at which the waves with one tile fewer than the
// others waited a whole tile round trip: ~2 us per segment.)
//
// LdsOwn: the decode kernel's own arrays: rounds of 8 segments, fp32 slots, the block table staged when it fits
// (147 KB, one workgroup per CU). The accessors fold to fixed LDS addresses once inlined.
template <int HK, bool BTL>
struct LdsOwn {
  static constexpr int kRoundSegs = 8;
  static constexpr int kSlots = kRoundSegs + kWaves - 1;
  static constexpr bool kBtl = BTL;
  static constexpr int kBtInts = BTL ? (kBtLds > kPlanRecInts ? kBtLds : kPlanRecInts) : kPlanRecInts;
  static constexpr int kSeqCap = kMaxSeqPerLaunch;
  uint16_t* vt_all;  // [kWaves][kTile][VROW]
  float* slots;      // [kSlots][kPartialFloats]
  int *ctx, *row, *snew, *start, *wtot, *wmax, *bt, *rtiles;
  __device__ __forceinline__ uint16_t* vt(int w) const { return vt_all + w * kTile * Tile<HK>::VROW; }
  // wave partial (head r16's O column slice jq, m, l) into slot si
  __device__ __forceinline__ void put(int si, int r16, int jq, const f32x4 (&acc)[8], float m, float l) const {
    float* sl = slots + si * kPartialFloats;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(&sl[r16 * kD + dt * 16 + jq * 4]) = acc[dt];
    if (jq == 0) {
      sl[kMOff + r16] = m;
      sl[kLOff + r16] = l;
    }
  }
  // head hh's dims d0 .. d0 + 8 of slot si, its m and l
  __device__ __forceinline__ void get(int si, int hh, int d0, f32x4 (&o)[2], float& m, float& l) const {
    const float* sl = slots + si * kPartialFloats;
    m = sl[kMOff + hh];
    l = sl[kLOff + hh];
    o[0] = *reinterpret_cast<const f32x4*>(&sl[hh * kD + d0]);
    o[1] = *reinterpret_cast<const f32x4*>(&sl[hh * kD + d0 + 4]);
  }
};

// LdsBorrowed: the decode rows of a mixed launch, sharing the CU with a prefill workgroup. The state lives in the
// prefill role's four 16 KiB tile buffers t0..t3 (wave w's V tile at the start of t_w, then slot w, then small
// arrays) and an area `aux` (slots 4, 5 and the plan record): rounds of 3 segments, slots holding O in bf16 (the
// partials that leave the workgroup stay fp32), the block table read from memory, at most kSeqCap sequences.
template <int HK>
struct LdsBorrowed {
  static constexpr int kRoundSegs = 3;
  static constexpr int kSlots = kRoundSegs + kWaves - 1;
  static constexpr bool kBtl = false;
  static constexpr int kBtInts = kPlanRecInts;
  static constexpr int kSeqCap = 256;
  static constexpr int kSlotBytes = kMaxHeads * kD * 2 + 2 * kMaxHeads * 4;  // O bf16, then m, l fp32
  static constexpr int kTail = Tile<HK>::VT_BYTES + kSlotBytes;               // where a buffer's small arrays start
  static constexpr int kBufBytes = 16384;
  static constexpr int kAuxBytes = 2 * kSlotBytes + kPlanRecInts * 4;
  static_assert(kTail % 16 == 0 && kTail + 2 * kSeqCap * 4 + 8 * 4 <= kBufBytes, "t0 tail: ctx, row, wtot, wmax");
  static_assert(kTail + (2 * kSeqCap + 1) * 4 <= kBufBytes, "t1 tail: snew, start");
  static_assert(kTail + kRecTiles * 4 <= kBufBytes, "t2 tail: rtiles");
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  // the buffers as LDS byte offsets in one register vector, opaque to the optimizer: a choice among the four by a
  // run-time index is then an element select (left as addresses of the arrays, or as four scalars, it became a table
  // in scratch memory)
  u32x4 off4;
  uint8_t* aux;
  int *ctx, *row, *snew, *start, *wtot, *wmax, *bt, *rtiles;
  static __device__ __forceinline__ uint32_t offset_of(uint8_t* p) { return (uint32_t)(uintptr_t)(lds_u8*)p; }
  static __device__ __forceinline__ uint8_t* at(uint32_t off) { return (uint8_t*)(lds_u8*)(uintptr_t)off; }
  __device__ __forceinline__ LdsBorrowed(uint8_t* b0, uint8_t* b1, uint8_t* b2, uint8_t* b3, uint8_t* a)
      : off4(u32x4{offset_of(b0), offset_of(b1), offset_of(b2), offset_of(b3)}), aux(a) {
    asm volatile("" : "+s"(off4));
    ctx = reinterpret_cast<int*>(b0 + kTail);
    row = ctx + kSeqCap;
    wtot = row + kSeqCap;
    wmax = wtot + kWaves;
    snew = reinterpret_cast<int*>(b1 + kTail);
    start = snew + kSeqCap;
    rtiles = reinterpret_cast<int*>(b2 + kTail);
    bt = reinterpret_cast<int*>(aux + 2 * kSlotBytes);
  }
  __device__ __forceinline__ uint8_t* buf(int i) const { return at(off4[i]); }
  __device__ __forceinline__ uint16_t* vt(int w) const { return reinterpret_cast<uint16_t*>(buf(w)); }
  __device__ __forceinline__ uint8_t* slot(int si) const {
    return si < kWaves ? buf(si) + Tile<HK>::VT_BYTES : aux + (si - kWaves) * kSlotBytes;
  }
  __device__ __forceinline__ void put(int si, int r16, int jq, const f32x4 (&acc)[8], float m, float l) const {
    uint8_t* sl = slot(si);
    uint16_t* o = reinterpret_cast<uint16_t*>(sl);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<u32x2*>(&o[r16 * kD + dt * 16 + jq * 4]) =
          u32x2{pack_bf16x2(acc[dt][0], acc[dt][1]), pack_bf16x2(acc[dt][2], acc[dt][3])};
    float* ml = reinterpret_cast<float*>(sl + kMaxHeads * kD * 2);
    if (jq == 0) {
      ml[r16] = m;
      ml[kMaxHeads + r16] = l;
    }
  }
  __device__ __forceinline__ void get(int si, int hh, int d0, f32x4 (&o)[2], float& m, float& l) const {
    const uint8_t* sl = slot(si);
    const u32x4 v = *reinterpret_cast<const u32x4*>(sl + (hh * kD + d0) * 2);
    o[0] = f32x4{bf16_bits_to_float(v[0] & 0xffffu), bf16_bits_to_float(v[0] >> 16), bf16_bits_to_float(v[1] & 0xffffu),
                 bf16_bits_to_float(v[1] >> 16)};
    o[1] = f32x4{bf16_bits_to_float(v[2] & 0xffffu), bf16_bits_to_float(v[2] >> 16), bf16_bits_to_float(v[3] & 0xffffu),
                 bf16_bits_to_float(v[3] >> 16)};
    const float* ml = reinterpret_cast<const float*>(sl + kMaxHeads * kD * 2);
    m = ml[hh];
    l = ml[kMaxHeads + hh];
  }
};

// The split-KV decode work of workgroup g of `grid` (4 waves, kThreads threads), its LDS state in L.
template <int HK, class LDS>
__device__ __forceinline__ void decode_split(const DecodeArgs& p, const int g, const int grid, const LDS& L) {
  using TT = Tile<HK>;
  constexpr bool BTL = LDS::kBtl;
  constexpr int kRoundSegs = LDS::kRoundSegs;
  constexpr int VROW = TT::VROW;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int jq = lane >> 4;
  const int H = p.num_heads;
  const int max_ctx = p.max_blocks * p.block_size;
  const int h = r16;
  // per-lane byte offsets of the tile loads: K row r16, dims jq*8 + [0, 8) (+ 32 per k-step); V piece 0 = row
  // lane / PPR, dims (lane % PPR) * 8 + [0, 8)
  const uint32_t koff = (uint32_t)(r16 * TT::ROW + jq * 8) * 2u;
  const uint32_t voff = (uint32_t)((lane / TT::PPR) * TT::ROW + (lane % TT::PPR) * 8) * 2u;
  const int mb = p.max_blocks;
  const bool varlen = p.cu_q != nullptr;
  const bool store = p.slot_mapping != nullptr;
  int* const s_bt = L.bt;

  // ---- the layout: from this workgroup's plan record (reuse mode), or from a block-wide scan
  int S = 0, G = 1, r = 0, r1 = 0, wb = 0;
  bool use_rec = false;
  // the window: lane k holds sequence wb + k (its steps [w_st, w_en), context, row, new-token slot)
  int w_st = 0, w_en = 0, w_ctx = 0, w_row = 0, w_snew = -1;
  if (p.plan_mode == kPlanReuse) {
    const u32x4 v = ld_g16(p.plan + (int64_t)g * kPlanRecInts + tid * 4);
    *reinterpret_cast<u32x4*>(&s_bt[tid * 4]) = v;
    __syncthreads();
    r = s_bt[kRecR];
    r1 = s_bt[kRecR1];
    S = s_bt[kRecS];
    G = s_bt[kRecG];
    wb = s_bt[kRecWb];
    // a record of this launch shape whose range fits it (the caller vouches for the rest: same lengths and tables)
    use_rec = s_bt[kRecValid] == 1 && s_bt[kRecBatch] == p.batch && s_bt[kRecGrid] == grid && G >= 1 &&
              G <= grid && 0 <= r && r <= r1 && r1 <= S && r1 - r <= kRecTiles &&
              (r == r1 || (0 <= wb && wb < p.batch));
    if (use_rec) {
      w_st = s_bt[kRecWin + lane];
      w_en = s_bt[kRecWin + kWave + lane];
      w_ctx = s_bt[kRecWin + 2 * kWave + lane];
      w_row = s_bt[kRecWin + 3 * kWave + lane];
      w_snew = s_bt[kRecWin + 4 * kWave + lane];
    } else {
      __syncthreads();  // every wave has read the record's flags before the table staging below overwrites them
      S = r = r1 = wb = 0;
      G = 1;
    }
  }

  // sequence bb's context and row: context_lens[bb] and bb, or in varlen mode its key count when it has one query
  auto seq_of = [&](int bb, int& row) -> int {
    if (!varlen) {
      row = bb;
      return p.context_lens[bb];
    }
    const int q0 = p.cu_q[bb], q1 = p.cu_q[bb + 1], k0 = p.cu_k[bb], k1 = p.cu_k[bb + 1];
    row = q0;
    return q1 - q0 == 1 ? k1 - k0 : 0;
  };
  // The sequence holding range position x < S: the last b with start[b] <= x (an empty sequence shares its start
  // with the next one, so the last such b is not empty); a search over chunks of 64 sequences, then inside the chunk.
  // (Lane-parallel ballots over LDS values rather than walks of dependent LDS reads: a binary search and serial walks
  // had taken 2.8 us between the layout and the first tile loads at config 4.)
  auto seq_at = [&](int x) -> int {
    const int nch = (p.batch + kWave - 1) / kWave;  // <= 8 at kMaxSeqPerLaunch
    const int c0 = lane < nch ? L.start[lane * kWave] : INT32_MAX;
    const uint64_t m0 = __builtin_amdgcn_ballot_w64(c0 <= x);  // chunk 0 at least (start[0] = 0)
    const int ch = 63 - __builtin_clzll(m0);
    const int i = ch * kWave + lane;
    const int c1 = i <= p.batch ? L.start[i] : INT32_MAX;  // start[batch] = S > x
    const uint64_t m1 = __builtin_amdgcn_ballot_w64(c1 <= x);
    return ch * kWave + 63 - __builtin_clzll(m1);
  };
  auto load_window = [&]() {  // from the LDS layout, one round trip
    const int sq = wb + lane;
    const bool in = sq < p.batch;
    w_st = in ? L.start[sq] : S;
    w_en = in ? L.start[sq + 1] : S;
    w_ctx = in ? L.ctx[sq] : 0;
    w_row = in ? L.row[sq] : 0;
    w_snew = in && store ? L.snew[sq] : -1;
  };
  auto lane_val = [&](int v, int k) { return __builtin_amdgcn_readlane(v, k); };

  bool rec_write = false;  // record mode: this workgroup's record is valid (its tile block ids are collected)
  int32_t* rec = p.plan + (int64_t)g * kPlanRecInts;
  auto write_record = [&](bool valid) {  // header and window of the record, by one wave
    rec[kRecWin + lane] = w_st;
    rec[kRecWin + kWave + lane] = w_en;
    rec[kRecWin + 2 * kWave + lane] = w_ctx;
    rec[kRecWin + 3 * kWave + lane] = w_row;
    rec[kRecWin + 4 * kWave + lane] = w_snew;
    if (lane < 8) {
      const int hdr[8] = {valid ? 1 : 0, r, r1, S, G, wb, p.batch, grid};
      int v = hdr[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) v = lane == i ? hdr[i] : v;
      rec[lane] = v;
    }
  };
  if (!use_rec) {
    // ---- block table into LDS and the step layout (a block-wide prefix sum over ceil(context / 16)). The lengths
    // of the first kThreads sequences and every table entry a thread stages are loaded before any of them is waited
    // for: one round trip (a load-then-store loop waits for each load in turn, one round trip per kThreads entries).
    int l0 = 0, l1 = 0, l2 = 0, l3 = 0, slot_first = -1;
    if (tid < p.batch) {
      if (varlen) {
        l0 = p.cu_q[tid];
        l1 = p.cu_q[tid + 1];
        l2 = p.cu_k[tid];
        l3 = p.cu_k[tid + 1];
      } else {
        l2 = p.context_lens[tid];
      }
      if (store && !varlen) slot_first = p.slot_mapping[tid];  // (varlen mode finds the new token by position)
    }
    if constexpr (BTL) {
      constexpr int kPer = (kBtLds + kThreads - 1) / kThreads;  // entries per thread at most
      const int nbt = p.batch * mb;
      // entry i = tid + j kThreads sits at row i / mb, column i % mb; one step of kThreads entries moves the row by
      // kThreads / mb and the column by kThreads % mb (with one carry at most)
      const int dq = kThreads / mb, dr = kThreads % mb;
      int row = tid / mb, col = tid % mb;
      int vals[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        vals[j] = tid + j * kThreads < nbt ? p.block_tables[(int64_t)row * p.bt_stride + col] : 0;
        row += dq;
        col += dr;
        if (col >= mb) {
          col -= mb;
          ++row;
        }
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j)
        if (tid + j * kThreads < nbt) s_bt[tid + j * kThreads] = vals[j];
    }
    const int row_first = varlen ? l0 : tid;
    const int ctx_first = !varlen ? l2 : (l1 - l0 == 1 ? l3 - l2 : 0);
    int run = 0;
    int nmax = 0;  // most steps of one sequence
    for (int base = 0; base < p.batch; base += kThreads) {
      const int bb = base + tid;
      int row = row_first;
      const int raw = base == 0 ? ctx_first : (bb < p.batch ? seq_of(bb, row) : 0);
      const int ctx = bb < p.batch ? max(0, min(raw, max_ctx)) : 0;
      const int n = (ctx + kTile - 1) / kTile;
      const int incl = wave_incl_scan(n, lane);
      int wmax = n;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) wmax = max(wmax, __shfl_xor(wmax, o, kWave));
      if (lane == kWave - 1) {
        L.wtot[w] = incl;
        L.wmax[w] = wmax;
      }
      __syncthreads();
      int before = 0, total = 0;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        before += ww < w ? L.wtot[ww] : 0;
        total += L.wtot[ww];
        nmax = max(nmax, L.wmax[ww]);
      }
      if (bb < p.batch) {
        L.ctx[bb] = ctx;
        if (store) L.snew[bb] = varlen ? -1 : base == 0 ? slot_first : p.slot_mapping[bb];
        L.row[bb] = row;
        L.start[bb] = run + before + incl - n;
      }
      run += total;
      __syncthreads();
    }
    if (tid == 0) L.start[p.batch] = run;
    __syncthreads();
    S = uniform(run);
    G = active_workgroups(grid, S, uniform(nmax));
    if (g == 0) {  // the layout decode_merge_kernel reads, then the active workgroup count (a record keeps it)
      for (int i = tid; i <= p.batch; i += kThreads) p.steps[i] = L.start[i];
      if (tid == 0) p.steps[p.batch + 1] = G;
    }
    if (g < G) {
      r1 = (int)muldiv(g + 1, S, 0, G);
      r = (int)muldiv(g, S, 0, G);
      wb = seq_at(r);
      load_window();
    }
    // record mode: the record covers the range when the window reaches past it and the range's tiles fit. An active
    // workgroup collects its tiles' block ids in LDS and writes the record when its range is done: a global store
    // among the tile loads made the compiler's waits for those loads wait for the store too (+2 us per call)
    rec_write = __builtin_amdgcn_readfirstlane(p.plan_mode == kPlanRecord &&
                                               (g < G && lane_val(w_en, kWave - 1) >= r1 && r1 - r <= kRecTiles));
    if (p.plan_mode == kPlanRecord && g >= G && w == 0) write_record(true);  // (no range)
  }

  if (g >= G) return;  // workgroup-uniform; WG 0 (always active) published the layout

  const int hg = h < H ? h / p.group : -1;
  uint16_t* vt = L.vt(w);
  // this lane's transposed-read address inside a d-tile: row jq*4 + r16/4, column 4*(r16%4)
  const uint16_t* vtr = vt + (jq * 4 + (r16 >> 2)) * VROW + 4 * (r16 & 3);
  const float c = p.scale_log2;

  uint64_t segs = 0;  // the round's segments: window lanes of the non-empty sequences it covers
  // block id of range tile t of the sequence at window lane k
  auto block_of = [&](int k, int t) -> int64_t {
    if (use_rec) return uniform(s_bt[kRecTileOff + (t - r)]);
    const int col = (t - lane_val(w_st, k)) * kTile / p.block_size;
    const int bs = wb + k;
    int blk;
    if constexpr (BTL) blk = uniform(s_bt[bs * mb + col]);
    else blk = p.block_tables[(int64_t)bs * p.bt_stride + col];
    if (rec_write && lane == 0) L.rtiles[t - r] = blk;
    return blk;
  };
  // the round's next segment after window lane k
  auto next_seg = [&](int k) { return __builtin_ctzll(k >= 63 ? 0ull : (segs >> (k + 1)) << (k + 1)); };
  auto issue = [&](Tile<HK>& T, int64_t blk, int k, int t) {  // loads of range tile t (window lane k), block blk
    T.ok = blk >= 0 && blk < p.num_blocks;
    const int tok = (t - lane_val(w_st, k)) * kTile;
    const int64_t slot0 = (T.ok ? blk : 0) * p.block_size + (tok % p.block_size);
    if (!store) {
      load_tile<HK>(T, p, slot0, koff, voff);
      return;
    }
    // store mode: the tile holds the new token when its slot lies in [slot0, slot0 + 16), or in varlen mode when it
    // holds the sequence's last key, the position of its one query (the caller's slots are those its tables give
    // the new tokens' positions); unmapped tiles are masked whatever they read
    const int64_t nrow = lane_val(w_row, k);  // the sequence's row of new_k / new_v (b, or its query row)
    const int64_t dn = varlen ? (int64_t)lane_val(w_ctx, k) - 1 - tok : (int64_t)lane_val(w_snew, k) - slot0;
    const int r_new = dn >= 0 && dn < kTile ? (int)dn : -1;
    load_tile_new<HK>(T, p, slot0, koff, voff, r_new, p.new_k + nrow * p.new_k_stride,
                      p.new_v + nrow * p.new_v_stride);
  };
  auto load_q = [&](u32x4 (&qv)[4], int k) {  // query row of head r16: d = kq*32 + jq*8 + [0, 8)
    const uint16_t* qb =
        p.q + (int64_t)lane_val(w_row, k) * p.q_row_stride + (int64_t)(h < H ? h : 0) * kD + jq * 8;
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) qv[kq] = ld_g16(qb + kq * 32);
  };

  int rr = r;   // round start (range position)
  while (rr < r1) {
    // the round: up to kRoundSegs non-empty sequences of the window that end after rr and start before r1 (a round
    // over a window with fewer segments ends at the window's last one; the next round moves the window on)
    if (!use_rec && lane_val(w_en, kWave - 1) <= rr) {
      wb = seq_at(rr);
      load_window();
    }
    const uint64_t cand = __builtin_amdgcn_ballot_w64(w_en > w_st && w_en > rr && w_st < r1);
    const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(cand >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)cand, 0));
    segs = __builtin_amdgcn_ballot_w64(((cand >> lane) & 1ull) && below < kRoundSegs);
    const int nseg = __builtin_popcountll(segs);
    const int k_last = 63 - __builtin_clzll(segs);
    const int re = min(r1, lane_val(w_en, k_last));
    const int R = re - rr;
    auto share_lo = [&](int ww) { return rr + (int)(((int64_t)R * ww) / kWaves); };
    const int t_lo = share_lo(w), t_hi = share_lo(w + 1);
    if (t_lo < t_hi) {
      // this wave's first tile: window lane kcur, round segment kc
      const uint64_t hold = __builtin_amdgcn_ballot_w64(((segs >> lane) & 1ull) && w_st <= t_lo && t_lo < w_en);
      int kcur = __builtin_ctzll(hold);
      int kc = __builtin_popcountll(segs & ((1ull << kcur) - 1ull));
      Tile<HK> T;
      u32x4 qv[4];
      load_q(qv, kcur);
      issue(T, block_of(kcur, t_lo), kcur, t_lo);
      // the tile to issue next (t_lo + 1: window lane ki) and its block id, read one tile ahead
      int ki = kcur;
      if (t_lo + 1 < t_hi && t_lo + 1 >= lane_val(w_en, kcur)) ki = next_seg(kcur);
      int64_t blk_pf = t_lo + 1 < t_hi ? block_of(ki, t_lo + 1) : 0;

      float m = -INFINITY;
      float lsum = 0.f;
      f32x4 acc[8];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
      u32x4 qop[TT::KC];
      bool fresh = true;  // the score operands of sequence bc are still to be built from qv

      // Scores, online softmax and P V of one loaded tile whose first token is t0 of a sequence of ctx tokens. The
      // scale goes into the exp2 argument (one FMA); the running max moves (rescaling acc and lsum) only when the
      // tile max exceeds it by more than 8 in log2 units (p <= 256, exact after the final 1 / l); the masks and zero
      // selects run only on a tile that is not fully valid.
      auto compute = [&](const Tile<HK>& T, int t0, int tok_end, auto&& between) {
        f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < TT::KC; ++kk) s = mfma_16x16x32(T.k[kk], qop[kk], s);
        const bool full = T.ok && t0 + kTile <= tok_end;  // wave-uniform
        // lane (head r16) holds tokens t0 + jq*4 + [0, 4)
        float x[4];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          x[q4] = full || (T.ok && (t0 + jq * 4 + q4) < tok_end) ? s[q4] : -INFINITY;
        // V tile -> LDS, row-major, 16-byte stores; rows of tokens past tok_end or of an unmapped block are zeroed
        // (they meet p = 0 in P V, and unwritten cache slots may hold any bit pattern)
        if (full) {
#pragma unroll
          for (int i = 0; i < TT::VP; ++i) {
            const int pc = i * 64 + lane;
            *reinterpret_cast<u32x4*>(vt + (pc / TT::PPR) * VROW + (pc % TT::PPR) * 8) = T.v[i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < TT::VP; ++i) {
            const int pc = i * 64 + lane;
            const bool ok = T.ok && (t0 + pc / TT::PPR) < tok_end;
            *reinterpret_cast<u32x4*>(vt + (pc / TT::PPR) * VROW + (pc % TT::PPR) * 8) = ok ? T.v[i] : zero4();
          }
        }
        wave_lds_sync();
        between();  // the tile's registers are free: the next tile's loads go out before the softmax and P V

        const float tm = col_max4(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]))) * c;
        const bool up = tm > m + 8.f;
        if (__builtin_amdgcn_ballot_w64(up) != 0) {  // wave-uniform
          const float alpha = up ? fast_exp2(m - tm) : 1.f;  // exp2(-inf) = 0 on the first update
          m = up ? tm : m;
          lsum *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
        }
        const float mu = m == -INFINITY ? 0.f : m;
        float ps = 0.f;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          x[q4] = fast_exp2(fmaf(x[q4], c, -mu));
          ps += x[q4];
        }
        lsum += ps;

        // P^T operand: k-slots jq*4 + [0, 4) = tokens jq*4 + [0, 4)
        const uint32_t p01 = pack_bf16x2(x[0], x[1]);
        const uint32_t p23 = pack_bf16x2(x[2], x[3]);
        const s16x4 pv = __builtin_bit_cast(s16x4, u32x2{p01, p23});
        const s16x4 pz = s16x4{0, 0, 0, 0};
#pragma unroll
        for (int gk = 0; gk < HK; ++gk) {
          const s16x4 pb = (hg == gk) ? pv : pz;
#pragma unroll
          for (int d4 = 0; d4 < 8; d4 += 4) {
            s16x4 va[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) va[u] = lds_read_tr16(vtr + gk * kD + (d4 + u) * 16);
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[d4 + u] = mfma_16x16x16(va[u], pb, acc[d4 + u]);
          }
        }
        wave_lds_sync();
      };

      for (int t = t_lo; t < t_hi; ++t) {
        if (fresh) {  // a new sequence: block-diagonal query operands (kk's kv head kk / 4)
#pragma unroll
          for (int kk = 0; kk < TT::KC; ++kk) qop[kk] = hg == kk / 4 ? qv[kk % 4] : zero4();
          fresh = false;
        }
        compute(T, (t - lane_val(w_st, kcur)) * kTile, lane_val(w_ctx, kcur), [&]() {
          if (t + 1 < t_hi) {
            if (ki != kcur) load_q(qv, ki);
            issue(T, blk_pf, ki, t + 1);
          }
        });
        // then the block id of the tile after it
        if (t + 1 < t_hi) {
          int kn = ki;
          if (t + 2 < t_hi && t + 2 >= lane_val(w_en, ki)) kn = next_seg(ki);
          blk_pf = t + 2 < t_hi ? block_of(kn, t + 2) : 0;
          const bool seq_done = ki != kcur;
          if (seq_done) {  // this wave's share of the current sequence is done: its partial goes to slot w + kc
            L.put(w + kc, r16, jq, acc, m, col_sum4(lsum));
            m = -INFINITY;
            lsum = 0.f;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            fresh = true;
            kcur = ki;
            ++kc;
          }
          ki = kn;
        }
      }
      L.put(w + kc, r16, jq, acc, m, col_sum4(lsum));  // the last sequence of the share
    }
    __syncthreads();  // every wave's partials of the round are in LDS

    // ---- merge the round's segments (fp32); thread (head hh, dims d0 .. d0 + kDpt) ----
    constexpr int kDpt = kMaxHeads * kD / kThreads;  // output dims per thread
    constexpr int kTpr = kD / kDpt;                    // threads per head
    static_assert(kDpt == 8, "a slot read covers 8 dims");
    const int hh = tid / kTpr;
    const int d0 = (tid % kTpr) * kDpt;
    uint64_t rest = segs;
    for (int k = 0; k < nseg; ++k) {
      const int kl = __builtin_ctzll(rest);  // segment k's window lane
      rest &= rest - 1ull;
      const int bs = wb + kl;
      const int sb = lane_val(w_st, kl), eb = lane_val(w_en, kl);
      const int a = max(rr, sb), e = min(re, eb);
      // the waves whose shares hold tiles of this segment, read in one pass (all loads before any use)
      float mw[kWaves], lw[kWaves];
      f32x4 ow[kWaves][kDpt / 4];
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const bool touched = share_lo(ww) < e && share_lo(ww + 1) > a && share_lo(ww) < share_lo(ww + 1);
        // (a slot no wave wrote in this launch holds whatever LDS held: its values are selected away, never scaled)
        f32x4 o2[2];
        float m2, l2;
        L.get(touched ? ww + k : k, hh, d0, o2, m2, l2);
        mw[ww] = touched ? m2 : -INFINITY;
        lw[ww] = touched ? l2 : 0.f;
#pragma unroll
        for (int i = 0; i < kDpt / 4; ++i) ow[ww][i] = touched ? o2[i] : f32x4{0.f, 0.f, 0.f, 0.f};
      }
      float M = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, mw[ww]);
      const float Mu = M == -INFINITY ? 0.f : M;
      float Ls = 0.f;
      f32x4 o[kDpt / 4];
#pragma unroll
      for (int i = 0; i < kDpt / 4; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const float ew = fast_exp2(mw[ww] - Mu);  // 0 (and lw, ow 0) for the waves that did not touch the segment
        Ls += ew * lw[ww];
#pragma unroll
        for (int i = 0; i < kDpt / 4; ++i) o[i] += ew * ow[ww][i];
      }
      if (a == sb && e == eb) {  // the whole sequence is in this workgroup's range: the output itself
        if (hh < H) {
          const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
          const int64_t row = lane_val(w_row, kl);
#pragma unroll
          for (int i = 0; i < kDpt / 4; ++i)
            *reinterpret_cast<u32x2*>(p.out + row * p.out_row_stride + (int64_t)hh * kD + d0 + 4 * i) =
                u32x2{pack_bf16x2(o[i][0] * inv, o[i][1] * inv), pack_bf16x2(o[i][2] * inv, o[i][3] * inv)};
        }
      } else {  // cut by a range boundary: partial for decode_merge_kernel, slot b + g
        float* part = p.partials + (int64_t)(bs + g) * kPartialFloats;
#pragma unroll
        for (int i = 0; i < kDpt / 4; ++i) *reinterpret_cast<f32x4*>(&part[hh * kD + d0 + 4 * i]) = o[i];
        if (tid % kTpr == 0) {
          part[kMOff + hh] = M;
          part[kLOff + hh] = Ls;
        }
      }
    }
    __syncthreads();  // the slots and V tiles are free for the next round
    rr = re;
  }
  if (p.plan_mode == kPlanRecord) {  // the record of this workgroup's range (tile ids collected behind the barrier)
    if (w == 0) write_record(rec_write);
    if (rec_write)
      for (int i = tid; i < r1 - r; i += kThreads) rec[kRecTileOff + i] = L.rtiles[i];
  }
}

// The merge of sequence b's split-KV partials into its output row (decode_merge_kernel).
// steps: the layout's total S, sequence b's first and end steps sb, eb, and the active workgroups G (with S >= 1, none
// has an empty range); [c0, c1): b's query rows (b's row alone outside varlen mode).
__device__ __forceinline__ void merge_row(const DecodeArgs& p, int b, int tid, int64_t S, int64_t sb, int64_t eb,
                                          int64_t G, int c0, int c1) {
  const int hh = tid >> 4;
  const int d0 = (tid & 15) * 8;
  const int H = p.num_heads;
  const int64_t row = c0;
  if (c1 - c0 != 1) return;  // varlen mode: not a one-query row, the prefill kernel writes it
  uint16_t* ob = p.out + row * p.out_row_stride + (int64_t)hh * kD + d0;
  if (hh >= H) return;
  if (eb == sb) {  // empty (padded) row: defined zeros
    *reinterpret_cast<u32x4*>(ob) = zero4();
    return;
  }
  const int g_first = (int)muldiv(sb + 1, G, S - 1, S) - 1;
  const int g_last = (int)min(G - 1, muldiv(eb, G, S - 1, S) - 1);
  if (g_first >= g_last) return;  // one workgroup held the whole sequence and wrote it

  float M2 = -INFINITY, L2 = 0.f;
  float o2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o2[i] = 0.f;
  for (int g0 = g_first; g0 <= g_last; g0 += kMergeBatch) {
    float mc[kMergeBatch], lc[kMergeBatch];
    f32x4 oa[kMergeBatch], obv[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      mc[u] = -INFINITY;
      lc[u] = 0.f;
      oa[u] = obv[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      // loads only up to the sequence's last range: the condition is workgroup-uniform, so the slots past it
      // cost no traffic
      const int64_t gg = g0 + u;
      if (gg <= g_last) {
        const float* pc = p.partials + (b + gg) * kPartialFloats;
        mc[u] = pc[kMOff + hh];
        lc[u] = pc[kLOff + hh];
        oa[u] = *reinterpret_cast<const f32x4*>(&pc[hh * kD + d0]);
        obv[u] = *reinterpret_cast<const f32x4*>(&pc[hh * kD + d0 + 4]);
      }
    }
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const float mn = fmaxf(M2, mc[u]);
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float a = fast_exp2(M2 - mu);
      const float e = fast_exp2(mc[u] - mu);
      L2 = L2 * a + e * lc[u];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o2[i] = o2[i] * a + e * oa[u][i];
        o2[i + 4] = o2[i + 4] * a + e * obv[u][i];
      }
      M2 = mn;
    }
  }
  const float inv = L2 > 0.f ? 1.f / L2 : 0.f;
  *reinterpret_cast<u32x4*>(ob) =
      u32x4{pack_bf16x2(o2[0] * inv, o2[1] * inv), pack_bf16x2(o2[2] * inv, o2[3] * inv),
            pack_bf16x2(o2[4] * inv, o2[5] * inv), pack_bf16x2(o2[6] * inv, o2[7] * inv)};
}

}  // namespace dec

}  // namespace

}  // namespace vox
