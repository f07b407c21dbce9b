// Kernel 2: varlen (optionally causal) GQA attention for prefill steps, on bf16 MFMA.
//
// Semantics (reference calls: nanovllm_voxcpm/model/layers.py:337-348 flash_attn_varlen_func, with or without
// block_table; :361 flash_attn_func for the non-causal short rows; the Triton paged_prefill_attention and
// short_causal_attention of nanovllm_voxcpm/kernels/prefill_attn.py:20-124 and kernels/short_attn.py:95-179):
// sequence b has nq = cu_q[b+1] - cu_q[b] queries and nk = cu_k[b+1] - cu_k[b] keys; with `causal` query i sees keys
// j <= nk - nq + i (bottom-right aligned), o = softmax(scale * q k^T) v in fp32, stored as bf16. Keys come from the
// paged cache through block_tables, or from packed [Tk, HK, D] rows when there is no block table.
//
// gfx950 mapping. A workgroup owns 128 query rows = (128 / G tokens) x (the G query heads of one kv head), as 4 waves
// of 32 rows on grids above 2048 workgroups, else 8 waves of 16; grids that fit two workgroups per CU take 64-row
// workgroups of 4 waves of 16. GQA shares every K/V tile across the group's heads.
// Per 64-key tile K and V go from global memory straight into LDS (range-checked buffer loads with the lds bit: no
// register staging; rows past the keys and unmapped blocks read as zeros), double-buffered, with the 16-byte chunks
// of each 256-byte row permuted so that the fragment reads meet no bank conflicts; each wave computes
// S^T[64 keys x its rows] = K Q^T with Q^T held in registers, an online softmax in fp32 (exp2, log2-prescaled scale),
// and O^T[128 d x rows] += V^T P^T, where P^T comes out of the score MFMA already in B-operand layout and V^T is read
// with ds_read_b64_tr_b16 (two transposed reads give a lane the 8 keys of one d column). The next tile's loads are
// issued before the current tile is computed and waited for only at the tile's one barrier; in paged mode the
// sequence's block-table row is held across the wave's lanes (one column per lane) and each tile's block id taken
// with v_readlane. The causal / length mask is only evaluated on tiles that reach past the first query's position or
// past the keys. Large grids deal contiguous work ranges per XCD, so the query tiles that re-read a sequence's K/V
// find it in that XCD's L2. (Paged caches whose block size is not a multiple of 64 stage per-piece loads through
// registers instead.)
//
// int8 output (QUANT; reference: the QUANT epilogues of kernels/prefill_attn.py:84-92 and kernels/short_attn.py:
// 55-64, 137-146): the o_proj GEMM takes o per token as int8 plus one fp32 scale over all heads, so a workgroup then
// holds the same query tokens for every KV group (one 4-wave half per group, each with its own K/V tiles; the
// halves step through the key tiles together). The epilogue multiplies the normalized fp32 o by inv_smooth, takes
// the per-token max |.| across both halves (LDS atomic max on the float bits, all values >= 0), and writes
// rint(o / scale) (round half to even) with scale = max(amax, 1e-6) / 127.
#include <type_traits>

#include "decode_body.h"
#include "vox_common.h"
#include "vox_kernels.h"

namespace vox {

namespace {

constexpr int kD = 128;
constexpr int kBK = 64;          // keys per tile
constexpr int kTB = kBK * 256;   // bytes of one K or V tile in LDS (the direct-to-LDS path)
constexpr int kRows = 128;       // query rows per workgroup (bf16 output)
// LDS row strides (bf16 elements) of the K and V tiles, chosen by measuring the kernel's own access patterns on
// gfx950: the K-fragment 16-byte reads run 1.7x faster at 144 than at 136 (and 4-8x faster than at 128 or 132),
// the transposed V reads are fastest from 152 up; the 16-byte staging writes do not care.
constexpr int kKsStride = kD + 16;
constexpr int kVsStride = kD + 24;
// word 3 of a raw buffer descriptor (32-bit data format; offsets in bytes, range-checked against num_records)
constexpr int kBufferWord3 = 0x00020000;
constexpr unsigned kXcds = 8;                  // MI355X: workgroups are dealt round-robin over 8 XCDs
constexpr unsigned kXcdOrderMinWorkgroups = 1024;
// Grids of up to this many workgroups take 8-wave workgroups (measured, bf16 output, causal: 1 x 512 tokens 14.5 ->
// 12.2 us, 44 x 46 paged over a 50-token prefix -4 %, 16 x 512 -3 %, 4 x 2048 -4 %, 2 x 8192 -3 %; at 4096
// workgroups (16 x 2048, 64 x 512) the 4-wave form is 2-3 % faster).
constexpr int64_t kSmallGridWorkgroups = 2048;
// Grid forms of prefill_kernel (below)
constexpr int kFormGrid = 0;
constexpr int kFormPersistent = 1;
constexpr int kFormRanked = 2;

// Where a workgroup's keys come from (one kernel instance each, so no path's loop-carried state constrains another's
// load waits): packed [Tk, HK, D] rows; the paged cache with block_size a multiple of 64 (a 64-key tile lies in one
// block: one block id per tile); the paged cache with any other block size (one block id per 16-byte piece).
enum KvSource { kPacked = 0, kPagedTiles = 1, kPagedPieces = 2, kPagedTilesNew = 3, kPagedTilesRows = 4 };
// kPagedTilesNew: paged tiles whose sequences' new keys come from the step's rows (PrefillArgs::new_from_rows; the
// mixed launch with a riding store), an instance of its own so the other paged launches keep their registers.
// kPagedTilesRows: the same for the plain and rank-major prefill forms, whose items with no cached key (nk == nq) run
// a tile loop of their own that reads only the rows.
constexpr bool kv_tiles(int kv) { return kv == kPagedTiles || kv == kPagedTilesNew || kv == kPagedTilesRows; }

// NW waves per KV group, each owning RT 16-row blocks of the 128 query rows: 4 waves x 32 rows keep the LDS reads per
// MFMA low (the largest grids); 8 waves x 16 rows halve each wave's work per key tile, which shortens a workgroup's
// chain of key tiles (smaller grids, where the longest chains end the launch).
// The double-buffered K and V tiles of the direct-to-LDS path ([NH] = one per KV-group half), four distinct __shared__
// arrays of the kernel: the compiler can then tell a tile's reads from the next tile's in-flight DMA writes (a
// mixed launch's decode workgroups use the same arrays for their own state).
template <int NH>
struct DmaBufs {
  uint8_t (*k0)[kTB];
  uint8_t (*k1)[kTB];
  uint8_t (*v0)[kTB];
  uint8_t (*v1)[kTB];
};

// One work item: query tile qt of sequence b, kv head gz (QUANT: every kv head, one per half of the workgroup).
template <bool QUANT, int KV, int NW, int RT>
__device__ __forceinline__ void prefill_tile(const PrefillArgs& p, int qt, int b, int gz,
                                             const DmaBufs<QUANT ? 2 : 1>& bufs) {
  constexpr int NH = QUANT ? 2 : 1;  // KV-group halves per workgroup
  constexpr int ROWS = 16 * RT * NW;  // query rows per KV group
  constexpr int NT = 64 * NW;        // threads per KV group
  constexpr int PR = 4 * NW;         // tile rows one load instruction of the group covers (16 bytes per thread)
  constexpr int NP = kBK / PR;       // load instructions per thread per 64-key tile
  __shared__ __attribute__((aligned(16))) uint16_t ks_all[NH][kBK][kKsStride];
  __shared__ __attribute__((aligned(16))) uint16_t vs_all[NH][2][kBK][kVsStride];  // V double-buffered
  __shared__ unsigned s_amax[QUANT ? ROWS : 1];  // QUANT: per token of the tile, float bits of max |o|
  // per-piece path: whether each key of the staged tile lies in a mapped block (an unmapped block's keys are masked)
  __shared__ __attribute__((aligned(16))) unsigned char s_keyok[NH][KV == kPagedPieces ? kBK : 4];

  const int half = QUANT ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / NT)) : 0;  // wave-uniform
  const int g = QUANT ? half : gz;
  auto& ks = ks_all[half];
  auto& vs2 = vs_all[half];
  // the sequence bounds, and (paged tiles) the sequence's block-table row beside them rather than after them: lane c
  // holds column c (c < 64), so the loop takes each tile's block id with v_readlane instead of a load. (A load per
  // tile, one tile ahead, made the compiler wait for it, and with it for the next tile's DMA, right after issuing
  // both: every step waited a full DMA round trip before its scores.)
  int q0, nq, k0, nk;
  int bid0 = 0;     // column 0, for the first tile's DMA (a scalar load: the DMA need not wait for the row's lanes)
  int bt_row = -1;
  {
    int q1, k1;
    q0 = b * p.uniform_q;
    q1 = q0 + p.uniform_q;
    k0 = b * p.uniform_k;
    k1 = k0 + p.uniform_k;
    if (p.cu_q) {
      q0 = p.cu_q[b];
      q1 = p.cu_q[b + 1];
    }
    if (p.cu_k) {
      k0 = p.cu_k[b];
      k1 = p.cu_k[b + 1];
    }
    if constexpr (kv_tiles(KV)) {
      bid0 = p.block_tables[(int64_t)b * p.bt_stride];
      const int col = (int)(threadIdx.x & 63);
      if (col < p.max_blocks) bt_row = p.block_tables[(int64_t)b * p.bt_stride + col];
    }
    nq = q1 - q0;
    nk = k1 - k0;
  }
  const int nk_all = nk;  // the sequence's keys (its new ones the last nq)
  if (KV != kPacked) nk = min(nk, p.max_blocks * p.block_size);  // keys the block table can address
  const int G = p.group;
  const int BQ = ROWS / G;  // query tokens per workgroup
  if (qt * BQ >= nq || (p.skip_single && nq == 1)) return;  // (one-query rows: the decode kernel's, in varlen mode)

  const int tid = threadIdx.x & (NT - 1);  // thread within the half
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  if constexpr (QUANT)
    if (threadIdx.x < (unsigned)BQ) s_amax[threadIdx.x] = 0u;  // ordered before the atomics by the barriers below
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int jq = lane >> 4;
  const int HK = p.num_kv_heads;

  // This lane's RT query rows (one per 16-row MFMA column tile): rho = w*16*RT + rt*16 + r16.
  u32x4 qop[RT][4];
  bool row_ok[RT];
  int qpos[RT];
  int tq_of[RT];
  int h_of[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int rho = (w * RT + rt) * 16 + r16;
    const int tq = qt * BQ + rho / G;
    const int h = g * G + rho % G;
    tq_of[rt] = tq;
    h_of[rt] = h;
    row_ok[rt] = tq < nq && (p.row_limit <= 0 || (int64_t)q0 + tq < p.row_limit);
    qpos[rt] = nk - nq + tq;
    const uint16_t* qp = p.q + (int64_t)(q0 + tq) * p.q_row_stride + (int64_t)h * kD + jq * 8;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) qop[rt][kc] = row_ok[rt] ? ld_g16(qp + kc * 32) : zero4();
  }

  const int tq_last = min(nq, (qt + 1) * BQ) - 1;
  const int kv_end = p.causal ? min(nk, nk - nq + tq_last + 1) : nk;

  float m[RT], l[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m[rt] = -INFINITY;
    l[rt] = 0.f;
  }
  f32x4 acc[8][RT];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[dt][rt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- K/V tile pieces: piece i of a tile is key lrow + PR i, dims dc .. dc + 8 (16 bytes per thread). Packed keys
  // and paged tiles inside one cache block (block_size a multiple of 64) go straight to LDS (the DMA path below);
  // other block sizes read each piece's block id one tile ahead (fetch_bids) and stage through registers.
  constexpr bool paged = KV != kPacked;
  constexpr bool blk_tiles = kv_tiles(KV);
  const int rs_k = paged ? HK * kD : (int)p.k_row_stride;  // elements between consecutive keys (< 2^24)
  const int rs_v = paged ? HK * kD : (int)p.v_row_stride;
  const int lrow = tid >> 4;
  const int dc = (tid & 15) * 8;
  u32x4 kr[NP], vr[NP];
  int bids[NP];  // per-piece block ids (paged, block_size not a multiple of 64)
#pragma unroll
  for (int i = 0; i < NP; ++i) bids[i] = 0;
  int tile_bid = 0;            // the block id of the next tile to load (paged, block_size a multiple of 64)
  unsigned live = 0;           // bit i: piece i is a real key
  auto fetch_bids = [&](int kv0) {
    if constexpr (!paged) return;
    if constexpr (blk_tiles) {
      const int col = min(kv0, nk - 1) / p.block_size;  // wave-uniform
      tile_bid = col < 64 ? __builtin_amdgcn_readlane(bt_row, col)
                          : p.block_tables[(int64_t)b * p.bt_stride + col];  // tables wider than 64 columns
      return;
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int jc = min(kv0 + lrow + PR * i, nk - 1);
      bids[i] = p.block_tables[(int64_t)b * p.bt_stride + jc / p.block_size];
    }
  };
  // register-staged loads (block sizes that are not a multiple of 64): unconditional and in bounds (a key past nk
  // reads the sequence's last key, an unmapped block reads block 0; both are zeroed when staged, and the keys of an
  // unmapped block are flagged for the mask)
  unsigned mapped = 0;         // bit i: piece i's block is mapped
  auto load_tile = [&](int kv0) {
    live = 0;
    mapped = 0;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int jj = kv0 + lrow + PR * i;
      const int jc = min(jj, nk - 1);
      const int64_t blk = bids[i];
      const bool inb = blk >= 0 && blk < p.num_blocks;
      const bool ok = jj < nk && inb;
      const int64_t off = (((ok ? blk : 0) * p.block_size + jc % p.block_size) * HK + g) * kD + dc;
      kr[i] = ld_g16(p.k_cache + off);
      vr[i] = ld_g16(p.v_cache + off);
      live |= (ok ? 1u : 0u) << i;
      mapped |= (inb ? 1u : 0u) << i;
    }
  };
  auto stage_tile = [&](int vb) {
    auto& vs = vs2[vb];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int pc = tid + i * NT;
      const bool ok = (live >> i) & 1u;
      *reinterpret_cast<u32x4*>(&ks[pc >> 4][(pc & 15) * 8]) = ok ? kr[i] : zero4();
      *reinterpret_cast<u32x4*>(&vs[pc >> 4][(pc & 15) * 8]) = ok ? vr[i] : zero4();
      if constexpr (KV == kPagedPieces)
        if ((pc & 15) == 0) s_keyok[half][pc >> 4] = (unsigned char)((mapped >> i) & 1u);
    }
  };
  // this lane's transposed-read address inside a 16-key x 16-d block: row jq*4 + r16/4, column 4*(r16%4)
  const int tr_off = (jq * 4 + (r16 >> 2)) * kVsStride + 4 * (r16 & 3);
  const int first_pos = nk - nq + qt * BQ;  // the position of the tile's first query token

  // ---- per-tile steps of the register-staged path (padded LDS rows; V double-buffered, K single-buffered)
  auto scores = [&](f32x4 (&sc)[4][RT]) {  // S^T[key][row] = K Q^T
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) sc[kt][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&ks[kt * 16 + r16][kc * 32 + jq * 8]);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sc[kt][rt] = mfma_16x16x32(a, qop[rt][kc], sc[kt][rt]);
      }
    }
    // keep four fragment reads in flight ahead of the MFMAs that consume them
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, RT, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4 * RT, 0);
  };
  // The causal / length mask, only where the tile reaches past the first query's position or past the keys.
  // Key j = kv0 + kt*16 + jq*4 + rr is kept when j < nk and (causal) j <= qpos: one limit per row, relative to the
  // lane's first key, so each element costs a compare against a constant and a select.
  auto mask = [&](f32x4 (&sc)[4][RT], int kv0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int last = (p.causal ? min(nk - 1, qpos[rt]) : nk - 1) - (kv0 + jq * 4);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sc[kt][rt][rr] = kt * 16 + rr <= last ? sc[kt][rt][rr] : -INFINITY;
    }
  };
  // Online softmax, one row per lane column, branch-free. The scale goes into the exp2 argument (one FMA); a row's
  // running max moves only when its tile max exceeds it by more than 8 in log2 units (p <= 256, exact after the
  // final 1 / l), so most tiles leave the accumulators alone. Returns whether any row of the wave moved; alpha is
  // the factor (1 for rows that did not move) that the accumulators, which still hold the previous tile's P V at
  // the old max, need once that P V has been added.
  auto softmax = [&](f32x4 (&sc)[4][RT], u32x4 (&pbo)[2][RT], float (&alpha)[RT]) -> bool {
    const float c = p.scale_log2;
    bool any_up = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float t = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        t = fmaxf(t, fmaxf(fmaxf(sc[kt][rt][0], sc[kt][rt][1]), fmaxf(sc[kt][rt][2], sc[kt][rt][3])));
      const float tm = col_max4(t) * c;  // scaled (log2) units; c > 0
      const bool up = tm > m[rt] + 8.f;
      any_up = any_up || up;
      alpha[rt] = up ? fast_exp2(m[rt] - tm) : 1.f;  // exp2(-inf) = 0 on a row's first update
      m[rt] = up ? tm : m[rt];
      const float mu = m[rt] == -INFINITY ? 0.f : m[rt];
      float s4[4];  // the row sum as a tree (depth 4, not a chain of 16 dependent adds)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sc[kt][rt][rr] = fast_exp2(fmaf(sc[kt][rt][rr], c, -mu));
        s4[kt] = (sc[kt][rt][0] + sc[kt][rt][1]) + (sc[kt][rt][2] + sc[kt][rt][3]);
      }
      l[rt] = l[rt] * alpha[rt] + ((s4[0] + s4[1]) + (s4[2] + s4[3]));
    }
    // P^T B operands; k-step k2 covers keys k2*32 + {jq*4 + [0,4), 16 + jq*4 + [0,4)} for lane jq, the order in
    // which the score MFMA left them in the lane's registers
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        pbo[k2][rt] = u32x4{pack_bf16x2(sc[2 * k2][rt][0], sc[2 * k2][rt][1]),
                            pack_bf16x2(sc[2 * k2][rt][2], sc[2 * k2][rt][3]),
                            pack_bf16x2(sc[2 * k2 + 1][rt][0], sc[2 * k2 + 1][rt][1]),
                            pack_bf16x2(sc[2 * k2 + 1][rt][2], sc[2 * k2 + 1][rt][3])};
    return __builtin_amdgcn_ballot_w64(any_up) != 0;
  };
  // Softmax against the running max as it stands (no tile max, no cross-lane step): p = exp2(s c - m). Valid
  // while every p stays <= 2^62, which the lane's partial row sums (each at least its largest term) check;
  // otherwise the caller redoes the tile through softmax (tile max, rescale). ps gets the lane's partial row sums.
  // Returns whether any lane of the wave failed the check. A tile's scores rarely pass the running max by 62
  // (log2 units) once the first tile has set it, and p of that size loses nothing in bf16 or in the fp32 sums.
  auto softmax_fixed = [&](const f32x4 (&sc)[4][RT], u32x4 (&pbo)[2][RT], float (&ps)[RT]) -> bool {
    const float c = p.scale_log2;
    bool big = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float mu = m[rt] == -INFINITY ? 0.f : m[rt];
      float s2[8];  // pair sums, added as a tree (depth 4, not a chain of 16 dependent adds)
      uint32_t pk[8];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const float e0 = fast_exp2(fmaf(sc[kt][rt][2 * h2], c, -mu));
          const float e1 = fast_exp2(fmaf(sc[kt][rt][2 * h2 + 1], c, -mu));
          s2[kt * 2 + h2] = e0 + e1;
          pk[kt * 2 + h2] = pack_bf16x2(e0, e1);
        }
      const float sum = ((s2[0] + s2[1]) + (s2[2] + s2[3])) + ((s2[4] + s2[5]) + (s2[6] + s2[7]));
      ps[rt] = sum;
      big = big || !(sum <= 0x1p62f);  // also catches inf
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) pbo[k2][rt] = u32x4{pk[4 * k2], pk[4 * k2 + 1], pk[4 * k2 + 2], pk[4 * k2 + 3]};
    }
    return __builtin_amdgcn_ballot_w64(big) != 0;
  };
  // O^T[d][row] += V^T P^T over one tile; V^T from the LDS buffer vb with two transposed reads per 8-key column
  auto pv = [&](const u32x4 (&pbi)[2][RT], int vb) {
    auto& vs = vs2[vb];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const uint16_t* vp = &vs[k2 * 32][dt * 16] + tr_off;
        const s16x4 lo = lds_read_tr16(vp);
        const s16x4 hi = lds_read_tr16(vp + 16 * kVsStride);
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
        const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
        const u32x4 a = u32x4{l2[0], l2[1], h2[0], h2[1]};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[dt][rt] = mfma_16x16x32(a, pbi[k2][rt], acc[dt][rt]);
      }
  };

  float alpha[RT];     // the last softmax's accumulator factors
  bool moved = false;  // ... and whether any of them is not 1
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) alpha[rt] = 1.f;
  auto rescale = [&]() {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[dt][rt] *= alpha[rt];
  };
  constexpr bool kDma = KV != kPagedPieces;
  if constexpr (kDma) {
    // ---- direct-to-LDS tiles (packed keys; paged tiles inside one cache block) ----
    // K and V tiles go from global memory straight into LDS (buffer_load_dwordx4 ... lds: lane i's 16 bytes land in
    // slot i of a 1 KB run = four 256-byte rows), with no register staging, so the 32 registers a staged tile
    // occupies are free for P V operand read-ahead. Both are double-buffered in separate arrays: the compiler can
    // then tell a tile's reads from the next tile's in-flight writes and waits for those only at the barrier that
    // ends the tile (one barrier per tile). Rows are 256 bytes, unpadded; bank conflicts are avoided by permuting the
    // 16-byte chunks of a row instead: chunk c of row R sits in slot c ^ (R & 15) in K (a K-fragment read's 16 rows
    // hit 16 different slots) and in slot c ^ 2 (R & 7) in V (the 8 rows under a transposed read's 32 lanes hit 16
    // different slots). The permutation is applied on the global side: the lane that fills slot lc of row R fetches
    // chunk lc ^ f(R).
    uint8_t (*const kt0)[kTB] = bufs.k0;
    uint8_t (*const kt1)[kTB] = bufs.k1;
    uint8_t (*const vt0)[kTB] = bufs.v0;
    uint8_t (*const vt1)[kTB] = bufs.v1;
    const int lc = lane & 15;
    const int fk = lrow & 15, fv = 2 * (lrow & 7);  // rows PR i + lrow share these
    const uint32_t dk_off = (uint32_t)((lrow * rs_k + ((lc ^ fk) << 3)) * 2);
    const uint32_t dv_off = (uint32_t)((lrow * rs_v + ((lc ^ fv) << 3)) * 2);
    // new keys from rows (paged tiles, new_from_rows): positions kn0 = nk - nq and later are the step's rows, strided
    // as packed keys (the lane offsets of the same chunk permutation over the row strides)
    constexpr bool fold = KV == kPagedTilesNew || KV == kPagedTilesRows;
    const int kn0 = nk_all - nq;
    const int rsr_k = fold ? (int)p.k_row_stride : 0, rsr_v = fold ? (int)p.v_row_stride : 0;
    const uint32_t dkr_off = (uint32_t)((lrow * rsr_k + ((lc ^ fk) << 3)) * 2);
    const uint32_t dvr_off = (uint32_t)((lrow * rsr_v + ((lc ^ fv) << 3)) * 2);
    typedef __attribute__((address_space(3))) void lvoid;
    // Issues one tile's NP + NP DMA loads into (kd, vd); piece i of wave w fills rows PR i + 4 w .. + 3. In a tile
    // with missing keys each piece is a raw buffer load whose descriptor covers exactly the piece's real keys: keys
    // past nk and a whole tile of an unmapped block read as zeros (the hardware's range check), so no address is
    // clamped and no tile is patched. (The buffer form also keeps the compiler's LDS wait counting exact; the global form makes it wait
    // for every LDS read to finish.)
    bool dma_mapped = true;  // whether the most recently loaded tile's block is mapped
    // all_rows: a std::integral_constant, true for the tiles of new keys only (kPagedTilesRows' second loop): they
    // read the rows. kPagedTilesNew (the mixed kernel, whose registers leave no room for a second loop) chooses the
    // source per tile instead.
    auto dma = [&](auto all_rows, uint8_t* kd, uint8_t* vd, int kv0) {
      const char* kbc;
      const char* vbc;
      int nreal = min(kBK, nk - kv0);  // keys of this tile that exist
      int sk = rs_k, sv = rs_v;        // elements between this tile's consecutive keys
      uint32_t ko = dk_off, vo = dv_off;
      uint8_t* kdw = kd + w * 1024;
      uint8_t* vdw = vd + w * 1024;
      if constexpr (!paged) {
        kbc = reinterpret_cast<const char*>(p.k_src + (int64_t)(k0 + kv0) * p.k_row_stride + g * kD);
        vbc = reinterpret_cast<const char*>(p.v_src + (int64_t)(k0 + kv0) * p.v_row_stride + g * kD);
      } else {
        const bool okb = tile_bid >= 0 && tile_bid < p.num_blocks;
        const int64_t row0 = (int64_t)(okb ? tile_bid : 0) * p.block_size + kv0 % p.block_size;
        kbc = reinterpret_cast<const char*>(p.k_cache + row0 * rs_k + g * kD);
        vbc = reinterpret_cast<const char*>(p.v_cache + row0 * rs_k + g * kD);
        if (!okb) nreal = 0;
        dma_mapped = okb;
        if (decltype(all_rows)::value || (KV == kPagedTilesNew && kv0 >= kn0)) {  // all new: the rows, packed
          kbc = reinterpret_cast<const char*>(p.k_src + ((int64_t)q0 + kv0 - kn0) * p.k_row_stride + g * kD);
          vbc = reinterpret_cast<const char*>(p.v_src + ((int64_t)q0 + kv0 - kn0) * p.v_row_stride + g * kD);
          sk = rsr_k;
          sv = rsr_v;
          ko = dkr_off;
          vo = dvr_off;
          nreal = min(kBK, nk - kv0);
          dma_mapped = true;
        }
      }
      if (nreal == kBK) {  // every key real: one descriptor per tile, the piece offset in the scalar offset
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kbc), (short)0, kBK * sk * 2, kBufferWord3);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vbc), (short)0, kBK * sv * 2, kBufferWord3);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lvoid*)(kdw + i * PR * 256), 16, ko, PR * i * sk * 2, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lvoid*)(vdw + i * PR * 256), 16, vo, PR * i * sv * 2, 0, 0);
        }
      } else {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
          const int rows = __builtin_amdgcn_readfirstlane(min(max(nreal - PR * i, 0), PR));  // real keys in the piece
          const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kbc + (int64_t)(PR * i) * sk * 2),
                                                            (short)0, rows * sk * 2, kBufferWord3);
          const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vbc + (int64_t)(PR * i) * sv * 2),
                                                            (short)0, rows * sv * 2, kBufferWord3);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lvoid*)(kdw + i * PR * 256), 16, ko, 0, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lvoid*)(vdw + i * PR * 256), 16, vo, 0, 0, 0);
        }
      }
    };
    // Tile 0 of an item whose first new key kn0 lies inside it (kPagedTilesRows, 0 < kn0 < 64): a lane whose key is
    // old loads its 16 bytes from the cache block, the others from the rows (key kn0 = row q0; keys past nk out of the
    // rows descriptor's range, read as zeros), two loads under complementary lane masks into the same LDS slots.
    // An unmapped block reads as zeros and the tile takes no weight, as in the cache-only form.
    auto dma_straddle0 = [&](uint8_t* kd, uint8_t* vd) {
      const bool okb = bid0 >= 0 && bid0 < p.num_blocks;
      const int64_t row0 = (int64_t)(okb ? bid0 : 0) * p.block_size;
      const auto rkc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.k_cache + row0 * rs_k + g * kD),
                                                         (short)0, okb ? kn0 * rs_k * 2 : 0, kBufferWord3);
      const auto rvc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.v_cache + row0 * rs_k + g * kD),
                                                         (short)0, okb ? kn0 * rs_v * 2 : 0, kBufferWord3);
      const int nnew = min(nk, kBK) - kn0;  // the tile's new keys
      const auto rkr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(p.k_src + (int64_t)q0 * p.k_row_stride + g * kD), (short)0, nnew * rsr_k * 2,
          kBufferWord3);
      const auto rvr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(p.v_src + (int64_t)q0 * p.v_row_stride + g * kD), (short)0, nnew * rsr_v * 2,
          kBufferWord3);
      uint8_t* kdw = kd + w * 1024;
      uint8_t* vdw = vd + w * 1024;
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        if (PR * i + lrow < kn0) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rkc, (lvoid*)(kdw + i * PR * 256), 16, dk_off, PR * i * rs_k * 2, 0,
                                                   0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rvc, (lvoid*)(vdw + i * PR * 256), 16, dv_off, PR * i * rs_v * 2, 0,
                                                   0);
        } else {  // byte (key - kn0) x row stride + chunk of the rows (non-negative in these lanes)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rkr, (lvoid*)(kdw + i * PR * 256), 16,
                                                   dkr_off + (uint32_t)((PR * i - kn0) * rsr_k * 2), 0, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rvr, (lvoid*)(vdw + i * PR * 256), 16,
                                                   dvr_off + (uint32_t)((PR * i - kn0) * rsr_v * 2), 0, 0, 0);
        }
      }
      dma_mapped = okb;
    };
    // K fragment (rows kt*16 + r16, chunk kc*4 + jq) at byte kt*4096 + (krd0 ^ (kc << 6))
    const uint32_t krd0 = (uint32_t)(r16 * 256 + ((jq ^ r16) << 4));
    auto scores_d = [&](const uint8_t* kd, f32x4 (&sc)[4][RT]) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sc[kt][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 4; ++kc)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(kd + kt * 4096 + (krd0 ^ (uint32_t)(kc << 6)));
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) sc[kt][rt] = mfma_16x16x32(a, qop[rt][kc], sc[kt][rt]);
        }
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, RT, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 8 * RT, 0);
    };
    // transposed V read for (dt, k2, half h): rows k2*32 + h*16 + jq*4 + r16/4, dims dt*16 + 4 (r16 & 3) .. + 3,
    // at byte k2*8192 + h*4096 + (vrd0 ^ (dt << 5))
    const int rl = jq * 4 + (r16 >> 2);
    const uint32_t vrd0 = (uint32_t)(rl * 256 + ((rl & 7) << 5) + ((r16 & 3) << 3));
    auto pv_read = [&](const uint8_t* vd, u32x4 (&va)[8][2]) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const uint8_t* vp = vd + k2 * 8192 + (vrd0 ^ (uint32_t)(dt << 5));
          const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr16(reinterpret_cast<const uint16_t*>(vp)));
          const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr16(reinterpret_cast<const uint16_t*>(vp + 4096)));
          va[dt][k2] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
    };
    auto pv_mfma = [&](const u32x4 (&va)[8][2], const u32x4 (&pbi)[2][RT]) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[dt][rt] = mfma_16x16x32(va[dt][k2], pbi[k2][rt], acc[dt][rt]);
    };
    // one tile: the scores, then the next tile's DMA, the softmax and P V, whose transposed V reads run 16 ahead of
    // the MFMAs that consume them (left alone, the compiler waits for each operand right after reading it); the next
    // tile has landed by the barrier. (The DMA issued before the scores held them up behind its issue: config 2
    // 13.0 -> 12.8 us, paged 13.5 -> 12.9 us, 16 x 2048 276 -> 269 us; issued after the softmax it lands too late.)
    auto step = [&](auto all_rows, auto from0, int kv0, int seg_end, const uint8_t* kc_, const uint8_t* vc_,
                    uint8_t* kn, uint8_t* vn) {
      const bool has_next = kv0 + kBK < seg_end;
      const bool mapped_here = decltype(all_rows)::value || dma_mapped;  // the last tile loaded (rows: mapped)
      f32x4 sc[4][RT];
      scores_d(kc_, sc);
      if (has_next) {
        dma(all_rows, kn, vn, kv0 + kBK);
        fetch_bids(kv0 + 2 * kBK);
      }
      const bool masked = kv0 + kBK > nk || (p.causal && kv0 + kBK - 1 > first_pos);
      if (masked) mask(sc, kv0);
      if (__builtin_expect(!mapped_here, 0)) {  // a tile of an unmapped block (read as zeros) takes no weight
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) sc[kt][rt] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      }
      u32x4 pb[2][RT];
      if (decltype(from0)::value && kv0 == 0) {
        softmax(sc, pb, alpha);  // the accumulators are still zero: no rescale
        moved = false;
      } else {
        float ps[RT];
        const bool big = softmax_fixed(sc, pb, ps);
        if (__builtin_expect(big, 0)) {  // rare: a score passed the running max by more than 62: redo with its max
          moved = softmax(sc, pb, alpha);
        } else {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) l[rt] += ps[rt];
          moved = false;
        }
      }
      if (__builtin_expect(moved, 0)) rescale();
      u32x4 va[8][2];
      pv_read(vc_, va);
      pv_mfma(va, pb);
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * RT, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 8 * RT, 1);
      __syncthreads();  // the next tile has landed (the barrier waits for this wave's DMA) and this one is free
    };
    if constexpr (fold) {
      // a tile that straddles kn0 (old keys below it, new ones from it) past tile 0 is read from the cache like the
      // old tiles: first this workgroup writes that tile's new keys of its kv head there from the rows (the same bytes
      // the launch's copy writes; every workgroup reading the tile writes them before its own read). The mixed
      // kernel waits for the stores here; the plain form's first tile (an older one) is waited for with them below,
      // before the barrier after which any wave loads the straddling tile. (kPagedTilesRows patches a straddling
      // tile 0 in LDS instead.)
      const int straddle_from = KV == kPagedTilesRows ? kBK : 1;
      if (kn0 >= straddle_from && kn0 % kBK != 0 && kn0 < min(nk, kv_end)) {
        const int t1 = min((kn0 / kBK + 1) * kBK, nk);  // past the tile's last real key
        const int col = kn0 / p.block_size;             // the tile's block (block_size a multiple of 64)
        const int blk = col < 64 ? __builtin_amdgcn_readlane(bt_row, col)
                                 : p.block_tables[(int64_t)b * p.bt_stride + col];
        if (blk >= 0 && blk < p.num_blocks) {
          // (key, K or V, 16-byte chunk): at most 63 x 32 = 8 NT, kU loads in flight before their stores (one in
          // the mixed kernel, whose registers are spoken for)
          constexpr int kU = KV == kPagedTilesRows ? 4 : 1;
          const int nchunk = (t1 - kn0) * 32;
          for (int c0 = 0; c0 < nchunk; c0 += kU * NT) {
            u32x4 d[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
              const int c = min(c0 + u * NT + tid, nchunk - 1);
              const int key = kn0 + (c >> 5), which = (c >> 4) & 1, ch = c & 15;
              const int64_t row = (int64_t)q0 + (key - kn0);
              d[u] = ld_g16((which ? p.v_src + row * p.v_row_stride : p.k_src + row * p.k_row_stride) + g * kD +
                            ch * 8);
            }
#pragma unroll
            for (int u = 0; u < kU; ++u) {
              const int c = c0 + u * NT + tid;
              if (c < nchunk) {
                const int key = kn0 + (c >> 5), which = (c >> 4) & 1, ch = c & 15;
                const int64_t slot = (int64_t)blk * p.block_size + key % p.block_size;
                uint16_t* dst = const_cast<uint16_t*>(which ? p.v_cache : p.k_cache) + (slot * HK + g) * kD;
                *reinterpret_cast<u32x4*>(dst + ch * 8) = d[u];
              }
            }
          }
        }
        if constexpr (KV == kPagedTilesNew) {
          wait_vmem_all();
          __syncthreads();
        }
      }
    }
    // the key tiles [kv_begin, kv_stop): the first one's DMA and its wait (unless `pre`: already loaded, into the
    // second buffers), then two steps per iteration over the double buffers (a segment's last step issues no DMA).
    // from0, pre: std::integral_constants. from0: the segment starts at key 0, whose tile takes the plain softmax;
    // the steps of a segment that starts later know that none of theirs is the first tile.
    auto tiles = [&](auto all_rows, auto from0, auto pre, int kv_begin, int kv_stop) {
      uint8_t* const ka = decltype(pre)::value ? kt1[half] : kt0[half];
      uint8_t* const va = decltype(pre)::value ? vt1[half] : vt0[half];
      uint8_t* const kb = decltype(pre)::value ? kt0[half] : kt1[half];
      uint8_t* const vb = decltype(pre)::value ? vt0[half] : vt1[half];
      if constexpr (decltype(from0)::value) kv_begin = 0;
      if (kv_stop <= kv_begin) return;
      if constexpr (!decltype(pre)::value) {
        if constexpr (decltype(from0)::value)
          tile_bid = bid0;
        else
          fetch_bids(kv_begin);
        dma(all_rows, ka, va, kv_begin);
        wait_vmem_all();  // the query, the segment's first tile and the table row (and a straddling tile's copy)
        fetch_bids(kv_begin + kBK);
        __syncthreads();
      }
      for (int kv0 = kv_begin; kv0 < kv_stop; kv0 += 2 * kBK) {
        step(all_rows, from0, kv0, kv_stop, ka, va, kb, vb);
        if (kv0 + kBK < kv_stop) step(all_rows, from0, kv0 + kBK, kv_stop, kb, vb, ka, va);
      }
    };
    using T = std::true_type;
    using F = std::false_type;
    if constexpr (KV == kPagedTilesRows) {
      // the tiles holding an old key come from the cache, the rest from the rows, in loops of one source each (a
      // per-tile choice of source inside one loop measured slower: config 2 paged 13.1 -> 17.3 us)
      if (kn0 <= 0) {
        tiles(T{}, T{}, F{}, 0, kv_end);
      } else if (kn0 < kBK) {
        // tile 0 straddles kn0: each lane's 16 bytes of it from the cache (an old key) or from the rows (a new one),
        // and tile 1 (all new) from the rows into the second buffers, all in one round trip
        if (kv_end > kBK) dma(T{}, kt1[half], vt1[half], kBK);
        dma_straddle0(kt0[half], vt0[half]);
        wait_vmem_all();
        __syncthreads();
        step(F{}, T{}, 0, kBK, kt0[half], vt0[half], kt1[half], vt1[half]);  // no DMA: tile 1 is loaded
        tiles(T{}, F{}, T{}, kBK, kv_end);
      } else {
        const int c_end = min(kv_end, (kn0 + kBK - 1) / kBK * kBK);
        tiles(F{}, T{}, F{}, 0, c_end);
        tiles(T{}, F{}, F{}, c_end, kv_end);
      }
    } else {
      tiles(F{}, T{}, F{}, 0, kv_end);
    }
  } else {
    if (kv_end > 0) {
      fetch_bids(0);
      load_tile(0);
      fetch_bids(kBK);
    }
    // The query and the first tile arrive in one round trip; waiting here (rather than at the first use) also lets
    // the compiler's wait analysis see the query registers complete at the loop head, so no wait inside the loop
    // covers the prefetched tile.
    wait_vmem_all();
    int vb = 0;       // LDS buffer of this tile's V
    for (int kv0 = 0; kv0 < kv_end; kv0 += kBK) {
      stage_tile(vb);
      __syncthreads();
      if (kv0 + kBK < kv_end) {  // in flight while this tile computes
        load_tile(kv0 + kBK);
        fetch_bids(kv0 + 2 * kBK);
      }
      f32x4 sc[4][RT];
      scores(sc);
      const bool masked = kv0 + kBK > nk || (p.causal && kv0 + kBK - 1 > first_pos);
      if (masked) mask(sc, kv0);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {  // keys kt*16 + jq*4 + [0, 4) of an unmapped block take no weight
        const uint32_t ok4 = *reinterpret_cast<const uint32_t*>(&s_keyok[half][kt * 16 + jq * 4]);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) sc[kt][rt][rr] = ((ok4 >> (8 * rr)) & 1u) ? sc[kt][rt][rr] : -INFINITY;
      }
      u32x4 pb[2][RT];
      if (softmax(sc, pb, alpha)) rescale();
      pv(pb, vb);
      vb ^= 1;
      __syncthreads();  // K and the previous V buffer are free for the next tile's staging
    }
  }

  if constexpr (QUANT) {
    // ---- int8 epilogue: o * inv_smooth, per-token amax over all heads, rint(o / scale) ----
    const int g_rows = G;
    float lmax[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      lmax[rt] = 0.f;
      const float L = col_sum4(l[rt]);
      const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        f32x4 o = acc[dt][rt] * inv;
        if (p.inv_smooth) o *= *reinterpret_cast<const f32x4*>(p.inv_smooth + h_of[rt] * kD + dt * 16 + jq * 4);
        acc[dt][rt] = o;
        lmax[rt] = fmaxf(lmax[rt], fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
      }
    }
    __syncthreads();  // s_amax cleared (also when no key tile ran)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      if (row_ok[rt]) atomicMax(&s_amax[((w * RT + rt) * 16 + r16) / g_rows], __float_as_uint(lmax[rt]));
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if (!row_ok[rt]) continue;
      const float scale = fmaxf(__uint_as_float(s_amax[((w * RT + rt) * 16 + r16) / g_rows]), 1e-6f) / 127.f;
      // rint(o / scale) without a division per element: x = o * (1 / scale) is within 2.5e-5 of the exact
      // quotient (|o / scale| <= 127.5, two roundings), so rint(x) is rint(o / scale) unless x lies within 1e-4 of
      // a half-integer; those rare elements take the division. Same codes as dividing every element.
      const float rs = 1.f / scale;
      int8_t* op = p.out_q + (int64_t)(q0 + tq_of[rt]) * p.out_row_stride + (int64_t)h_of[rt] * kD + jq * 4;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const f32x4 o = acc[dt][rt];
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = o[e] * rs;
          float r = __builtin_rintf(x);
          if (__builtin_expect(fabsf(fabsf(x - r) - 0.5f) < 1e-4f, 0)) r = __builtin_rintf(o[e] / scale);
          packed |= (uint32_t)(uint8_t)(int8_t)(int)r << (8 * e);
        }
        *reinterpret_cast<uint32_t*>(op + dt * 16) = packed;
      }
    }
    if (threadIdx.x < (unsigned)BQ && qt * BQ + (int)threadIdx.x < nq &&
        (p.row_limit <= 0 || (int64_t)q0 + qt * BQ + (int)threadIdx.x < p.row_limit))
      p.out_scale[q0 + qt * BQ + threadIdx.x] = fmaxf(__uint_as_float(s_amax[threadIdx.x]), 1e-6f) / 127.f;
    return;
  }

  // ---- epilogue: normalize, bf16, 4 consecutive dims per lane per d-tile ----
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float L = col_sum4(l[rt]);
    if (!row_ok[rt]) continue;
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint16_t* op = p.out + (int64_t)(q0 + tq_of[rt]) * p.out_row_stride + (int64_t)h_of[rt] * kD + jq * 4;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4 v = acc[dt][rt];
      *reinterpret_cast<u32x2*>(op + dt * 16) =
          u32x2{pack_bf16x2(v[0] * inv, v[1] * inv), pack_bf16x2(v[2] * inv, v[3] * inv)};
    }
  }
}

// Grid forms. Plain grid (kFormGrid): one workgroup per (q tile, sequence, kv head) of the grid. Workgroup i runs on XCD
// i % 8; with xcd_order each XCD gets a contiguous run of work items, so the query tiles that re-read a sequence's
// K/V tiles find them in that XCD's L2 (the launcher sets it for large grids; on small ones the runs would hold
// uneven numbers of empty tiles). A causal run starts at each sequence's last query tile, the one with the most key
// tiles, so the light tiles fill the end of the run instead of the heavy ones (16 x 2048 tokens -3 %, 2 x 8192 -5 %).
// Persistent (kFormPersistent): a fixed grid, for calls whose (q tile, sequence) grid would be mostly empty (a mixed
// step's decode rows, left to the decode kernel): each workgroup reads cu_q once, numbers the items of the sequences
// that have work and walks its share of them (order below). An empty workgroup of the plain grid costs a memory round
// trip to find it has nothing to do; a grid of a few thousand of them took longer than the work itself.
// Rank-major (kFormRanked): a causal grid of more work items than fit on the CUs at once, one 1-D grid in rank order:
// rank r = the r-th heaviest q tile of every (sequence, kv head), so the longest chains of key tiles start first
// and the light tiles fill in behind them (with the plain grid, the second kv head's heavy tiles waited for a free
// slot: config 2, 832 items on 512 slots, 16.5 -> 13.4 us). Within a rank the (sequence, kv head) pairs rotate by
// r, so a pair's tiles are dealt over all eight XCDs rather than all landing on one. A form of its own: the extra
// index arithmetic in the plain grid's kernel cost the short non-causal steps 4-7 %.
constexpr int kRankCap = 1024;  // longest sequence, in q tiles, that the persistent rank order covers

// LDS of the persistent walk, for up to `cap` sequences (p.batch <= cap)
struct ItemLds {
  int* nt;      // [cap] q tiles of each sequence (0: nothing for this kernel)
  int* act;     // [cap] the sequences with q tiles, in order
  int* sorted;  // [cap] ... most tiles first (stable)
  int* snt;     // [cap] their tile counts
  int* P;       // [kRankCap + 1] items of the ranks before r
  int* red;     // [2 x waves]
  int* first;   // [cap + 1] first item of each sequence (sequence-by-sequence order)
};
constexpr int item_lds_ints(int cap, int waves) { return 5 * cap + 1 + kRankCap + 1 + 2 * waves; }
__device__ __forceinline__ ItemLds item_lds(int* base, int cap, int waves) {
  return ItemLds{base, base + cap, base + 2 * cap, base + 3 * cap, base + 4 * cap, base + 4 * cap + kRankCap + 1,
                 base + 4 * cap + kRankCap + 1 + 2 * waves};
}

// The persistent walk of workgroup g of G (kFormPersistent, and the prefill workgroups of a mixed launch): reads
// cu_q once, numbers the items of the sequences that have work and walks its share of them (order below).
template <bool QUANT, int KV, int NW, int RT>
__device__ __forceinline__ void prefill_items(const PrefillArgs& p, const int g, const int G,
                                              const DmaBufs<QUANT ? 2 : 1>& bufs, const ItemLds& A) {
  {
    constexpr int NTH = 64 * NW * (QUANT ? 2 : 1);
    constexpr int ROWS = 16 * RT * NW;
    int* const s_nt = A.nt;
    int* const s_act = A.act;
    int* const s_sorted = A.sorted;
    int* const s_snt = A.snt;
    int* const s_P = A.P;
    int* const s_red = A.red;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int BQ = ROWS / p.group;
    const int HKz = QUANT ? 1 : p.num_kv_heads;
    // q tiles per sequence; the sequences that have any, compacted in order (a block-wide scan); the most tiles
    int maxnt = 0, nact = 0, run = 0;
    for (int base = 0; base < p.batch; base += NTH) {
      const int bb = base + tid;
      int nt = 0;
      if (bb < p.batch) {
        const int nq = max(p.cu_q[bb + 1] - p.cu_q[bb], 0);
        nt = (p.skip_single && nq == 1) ? 0 : (nq + BQ - 1) / BQ;
        s_nt[bb] = nt;
      }
      const int incl = wave_incl_scan(nt > 0 ? 1 : 0, lane);
      int wmax = nt;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) wmax = max(wmax, __shfl_xor(wmax, o, kWave));
      if (lane == kWave - 1) {
        s_red[w] = incl;
        s_red[NTH / 64 + w] = wmax;
      }
      __syncthreads();
      int before = 0, total = 0;
#pragma unroll
      for (int ww = 0; ww < NTH / 64; ++ww) {
        before += ww < w ? s_red[ww] : 0;
        total += s_red[ww];
        maxnt = max(maxnt, s_red[NTH / 64 + ww]);
      }
      if (nt > 0) s_act[run + before + incl - 1] = bb;
      run += total;
      __syncthreads();
    }
    nact = __builtin_amdgcn_readfirstlane(run);
    maxnt = __builtin_amdgcn_readfirstlane(maxnt);
    // Items in rank order: rank r holds the r-th heaviest q tile (causal: the r-th from the end) of every sequence
    // that has more than r tiles, sequences with the most tiles first, both kv heads of a tile together. With the
    // sequences sorted by tile count, rank r is the first c(r) = #{nt > r} of them, and P(r) = HKz sum min(nt, r)
    // items come before it. Walking this order in a snake over the workgroups (g, 2G - 1 - g, 2G + g, ...) hands the
    // heaviest tiles out first and pairs heavy with light ones: for a mixed step's 6 prefills of 300-600 tokens the
    // most a workgroup walks drops from 14 key tiles (sequence by sequence) to 9, the heaviest single item.
    // Longer sequences than kRankCap tiles keep the sequence-by-sequence order.
    const bool ranked = maxnt <= kRankCap;
    if (ranked) {
      for (int a = tid; a < nact; a += NTH) {  // stable rank of each active sequence by tile count
        const int bb = s_act[a];
        const int nt = s_nt[bb];
        int pos = 0;
#pragma unroll 8
        for (int a2 = 0; a2 < nact; ++a2) {
          const int n2 = s_nt[s_act[a2]];
          pos += n2 > nt || (n2 == nt && a2 < a);
        }
        s_sorted[pos] = bb;
        s_snt[pos] = nt;
      }
      __syncthreads();
      for (int r = tid; r <= maxnt; r += NTH) {
        int sum = 0;
#pragma unroll 8
        for (int j = 0; j < nact; ++j) sum += min(s_snt[j], r);
        s_P[r] = sum * HKz;
      }
      __syncthreads();
      const int W = __builtin_amdgcn_readfirstlane(s_P[maxnt]);
      for (int t = 0; t * G < W; ++t) {
        const int k = t * G + ((t & 1) ? G - 1 - g : g);
        if (k >= W) continue;
        int lo = 0, hi = maxnt;  // the rank r with s_P[r] <= k < s_P[r + 1]
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (__builtin_amdgcn_readfirstlane(s_P[mid]) <= k) lo = mid; else hi = mid;
        }
        const int local = k - __builtin_amdgcn_readfirstlane(s_P[lo]);
        const int bq = __builtin_amdgcn_readfirstlane(s_sorted[local / HKz]);
        const int nt = __builtin_amdgcn_readfirstlane(s_nt[bq]);
        prefill_tile<QUANT, KV, NW, RT>(p, p.causal ? nt - 1 - lo : lo, bq, local % HKz, bufs);
        __syncthreads();  // the item's LDS is free for the next one
      }
      return;
    }
    // sequence-by-sequence order (heaviest causal q tile first within a sequence), every G-th item
    int* const s_first = A.first;  // first item of each sequence; s_first[batch] = the total
    run = 0;
    for (int base = 0; base < p.batch; base += NTH) {
      const int bb = base + tid;
      const int n = bb < p.batch ? s_nt[bb] * HKz : 0;
      const int incl = wave_incl_scan(n, lane);
      if (lane == kWave - 1) s_red[w] = incl;
      __syncthreads();
      int before = 0, total = 0;
#pragma unroll
      for (int ww = 0; ww < NTH / 64; ++ww) {
        before += ww < w ? s_red[ww] : 0;
        total += s_red[ww];
      }
      if (bb < p.batch) s_first[bb] = run + before + incl - n;
      run += total;
      __syncthreads();
    }
    if (tid == 0) s_first[p.batch] = run;
    __syncthreads();
    for (int i = g; i < run; i += G) {
      int lo = 0, hi = p.batch;  // the last b with s_first[b] <= i (an empty sequence shares the next one's start)
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (__builtin_amdgcn_readfirstlane(s_first[mid]) <= i) lo = mid; else hi = mid;
      }
      const int first = __builtin_amdgcn_readfirstlane(s_first[lo]);
      const int nt = (__builtin_amdgcn_readfirstlane(s_first[lo + 1]) - first) / HKz;
      const int local = i - first;
      const int r = local / HKz;
      prefill_tile<QUANT, KV, NW, RT>(p, p.causal ? nt - 1 - r : r, lo, local % HKz, bufs);
      __syncthreads();  // the item's LDS is free for the next one
    }
  }
}

// The KV store riding in a packed launch (PrefillArgs::store_rows; what store_kvcache_kernel does): workgroup wid of
// the store_wgs copying ones copies rows wid, wid + store_wgs, ..., 16 bytes per lane, every load of a batch issued
// before its stores. Nothing in a packed launch reads the cache, so the copy may run anywhere in it. It runs after
// the workgroup's item (before it, the item's first wait also waited for the copy's stores: config 2 step 13.3 ->
// 14.3 us), in workgroups [256, 512) of the launch order: at config 2 the rank-major grid's medium items, resident
// from the start and done well before the heaviest chains (the grid's last 256, dispatched last, 13.9 us; here
// 13.3 us, the time of the launch without the store). Non-temporal stores, as nothing in the step reads them back.
__device__ __forceinline__ void store_rows(const PrefillArgs& p, int wid) {
  const int row = p.num_kv_heads * kD;  // elements of one K (or V) row
  const int pieces = row / 8;           // 16-byte pieces per row
  const int per_row = 2 * pieces;
  const int64_t rows = (p.store_rows - wid + p.store_wgs - 1) / p.store_wgs;
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
      const int64_t tok = wid + r_local * p.store_wgs;
      const uint16_t* src = (which ? p.v_src + tok * p.v_row_stride : p.k_src + tok * p.k_row_stride) + piece * 8;
      val[u] = in ? ld_g16(src) : zero4();
      slot[u] = in ? (int64_t)p.store_slots[tok] : -1;
      dst[u] = (which ? p.store_v_cache : p.store_k_cache) + piece * 8;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (slot[u] >= 0 && slot[u] < p.store_num_slots)
        __builtin_nontemporal_store(val[u], reinterpret_cast<u32x4*>(dst[u] + slot[u] * row));
  }
}

// Waves per SIMD the registers must allow: two 4-wave workgroups per CU (their 64 KB of LDS each fits twice), two
// 8-wave ones (at most 128 VGPRs: the riding store's paged form would take 132 and hold one workgroup per CU, which
// ran the 44 x 46-token step's 264 workgroups in two rounds, 15.4 -> 17.6 us), one int8 workgroup (128 KB of LDS).
constexpr int prefill_waves_per_simd(bool quant, int nw) { return quant ? 1 : (nw == 8 ? 4 : 2); }

template <bool QUANT, int KV, int NW, int RT, int FORM>
__global__ __launch_bounds__(64 * NW * (QUANT ? 2 : 1), prefill_waves_per_simd(QUANT, NW)) void prefill_kernel(
    PrefillArgs p) {
  constexpr int NH = QUANT ? 2 : 1;
  __shared__ __attribute__((aligned(1024))) uint8_t kt0[NH][kTB];
  __shared__ __attribute__((aligned(1024))) uint8_t kt1[NH][kTB];
  __shared__ __attribute__((aligned(1024))) uint8_t vt0[NH][kTB];
  __shared__ __attribute__((aligned(1024))) uint8_t vt1[NH][kTB];
  const DmaBufs<NH> bufs{kt0, kt1, vt0, vt1};
  if constexpr (FORM == kFormRanked) {
    const int nz = QUANT ? 1 : p.num_kv_heads;  // (QUANT: a workgroup holds every kv head)
    const int n = p.batch * nz, id = blockIdx.x, r = id / n, c = (id + r) % n;
    const int qt = p.causal ? (int)gridDim.x / n - 1 - r : r;
    prefill_tile<QUANT, KV, NW, RT>(p, qt, c / nz, c % nz, bufs);
    if constexpr (KV == kPacked || KV == kPagedTilesRows)
      if (p.store_rows > 0 && id >= p.store_first && id < p.store_first + p.store_wgs) store_rows(p, id - p.store_first);
  } else if constexpr (FORM == kFormPersistent) {
    constexpr int NWV = NW * (QUANT ? 2 : 1);
    __shared__ int s_items[item_lds_ints(kMaxSeqPerLaunch, NWV)];
    prefill_items<QUANT, KV, NW, RT>(p, (int)blockIdx.x, (int)gridDim.x, bufs,
                                     item_lds(s_items, kMaxSeqPerLaunch, NWV));
  } else {
    int qt = blockIdx.x, b = blockIdx.y, gz = blockIdx.z;
    if (p.xcd_order) {
      const unsigned nwg = gridDim.x * gridDim.y * gridDim.z;
      const unsigned id = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
      const unsigned xq = nwg / kXcds, xr = nwg % kXcds, xcd = id % kXcds, loc = id / kXcds;
      const unsigned work = (xcd < xr ? xcd * (xq + 1) : xr * (xq + 1) + (xcd - xr) * xq) + loc;
      qt = (int)(work % gridDim.x);
      b = (int)((work / gridDim.x) % gridDim.y);
      gz = (int)(work / (gridDim.x * gridDim.y));
      if (p.causal) qt = (int)gridDim.x - 1 - qt;  // heavy query tiles first
    }
    prefill_tile<QUANT, KV, NW, RT>(p, qt, b, gz, bufs);
    if constexpr (KV == kPacked || KV == kPagedTilesRows) {
      if (p.store_rows > 0) {
        const int id = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
        if (id >= p.store_first && id < p.store_first + p.store_wgs) store_rows(p, id - p.store_first);
      }
    }
  }
}

// Mixed prefill + decode step in one launch (a paged varlen call whose one-query rows go to the split-KV decode
// work): workgroups [0, nd) run decode_split over the one-query rows (da, nd = da.grid workgroups), the others walk
// the prefill items of the other rows (pa, persistent order, 128-row items). Both roles fit two workgroups per CU
// (the decode role's state borrows the prefill role's tile buffers: rounds of 3 segments, bf16 slots), so a CU holds
// one of each and the prefill rows' MFMA and LDS work runs beside the decode rows' memory stream instead of after it
// (the dispatcher places workgroups [0, nd) one per CU, then the rest in the second slots: read back from HW_ID in a
// working probe). One 4-wave workgroup shape, paged tiles (block_size a multiple of 64), at most 256 sequences.
template <int HK, bool NEW>
__global__ __launch_bounds__(256, 2) void mixed_kernel(PrefillArgs pa, DecodeArgs da) {
  using LB = dec::LdsBorrowed<HK>;
  static_assert(LB::kBufBytes == kTB, "the decode role borrows the prefill tile buffers");
  constexpr int kItemInts = item_lds_ints(LB::kSeqCap, 4);
  constexpr int kAux = LB::kAuxBytes > kItemInts * 4 ? LB::kAuxBytes : kItemInts * 4;
  __shared__ __attribute__((aligned(1024))) uint8_t kt0[1][kTB];
  __shared__ __attribute__((aligned(1024))) uint8_t kt1[1][kTB];
  __shared__ __attribute__((aligned(1024))) uint8_t vt0[1][kTB];
  __shared__ __attribute__((aligned(1024))) uint8_t vt1[1][kTB];
  __shared__ __attribute__((aligned(16))) uint8_t aux[kAux];
  const int nd = da.grid;
  if ((int)blockIdx.x < nd) {
    const LB L(kt0[0], kt1[0], vt0[0], vt1[0], aux);
    dec::decode_split<HK>(da, (int)blockIdx.x, nd, L);
    return;
  }
  // The prefill rows are the longer pole (alone on the CUs they would take 2x the time they take at two workgroups
  // per CU), the decode rows a memory stream that tolerates waiting: the prefill waves issue first (config 5, the
  // attention call: 53.6 -> 49.6 us), and take 128-row items (4 waves x 32 rows), which halve the key-tile steps of
  // the 64-row items for the same LDS (49.6 -> 44.0 us).
  __builtin_amdgcn_s_setprio(1);
  const DmaBufs<1> bufs{kt0, kt1, vt0, vt1};
  prefill_items<false, NEW ? kPagedTilesNew : kPagedTiles, 4, 2>(
      pa, (int)blockIdx.x - nd, (int)gridDim.x - nd, bufs, item_lds(reinterpret_cast<int*>(aux), LB::kSeqCap, 4));
}

}  // namespace

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;  // MI355X
  }
  return cus;
}

template <bool QUANT, int NW, int RT, int FORM = kFormGrid>
hipError_t launch_prefill_kind(const PrefillArgs& a, dim3 grid, hipStream_t stream) {
  const dim3 block(64 * NW * (QUANT ? a.num_kv_heads : 1));
  if (!a.block_tables)
    prefill_kernel<QUANT, kPacked, NW, RT, FORM><<<grid, block, 0, stream>>>(a);
  else if (a.block_size % kBK == 0 && a.new_from_rows) {
    if constexpr (FORM != kFormPersistent)  // (the plain and rank-major forms take a riding store)
      prefill_kernel<QUANT, kPagedTilesRows, NW, RT, FORM><<<grid, block, 0, stream>>>(a);
    else
      return hipErrorInvalidValue;
  } else if (a.block_size % kBK == 0)
    prefill_kernel<QUANT, kPagedTiles, NW, RT, FORM><<<grid, block, 0, stream>>>(a);
  else
    prefill_kernel<QUANT, kPagedPieces, NW, RT, FORM><<<grid, block, 0, stream>>>(a);
  return hipGetLastError();
}

bool mixed_launch_fits(const PrefillArgs& a, int num_kv_heads) {
  return a.cu_q && a.block_tables && a.block_size % kBK == 0 && a.group > 0 && kRows % a.group == 0 &&
         a.batch >= 1 && a.batch <= dec::LdsBorrowed<2>::kSeqCap && (num_kv_heads == 1 || num_kv_heads == 2);
}

hipError_t launch_mixed(const PrefillArgs& a, int max_seqlen_q, const DecodeArgs& d, int num_kv_heads,
                        hipStream_t stream) {
  if (!mixed_launch_fits(a, num_kv_heads) || d.batch != a.batch || d.grid < 1 || max_seqlen_q <= 0)
    return hipErrorInvalidValue;
  // a riding store: the prefill role's new keys from the rows, the decode role's by slot, the copy in the merge kernel
  if (a.new_from_rows && (!a.k_src || !a.v_src || !d.slot_mapping || !d.new_k || !d.new_v || !d.cu_q ||
                          d.copy_rows <= 0 || d.copy_wgs < 1))
    return hipErrorInvalidValue;
  // the prefill workgroups: at most one per 128-row item, and one per CU (the other slot of each CU holds a decode
  // workgroup; a third of them more, waiting for free slots, measured slower: 49.6 -> 57.2 us)
  const int64_t bq = kRows / a.group;
  const int64_t items = ((int64_t)max_seqlen_q + bq - 1) / bq * a.batch * a.num_kv_heads;
  const int64_t np = items < device_cus() ? items : device_cus();
  const dim3 grid((unsigned)(d.grid + np)), block(256);
  if (num_kv_heads == 1 && a.new_from_rows)
    mixed_kernel<1, true><<<grid, block, 0, stream>>>(a, d);
  else if (num_kv_heads == 1)
    mixed_kernel<1, false><<<grid, block, 0, stream>>>(a, d);
  else if (a.new_from_rows)
    mixed_kernel<2, true><<<grid, block, 0, stream>>>(a, d);
  else
    mixed_kernel<2, false><<<grid, block, 0, stream>>>(a, d);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_decode_merge(d, stream);
}

hipError_t launch_prefill(const PrefillArgs& a0, int max_seqlen_q, hipStream_t stream) {
  // a riding store: packed keys, or paged tiles with the new keys from the rows (new_from_rows)
  if (a0.new_from_rows && (!a0.block_tables || a0.block_size % kBK || a0.persistent || !a0.k_src || !a0.v_src ||
                           a0.store_rows <= 0))
    return hipErrorInvalidValue;
  if (a0.store_rows > 0 && ((a0.block_tables && !a0.new_from_rows) || a0.persistent || !a0.store_slots))
    return hipErrorInvalidValue;
  if (max_seqlen_q <= 0 || a0.batch <= 0) return hipSuccess;
  PrefillArgs a = a0;
  if (a.persistent) {
    // 4 waves of 16 rows (64 / G tokens per item; the shorter key-tile chain per item), two workgroups per CU, at
    // most one workgroup per item; sequences in slices of kMaxSeqPerLaunch (rows stay absolute through cu_q)
    if (!a.cu_q || 64 % a.group) return hipErrorInvalidValue;
    const int64_t bq = 64 / a.group;
    for (int b0 = 0; b0 < a0.batch; b0 += kMaxSeqPerLaunch) {
      PrefillArgs s = a;
      s.batch = a0.batch - b0 < kMaxSeqPerLaunch ? a0.batch - b0 : kMaxSeqPerLaunch;
      s.cu_q = a.cu_q + b0;
      s.cu_k = a.cu_k + b0;
      if (s.block_tables) s.block_tables = a.block_tables + (int64_t)b0 * a.bt_stride;
      const int64_t items = ((int64_t)max_seqlen_q + bq - 1) / bq * s.batch * s.num_kv_heads;
      const int64_t grid = items < 2 * device_cus() ? items : 2 * device_cus();
      const hipError_t e = launch_prefill_kind<false, 4, 1, kFormPersistent>(s, dim3((unsigned)grid), stream);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  // 4 waves of 16 rows (64 / G tokens per workgroup) when that grid fits two workgroups per CU at once: rows that
  // hold no query token still run every key tile, and a 128-row workgroup over a few tokens is mostly such rows
  // (measured: head-start step 200 x 7 tokens 7.4 -> 6.8 us, LocEnc 150 x 5 6.1 -> 5.5 us). Up to four per CU when
  // the longest sequence spans 16+ such tiles: halving a workgroup's rows halves the work of its chain of key tiles
  // (config 2: 16.9 -> 16.2 us), while on short sequences the doubled tile loads cost more than that saves (44 x 46
  // tokens paged 12.8 -> 14.0 us, LocDiT 150 x 11 8.4 -> 10.0 us with the wider rule). A causal grid beyond two per
  // CU runs rank-major (heaviest q tiles first).
  // a riding KV store (packed keys, or paged tiles with the new keys from the rows) is copied by min(grid, 256)
  // workgroups: [256, 512) in launch order, or the last ones of a smaller grid
  auto store_by = [&](int64_t nwg) {
    a.store_wgs = a.store_rows > 0 ? (int)(nwg < 256 ? nwg : 256) : 0;
    a.store_first = (int)(nwg - a.store_wgs < 256 ? nwg - a.store_wgs : 256);
  };
  const bool fits64 = 64 % a.group == 0;  // group sizes above 64 take the 128-row form only
  const int64_t tiles64 = fits64 ? (max_seqlen_q + 64 / a.group - 1) / (64 / a.group) : 0;
  const int64_t grid64 = tiles64 * a.batch * a.num_kv_heads, cus = device_cus();
  if (fits64 && (grid64 <= 2 * cus || (grid64 <= 4 * cus && tiles64 >= 16))) {
    a.xcd_order = 0;
    store_by(grid64);
    if (a.causal && grid64 > 2 * cus && grid64 <= INT32_MAX)
      return launch_prefill_kind<false, 4, 1, kFormRanked>(a, dim3((unsigned)grid64), stream);
    return launch_prefill_kind<false, 4, 1>(a, dim3((unsigned)tiles64, (unsigned)a.batch, (unsigned)a.num_kv_heads),
                                            stream);
  }
  const int bq = kRows / a.group;
  const int q_tiles = (max_seqlen_q + bq - 1) / bq;
  const int64_t nwg = (int64_t)q_tiles * a.batch * a.num_kv_heads;
  a.xcd_order = nwg >= kXcdOrderMinWorkgroups;
  store_by(nwg);
  const dim3 grid((unsigned)q_tiles, (unsigned)a.batch, (unsigned)a.num_kv_heads);
  if (nwg <= kSmallGridWorkgroups) return launch_prefill_kind<false, 8, 1>(a, grid, stream);
  return launch_prefill_kind<false, 4, 2>(a, grid, stream);
}

// The fused int8 epilogue needs every KV group of a token in one workgroup: two 4-wave halves that share every
// barrier, 128 KB of LDS, one workgroup per CU, so a CU runs one chain of key tiles where the bf16 kernel runs two
// workgroups' chains side by side. Where the 16-row halves outnumber the CUs and the sequences span 16+ such
// tiles (the rank-major int8 grids: long chains, more than one round of workgroups), the bf16 kernel followed by a
// quantization pass over its rows is faster; short steps keep the fused epilogue (the second launch would cost more
// than it saves).
bool prefill_int8_two_pass(int batch, int max_seqlen_q, int num_heads, int num_kv_heads, int causal) {
  if (batch <= 0 || max_seqlen_q <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return false;
  const int group = num_heads / num_kv_heads;
  if (64 % group) return false;
  const int64_t tiles16 = (max_seqlen_q + 64 / group - 1) / (64 / group);
  return causal && tiles16 >= 16 && tiles16 * batch > device_cus();
}

hipError_t launch_prefill_int8(const PrefillArgs& a0, int max_seqlen_q, hipStream_t stream) {
  if (max_seqlen_q <= 0 || a0.batch <= 0) return hipSuccess;
  if (a0.num_kv_heads < 1 || a0.num_kv_heads > 2) return hipErrorInvalidValue;
  // Each KV-group half: 4 waves of 16 rows (64 / G tokens per workgroup) when that grid still fits one workgroup per
  // CU (this instance's LDS allows one), or two rounds of them when the longest sequence spans 16+ such tiles (its
  // key-tile chains are long enough to gain from half the rows), else 4 waves of 32 rows. Measured: 150 streams x 5
  // tokens 8.9 -> 6.7 us, config 2 24.6 -> 24.0 us; where the smaller tiles need a second round of workgroups over
  // short sequences (150 x 11 tokens, 44 x 46) they cost 27-40 %.
  const bool fits64 = 64 % a0.group == 0;  // group sizes above 64 take the 32-row form only
  const int64_t tiles16 = fits64 ? (max_seqlen_q + 64 / a0.group - 1) / (64 / a0.group) : 0;
  const int64_t grid16 = tiles16 * a0.batch, cus = device_cus();
  const bool r16 = fits64 && (grid16 <= cus || (grid16 <= 2 * cus && tiles16 >= 16));
  const int bq = (r16 ? 64 : 128) / a0.group;
  const int q_tiles = (max_seqlen_q + bq - 1) / bq;
  PrefillArgs a = a0;
  a.xcd_order = (int64_t)q_tiles * a.batch >= kXcdOrderMinWorkgroups;
  const dim3 grid((unsigned)q_tiles, (unsigned)a.batch, 1u);
  // a riding KV store (packed keys, or paged tiles with the new keys from the rows) is copied by the launch's last
  // min(grid, 256) workgroups after their items
  if (a.new_from_rows && (!a.block_tables || a.block_size % kBK || !a.k_src || !a.v_src || a.store_rows <= 0))
    return hipErrorInvalidValue;
  if (a.store_rows > 0) {
    if ((a.block_tables && !a.new_from_rows) || !a.store_slots) return hipErrorInvalidValue;
    const int64_t nwg = (int64_t)q_tiles * a.batch;
    a.store_wgs = (int)(nwg < 256 ? nwg : 256);
    a.store_first = (int)(nwg - a.store_wgs);
  }
  if (r16 && a.causal && grid16 > cus)  // more items than CUs: rank-major, heaviest first
    return launch_prefill_kind<true, 4, 1, kFormRanked>(a, dim3((unsigned)grid16), stream);
  if (r16) return launch_prefill_kind<true, 4, 1>(a, grid, stream);
  return launch_prefill_kind<true, 4, 2>(a, grid, stream);
}

}  // namespace vox
