// Kernel 3: paged decode attention (one query token per sequence) over a block-table KV cache.
//
// Semantics (reference call: nanovllm_voxcpm/model/layers.py:350-358, flash_attn_with_kvcache with cache_seqlens and
// block_table, causal, softmax_scale): for every sequence b and query head h,
//   o[b, h] = softmax_j(scale * q[b, h] . K[b, j, h // G]) V[b, j, h // G],   j < context_lens[b],
// where token j lives in cache block block_tables[b, j // block_size] at slot j % block_size, G = H / HK.
//
// gfx950 mapping.
//  * A workgroup (4 waves) owns one chunk of `chunk` consecutive tokens of one sequence and ALL query heads (<= 16).
//    A cache slot row [HK][D] is contiguous (HK * 256 bytes), so the score GEMM contracts over the whole row
//    c = (kv head, d) with a block-diagonal query operand B[c, h] = q[h, d] if c's kv head is h's group else 0:
//    the 16 MFMA columns are 16 real heads instead of 8 heads padded to 16, and each K slot row feeds the MFMA A
//    operand straight from global memory (lane = token, 16 contiguous bytes per k-step).
//  * Each wave walks 16-token tiles (K loaded into registers in MFMA layout, V coalesced; three waves per SIMD
//    keep loads in flight): S^T[16 tok x 16 heads] = K Q^T (HK*4 MFMA 16x16x32), online softmax in fp32 with exp2, then
//    O^T[c, h] += V^T P^T (MFMA 16x16x16 per 16 output dims and kv head). V is written row-major into a private LDS
//    tile with 16-byte stores and read back transposed by ds_read_b64_tr_b16, which hands each lane four tokens of
//    one column: exactly the A operand. P^T is already in the B layout, no shuffles.
//  * Split-KV: chunks of a sequence run as independent workgroups. The four waves of a workgroup are merged in LDS;
//    a sequence that fits one chunk is written directly, the others leave fp32 partials (O, m, l) that a small
//    second kernel merges. Merging in the split kernel itself (last workgroup to arrive) was measured slower: every
//    workgroup then holds its CU slot through a write-through wait and an atomic round trip.
#include "vox_common.h"
#include "vox_kernels.h"

namespace vox {

namespace {

constexpr int kD = 128;
constexpr int kTile = 16;     // tokens per wave iteration
constexpr int kWaves = 4;
constexpr int kMaxHeads = 16;

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma_16x16x16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// Transposed LDS read: within each 16-lane group, lane j returns element j%4 of the 8-byte chunks that lanes
// 4r + j/4 (r = 0..3) address, i.e. four rows of one column when lanes 4r + q point at row r, column 4q.
__device__ __forceinline__ s16x4 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

template <int HK>
struct Tile {
  static constexpr int ROW = HK * kD;              // elements per cache slot row
  static constexpr int KC = ROW / 32;              // score MFMA k-steps
  static constexpr int VP = kTile * ROW / 8 / 64;  // 16-byte V pieces per lane per tile
  static constexpr int PPR = ROW / 8;              // 16-byte pieces per slot row
  u32x4 k[KC];
  u32x4 v[VP];
  bool ok;  // the tile's cache block is mapped
};

// Issues the loads of the 16-token tile whose first token sits at cache slot slot0 (a tile never straddles a cache
// block). Every load is unconditional and in bounds, so the compiler can count outstanding loads exactly: the caller
// maps an unmapped block to block 0 and masks what it read. K rows land in MFMA A layout (lane = token r16), V
// pieces coalesced (16 bytes per lane, whole slot rows per instruction).
template <int HK>
__device__ __forceinline__ void load_tile(Tile<HK>& T, const DecodeArgs& p, int64_t slot0, int r16, int jq,
                                          int lane) {
  using TT = Tile<HK>;
  const uint16_t* kp = p.k_cache + (slot0 + r16) * TT::ROW + jq * 8;
#pragma unroll
  for (int kc = 0; kc < TT::KC; ++kc) T.k[kc] = ld_g16(kp + kc * 32);
#pragma unroll
  for (int i = 0; i < TT::VP; ++i) {
    const int pc = i * 64 + lane;
    T.v[i] = ld_g16(p.v_cache + (slot0 + pc / TT::PPR) * TT::ROW + (pc % TT::PPR) * 8);
  }
}

template <int HK>
__global__ __launch_bounds__(256, 3) void decode_kernel(DecodeArgs p) {
  using TT = Tile<HK>;
  constexpr int ROW = TT::ROW;
  constexpr int VROW = ROW + 16;  // padded LDS row: the 16 rows a transposed read touches hit distinct banks
  // Per-wave V tiles [16 tokens][VROW]; reused as fp32 scratch for the in-workgroup merge.
  constexpr int kVtElems = kWaves * kTile * VROW;
  constexpr int kRedFloats = kWaves * kMaxHeads * kD + 2 * kWaves * kMaxHeads;
  constexpr int kLdsBytes = (kVtElems * 2 > kRedFloats * 4) ? kVtElems * 2 : kRedFloats * 4;
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[kLdsBytes];

  // Sequences vary fastest in dispatch order: chunk 0 of every sequence first, so the trailing chunk ids that most
  // sequences do not have (early exits) are dispatched last instead of between live workgroups.
  const int b = blockIdx.x;
  const int c = blockIdx.y;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int jq = lane >> 4;
  const int H = p.num_heads;
  const int max_ctx = p.max_blocks * p.block_size;
  const int tok0 = c * p.chunk;  // < max_ctx: c < max_chunks
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;

  // Independent loads issued together (one round trip): the context length, this lane's query row and the block
  // id of this wave's first tile. Query row of head r16: d = kq*32 + jq*8 + [0, 8); the score B operand for k-step
  // kc is piece kc % 4 when kc's kv head (kc / 4) is the lane's group, else zero: block-diagonal over (kv head, d).
  const int ctx_raw = p.context_lens[b];
  const int h = r16;
  const int hg = h < H ? h / p.group : -1;
  u32x4 qv[4];
  {
    const uint16_t* qb = p.q + (int64_t)b * p.q_row_stride + (int64_t)(h < H ? h : 0) * kD + jq * 8;
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) qv[kq] = ld_g16(qb + kq * 32);
  }
  int64_t blk = bt_row[min(tok0 + w * kTile, max_ctx - 1) / p.block_size];

  // A context longer than the block table can address is cut to it: keeps chunk ids inside the partial buffer.
  const int ctx = min(ctx_raw, max_ctx);
  uint16_t* out_b = p.out + (int64_t)b * H * kD;
  if (ctx <= 0) {  // padded row of a captured batch: defined zeros
    if (c == 0)
      for (int i = tid; i < H * kD; i += 256) out_b[i] = 0;
    return;
  }
  const int n_chunks = (ctx + p.chunk - 1) / p.chunk;
  if (c >= n_chunks) return;
  const int tok_end = min(ctx, tok0 + p.chunk);

  float m = -INFINITY;
  float lsum = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint16_t* vt = reinterpret_cast<uint16_t*>(lds_raw) + w * kTile * VROW;
  // this lane's transposed-read address inside a d-tile: row jq*4 + r16/4, column 4*(r16%4)
  const uint16_t* vtr = vt + (jq * 4 + (r16 >> 2)) * VROW + 4 * (r16 & 3);

  auto compute = [&](const Tile<HK>& T, int t0) {
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < TT::KC; ++kc) s = mfma_16x16x32(T.k[kc], hg == kc / 4 ? qv[kc % 4] : zero4(), s);
    // lane (head r16) holds tokens t0 + jq*4 + [0, 4)
    float x[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const bool ok = T.ok && (t0 + jq * 4 + rr) < tok_end;
      x[rr] = ok ? s[rr] * p.scale_log2 : -INFINITY;
      tmax = fmaxf(tmax, x[rr]);
    }
    tmax = col_max4(tmax);
    const float m_new = fmaxf(m, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    float ps = 0.f;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      x[rr] = fast_exp2(x[rr] - m_use);
      ps += x[rr];
    }
    lsum = lsum * alpha + ps;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;

    // V tile -> LDS, row-major, 16-byte stores; rows of tokens past tok_end or of an unmapped block are zeroed
    // (they meet p = 0 in P V, and unwritten cache slots may hold any bit pattern)
#pragma unroll
    for (int i = 0; i < TT::VP; ++i) {
      const int pc = i * 64 + lane;
      const bool ok = T.ok && (t0 + pc / TT::PPR) < tok_end;
      *reinterpret_cast<u32x4*>(vt + (pc / TT::PPR) * VROW + (pc % TT::PPR) * 8) = ok ? T.v[i] : zero4();
    }
    wave_lds_sync();

    // P^T operand: k-slots jq*4 + [0, 4) = tokens jq*4 + [0, 4)
    const uint32_t p01 = pack_bf16x2(x[0], x[1]);
    const uint32_t p23 = pack_bf16x2(x[2], x[3]);
    const s16x4 pv = __builtin_bit_cast(s16x4, u32x2{p01, p23});
    const s16x4 pz = s16x4{0, 0, 0, 0};
#pragma unroll
    for (int g = 0; g < HK; ++g) {
      const s16x4 pb = (hg == g) ? pv : pz;
      s16x4 va[8];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) va[dt] = lds_read_tr16(vtr + g * kD + dt * 16);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[dt] = mfma_16x16x16(va[dt], pb, acc[dt]);
    }
    wave_lds_sync();
  };

  // This wave's tiles: tok0 + w*16 + k*64. Latency is hidden across waves (3 per SIMD), not inside one; the next
  // tile's block id is read one tile ahead so each tile costs one memory round trip. Columns stay below max_blocks
  // because the context is cut to the table's reach.
  const int step = kWaves * kTile;
  for (int t0 = tok0 + w * kTile; t0 < tok_end; t0 += step) {
    const int tn = min(t0 + step, tok_end - 1);
    const int64_t blk_next = bt_row[tn / p.block_size];
    Tile<HK> T;
    T.ok = blk >= 0 && blk < p.num_blocks;
    load_tile<HK>(T, p, (T.ok ? blk : 0) * p.block_size + (t0 % p.block_size), r16, jq, lane);
    __builtin_amdgcn_sched_barrier(0);  // all of the tile's loads issue before any of them is waited on
    compute(T, t0);
    blk = blk_next;
  }

  // ---- merge the four waves of this workgroup (fp32, in LDS) ----
  lsum = col_sum4(lsum);
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds_raw);
  constexpr int kMOff = kWaves * kMaxHeads * kD;
  constexpr int kLOff = kMOff + kWaves * kMaxHeads;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    *reinterpret_cast<f32x4*>(&red[(w * kMaxHeads + r16) * kD + dt * 16 + jq * 4]) = acc[dt];
  if (jq == 0) {
    red[kMOff + w * kMaxHeads + r16] = m;
    red[kLOff + w * kMaxHeads + r16] = lsum;
  }
  __syncthreads();

  const int hh = tid >> 4;        // head
  const int d0 = (tid & 15) * 8;  // 8 consecutive dims
  float M = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, red[kMOff + ww * kMaxHeads + hh]);
  const float Mu = M == -INFINITY ? 0.f : M;
  float L = 0.f;
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;
#pragma unroll
  for (int ww = 0; ww < kWaves; ++ww) {
    const float e = fast_exp2(red[kMOff + ww * kMaxHeads + hh] - Mu);
    L += e * red[kLOff + ww * kMaxHeads + hh];
    const float* src = &red[(ww * kMaxHeads + hh) * kD + d0];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] += e * src[i];
  }

  if (n_chunks == 1) {
    if (hh < H) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      const u32x4 ov = u32x4{pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv),
                             pack_bf16x2(o[4] * inv, o[5] * inv), pack_bf16x2(o[6] * inv, o[7] * inv)};
      *reinterpret_cast<u32x4*>(out_b + hh * kD + d0) = ov;
    }
    return;
  }

  // ---- split-KV: publish this chunk's partial; decode_merge_kernel (next on the stream) combines them ----
  float* part = p.partials + ((int64_t)b * p.max_chunks + c) * kPartialFloats;
  *reinterpret_cast<f32x4*>(&part[hh * kD + d0]) = f32x4{o[0], o[1], o[2], o[3]};
  *reinterpret_cast<f32x4*>(&part[hh * kD + d0 + 4]) = f32x4{o[4], o[5], o[6], o[7]};
  if ((tid & 15) == 0) {
    part[kMaxHeads * kD + hh] = M;
    part[kMaxHeads * kD + kMaxHeads + hh] = L;
  }
}

// Combines the chunk partials of every sequence that the decode kernel split (n_chunks > 1): online rescale over
// the chunks (fp32), normalize, bf16. One workgroup per sequence, thread = (head, 8 dims); partial loads of four
// chunks are issued together. Runs after decode_kernel on the same stream, which makes the partials visible.
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs p) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int hh = tid >> 4;
  const int d0 = (tid & 15) * 8;
  const int ctx = min(p.context_lens[b], p.max_blocks * p.block_size);
  const int n_chunks = (ctx + p.chunk - 1) / p.chunk;
  if (n_chunks <= 1 || hh >= p.num_heads) return;
  const float* pb = p.partials + (int64_t)b * p.max_chunks * kPartialFloats;
  float M2 = -INFINITY, L2 = 0.f;
  float o2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o2[i] = 0.f;
  for (int c0 = 0; c0 < n_chunks; c0 += 4) {
    float mc[4], lc[4];
    f32x4 oa[4], ob[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float* pc = pb + (int64_t)min(c0 + u, n_chunks - 1) * kPartialFloats;
      mc[u] = (c0 + u < n_chunks) ? pc[kMaxHeads * kD + hh] : -INFINITY;
      lc[u] = pc[kMaxHeads * kD + kMaxHeads + hh];
      oa[u] = *reinterpret_cast<const f32x4*>(&pc[hh * kD + d0]);
      ob[u] = *reinterpret_cast<const f32x4*>(&pc[hh * kD + d0 + 4]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float mn = fmaxf(M2, mc[u]);
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float a = fast_exp2(M2 - mu);
      const float e = fast_exp2(mc[u] - mu);
      L2 = L2 * a + e * lc[u];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o2[i] = o2[i] * a + e * oa[u][i];
        o2[i + 4] = o2[i + 4] * a + e * ob[u][i];
      }
      M2 = mn;
    }
  }
  const float inv = L2 > 0.f ? 1.f / L2 : 0.f;
  const u32x4 ov = u32x4{pack_bf16x2(o2[0] * inv, o2[1] * inv), pack_bf16x2(o2[2] * inv, o2[3] * inv),
                         pack_bf16x2(o2[4] * inv, o2[5] * inv), pack_bf16x2(o2[6] * inv, o2[7] * inv)};
  *reinterpret_cast<u32x4*>(p.out + ((int64_t)b * p.num_heads + hh) * kD + d0) = ov;
}

}  // namespace

int decode_chunk_tokens(int batch, int max_ctx) {
  // Chunks are multiples of one 4-wave x 16-token step. Prefer 256-token chunks (fewer partials to merge), halve
  // them while the grid would leave the 256 CUs with less than ~4 workgroups each.
  int chunk = 256;
  while (chunk > kWaves * kTile * 2) {
    const int64_t wgs = (int64_t)batch * ((max_ctx + chunk - 1) / chunk);
    if (wgs >= 1024) break;
    chunk /= 2;
  }
  return chunk;
}

hipError_t launch_decode(const DecodeArgs& a, int num_kv_heads, int max_ctx, hipStream_t stream) {
  const int n_chunks = (max_ctx + a.chunk - 1) / a.chunk;
  dim3 grid((unsigned)a.batch, (unsigned)(n_chunks > 0 ? n_chunks : 1));
  if (num_kv_heads == 1)
    decode_kernel<1><<<grid, dim3(256), 0, stream>>>(a);
  else
    decode_kernel<2><<<grid, dim3(256), 0, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || n_chunks <= 1) return e;
  decode_merge_kernel<<<dim3((unsigned)a.batch), dim3(256), 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace vox
