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
//  * Each wave walks 32-token tiles: S^T[32 tok x 16 heads] = K Q^T (2 x HK*4 MFMAs 16x16x32), online softmax in
//    fp32 with exp2, then O^T[d, h] += V^T P^T. V needs its token axis contiguous per lane, so each wave transposes
//    its V tile through a private LDS buffer; P^T is already in the MFMA B layout (no shuffles).
//  * Split-KV: chunks of a sequence run as independent workgroups. The four waves of a workgroup are merged in LDS;
//    chunks are merged by the last workgroup of the sequence to finish (atomic arrival counter, reset to zero by
//    that workgroup), so one launch per layer does the whole decode with no combine kernel.
#include "vox_common.h"
#include "vox_kernels.h"

namespace vox {

namespace {

constexpr int kD = 128;
constexpr int kTile = 32;     // tokens per wave iteration
constexpr int kWaves = 4;
constexpr int kVtStride = 36; // bf16 per LDS row of a transposed V tile (32 tokens + 4 pad)
constexpr int kMaxHeads = 16;

template <int HK>
__global__ __launch_bounds__(256, 2) void decode_kernel(DecodeArgs p) {
  constexpr int ROW = HK * kD;   // elements per cache slot row
  constexpr int KC = ROW / 32;   // MFMA k-steps per score tile
  // Per-wave transposed V tiles; reused as fp32 scratch for the in-workgroup merge.
  __shared__ __attribute__((aligned(16))) uint16_t vt[kWaves][ROW][kVtStride];
  __shared__ int last_flag;

  const int b = blockIdx.y;
  const int c = blockIdx.x;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int jq = lane >> 4;
  const int H = p.num_heads;
  // A context longer than the block table can address is cut to it: keeps chunk ids inside the partial buffer.
  const int ctx = min(p.context_lens[b], p.max_blocks * p.block_size);
  uint16_t* out_b = p.out + (int64_t)b * H * kD;

  if (ctx <= 0) {  // padded row of a captured batch: defined zeros
    if (c == 0)
      for (int i = tid; i < H * kD; i += 256) out_b[i] = 0;
    return;
  }
  const int n_chunks = (ctx + p.chunk - 1) / p.chunk;
  if (c >= n_chunks) return;
  const int tok0 = c * p.chunk;
  const int tok_end = min(ctx, tok0 + p.chunk);

  // Block-diagonal query operand, lane (head r16, k-group jq): c = kc*32 + jq*8 + [0, 8).
  const int h = r16;
  const int hg = h < H ? h / p.group : -1;
  u32x4 qop[KC];
  {
    const uint16_t* qb = p.q + (int64_t)b * p.q_row_stride + (int64_t)h * kD + jq * 8;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) qop[kc] = (hg == kc / 4) ? ld_g16(qb + (kc % 4) * 32) : zero4();
  }

  float m = -INFINITY;
  float lsum = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint16_t(*vtw)[kVtStride] = vt[w];

  for (int t0 = tok0 + w * kTile; t0 < tok_end; t0 += kWaves * kTile) {
    // A 32-token tile never straddles a cache block (block_size % 32 == 0, t0 % 32 == 0).
    const int col = t0 / p.block_size;
    const int64_t blk = col < p.max_blocks ? (int64_t)p.block_tables[(int64_t)b * p.bt_stride + col] : -1;
    const bool blk_ok = blk >= 0 && blk < p.num_blocks;
    const int64_t slot0 = blk * p.block_size + (t0 % p.block_size);

    u32x4 kr[2][KC], vr[2][KC];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const bool ok = blk_ok && (t0 + s * 16 + r16) < tok_end;
      const int64_t off = (slot0 + s * 16 + r16) * ROW + jq * 8;
      const uint16_t* kp = p.k_cache + off;
      const uint16_t* vp = p.v_cache + off;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        kr[s][kc] = ok ? ld_g16(kp + kc * 32) : zero4();
        vr[s][kc] = ok ? ld_g16(vp + kc * 32) : zero4();
      }
    }

    // S^T tile: lane (head r16) holds tokens t0 + s*16 + jq*4 + [0, 4).
    f32x4 sacc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      sacc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) sacc[s] = mfma_16x16x32(kr[s][kc], qop[kc], sacc[s]);
    }

    float x[2][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const bool ok = blk_ok && (t0 + s * 16 + jq * 4 + rr) < tok_end;
        x[s][rr] = ok ? sacc[s][rr] * p.scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, x[s][rr]);
      }
    tmax = col_max4(tmax);
    const float m_new = fmaxf(m, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    float ps = 0.f;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        x[s][rr] = fast_exp2(x[s][rr] - m_use);
        ps += x[s][rr];
      }
    lsum = lsum * alpha + ps;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;

    // V tile -> LDS, transposed to [c][token].
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const u32x4 vv = vr[s][kc];
        const int row = kc * 32 + jq * 8;
        const int tc = s * 16 + r16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vtw[row + 2 * e][tc] = (uint16_t)(vv[e] & 0xffffu);
          vtw[row + 2 * e + 1][tc] = (uint16_t)(vv[e] >> 16);
        }
      }
    wave_lds_sync();

    // P^T operand: k-slots jq*8 + [0,4) = tokens jq*4 + [0,4), jq*8 + [4,8) = tokens 16 + jq*4 + [0,4).
    const u32x4 pv = u32x4{pack_bf16x2(x[0][0], x[0][1]), pack_bf16x2(x[0][2], x[0][3]),
                           pack_bf16x2(x[1][0], x[1][1]), pack_bf16x2(x[1][2], x[1][3])};
#pragma unroll
    for (int g = 0; g < HK; ++g) {
      const u32x4 pb = (hg == g) ? pv : zero4();
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint16_t* row = vtw[g * kD + dt * 16 + r16];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(row + jq * 4);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(row + 16 + jq * 4);
        acc[dt] = mfma_16x16x32(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb, acc[dt]);
      }
    }
    wave_lds_sync();
  }

  // ---- merge the four waves of this workgroup (fp32, in LDS) ----
  lsum = col_sum4(lsum);
  __syncthreads();
  float* red = reinterpret_cast<float*>(&vt[0][0][0]);
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

  // ---- split-KV: publish this chunk's partial, the last chunk of the sequence to arrive merges them ----
  float* part = p.partials + ((int64_t)b * p.max_chunks + c) * kPartialFloats;
  *reinterpret_cast<f32x4*>(&part[hh * kD + d0]) = f32x4{o[0], o[1], o[2], o[3]};
  *reinterpret_cast<f32x4*>(&part[hh * kD + d0 + 4]) = f32x4{o[4], o[5], o[6], o[7]};
  if ((tid & 15) == 0) {
    part[kMaxHeads * kD + hh] = M;
    part[kMaxHeads * kD + kMaxHeads + hh] = L;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(&p.counters[b], 1);
    last_flag = (prev == n_chunks - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();

  const float* pb = p.partials + (int64_t)b * p.max_chunks * kPartialFloats;
  float M2 = -INFINITY;
  for (int cc = 0; cc < n_chunks; ++cc) M2 = fmaxf(M2, pb[cc * kPartialFloats + kMaxHeads * kD + hh]);
  const float M2u = M2 == -INFINITY ? 0.f : M2;
  float L2 = 0.f;
  float o2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o2[i] = 0.f;
  for (int cc = 0; cc < n_chunks; ++cc) {
    const float* pc = pb + cc * kPartialFloats;
    const float e = fast_exp2(pc[kMaxHeads * kD + hh] - M2u);
    L2 += e * pc[kMaxHeads * kD + kMaxHeads + hh];
    const f32x4 a = *reinterpret_cast<const f32x4*>(&pc[hh * kD + d0]);
    const f32x4 bq = *reinterpret_cast<const f32x4*>(&pc[hh * kD + d0 + 4]);
    o2[0] += e * a[0];
    o2[1] += e * a[1];
    o2[2] += e * a[2];
    o2[3] += e * a[3];
    o2[4] += e * bq[0];
    o2[5] += e * bq[1];
    o2[6] += e * bq[2];
    o2[7] += e * bq[3];
  }
  if (hh < H) {
    const float inv = L2 > 0.f ? 1.f / L2 : 0.f;
    const u32x4 ov = u32x4{pack_bf16x2(o2[0] * inv, o2[1] * inv), pack_bf16x2(o2[2] * inv, o2[3] * inv),
                           pack_bf16x2(o2[4] * inv, o2[5] * inv), pack_bf16x2(o2[6] * inv, o2[7] * inv)};
    *reinterpret_cast<u32x4*>(out_b + hh * kD + d0) = ov;
  }
  if (tid == 0) atomicExch(&p.counters[b], 0);
}

}  // namespace

int decode_chunk_tokens(int batch, int max_ctx) {
  // Chunks are multiples of one 4-wave x 32-token step. Prefer 256-token chunks (fewer partials to merge), halve
  // them while the grid would leave the 256 CUs with less than ~8 workgroups each.
  int chunk = 256;
  while (chunk > kWaves * kTile) {
    const int64_t wgs = (int64_t)batch * ((max_ctx + chunk - 1) / chunk);
    if (wgs >= 2048) break;
    chunk /= 2;
  }
  return chunk;
}

hipError_t launch_decode(const DecodeArgs& a, int num_kv_heads, int max_ctx, hipStream_t stream) {
  const int n_chunks = (max_ctx + a.chunk - 1) / a.chunk;
  dim3 grid((unsigned)(n_chunks > 0 ? n_chunks : 1), (unsigned)a.batch);
  if (num_kv_heads == 1)
    decode_kernel<1><<<grid, dim3(256), 0, stream>>>(a);
  else
    decode_kernel<2><<<grid, dim3(256), 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace vox
