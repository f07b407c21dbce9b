// Per-token int8 quantization of bf16 rows: the second pass of vox_prefill_attn_int8's two-pass form.
//
// Row t (one token: every head's output, row_elems = H x 128 bf16 values) becomes
//   x = o * inv_smooth (fp32; inv_smooth null = 1), scale = max(max |x|, 1e-6) / 127,
//   out_q[t, c] = rint(x[c] / scale) (round half to even), out_scale[t] = scale,
// the formula of the fused epilogue in prefill_attn.hip, applied to the bf16 output of the attention pass instead of
// its fp32 accumulators (reference: the QUANT epilogue of nanovllm_voxcpm/kernels/prefill_attn.py:84-92, which the
// reference's unfused path applies to flash-attn's bf16 output the same way).
//
// One wave per row: lane l takes the 16-byte chunks l, l + 64, ... of the row (8 values each, coalesced; all of a
// lane's loads, and those of inv_smooth, issued before any is used), the row max is a wave reduction (DPP and lane
// swaps, no LDS), and each chunk leaves as 8 int8 codes in one 8-byte store. Short and latency-bound (one load round
// trip, a reduction, the stores); the rows are the attention pass's output, which runs just before it on the stream.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vox_common.h"
#include "vox_kernels.h"

namespace vox {
namespace {

constexpr int kQWaves = 4;
constexpr int kQMaxChunks = 4;  // 16-byte chunks per lane: rows of up to 64 x 4 x 8 = 2048 values (16 heads)

template <bool SMOOTH>
__global__ __launch_bounds__(64 * kQWaves) void quantize_rows_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                                     int row_elems, const float* __restrict__ inv_smooth,
                                                                     int8_t* __restrict__ out_q, int64_t out_row_stride,
                                                                     float* __restrict__ out_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQWaves + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int nchunk = row_elems >> 3;
  const uint16_t* xr = x + row * row_elems;
  // every load first, unconditional and in bounds (a lane past the row rereads its last chunk, then ignores it), so
  // they share one round trip (guarded loads had each waited for the one before)
  u32x4 w[kQMaxChunks];
  f32x4 sa[kQMaxChunks], sb[kQMaxChunks];
#pragma unroll
  for (int i = 0; i < kQMaxChunks; ++i) w[i] = ld_g16(xr + min(lane + 64 * i, nchunk - 1) * 8);
#pragma unroll
  for (int i = 0; i < kQMaxChunks; ++i) {
    if constexpr (SMOOTH) {
      const float* sp = inv_smooth + min(lane + 64 * i, nchunk - 1) * 8;
      sa[i] = *reinterpret_cast<const f32x4*>(sp);
      sb[i] = *reinterpret_cast<const f32x4*>(sp + 4);
    } else {
      sa[i] = sb[i] = f32x4{1.f, 1.f, 1.f, 1.f};
    }
  }
  float v[kQMaxChunks][8];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kQMaxChunks; ++i) {
    const bool live = lane + 64 * i < nchunk;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i][2 * j] = bf16_bits_to_float(w[i][j] & 0xFFFFu) * (j < 2 ? sa[i][2 * j] : sb[i][2 * j - 4]);
      v[i][2 * j + 1] = bf16_bits_to_float(w[i][j] >> 16) * (j < 2 ? sa[i][2 * j + 1] : sb[i][2 * j - 3]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = live ? fmaxf(amax, fabsf(v[i][e])) : amax;
  }
  amax = wave_max(amax);
  const float scale = fmaxf(amax, 1e-6f) / 127.f;
  // rint(x / scale) without a division per element, as in the fused epilogue: y = x * (1 / scale) is within 2.5e-5 of
  // the quotient (|x / scale| <= 127.5, two roundings), so rint(y) is the same code unless y lies within 1e-4 of a
  // half-integer; those rare elements take the division.
  const float rs = 1.f / scale;
  int8_t* qr = out_q + row * out_row_stride;
#pragma unroll
  for (int i = 0; i < kQMaxChunks; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunk) {
      uint32_t packed[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = v[i][e] * rs;
        float r = __builtin_rintf(y);
        if (__builtin_expect(fabsf(fabsf(y - r) - 0.5f) < 1e-4f, 0)) r = __builtin_rintf(v[i][e] / scale);
        packed[e >> 2] |= (uint32_t)(uint8_t)(int8_t)(int)r << (8 * (e & 3));
      }
      *reinterpret_cast<u32x2*>(qr + c * 8) = u32x2{packed[0], packed[1]};
    }
  }
  if (lane == 0) out_scale[row] = scale;
}

}  // namespace

hipError_t launch_quantize_rows(const uint16_t* x, int64_t rows, int row_elems, const float* inv_smooth, int8_t* out_q,
                                int64_t out_row_stride, float* out_scale, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (row_elems <= 0 || row_elems % 8 || row_elems > 64 * 8 * kQMaxChunks) return hipErrorInvalidValue;
  const int64_t grid = (rows + kQWaves - 1) / kQWaves;
  if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
  if (inv_smooth)
    quantize_rows_kernel<true><<<dim3((unsigned)grid), dim3(64 * kQWaves), 0, stream>>>(x, rows, row_elems, inv_smooth,
                                                                                      out_q, out_row_stride, out_scale);
  else
    quantize_rows_kernel<false><<<dim3((unsigned)grid), dim3(64 * kQWaves), 0, stream>>>(x, rows, row_elems, nullptr,
                                                                                       out_q, out_row_stride, out_scale);
  return hipGetLastError();
}

}  // namespace vox
