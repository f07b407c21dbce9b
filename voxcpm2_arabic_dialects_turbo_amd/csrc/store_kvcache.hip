// Kernel 1: scatter of a step's K/V rows into the paged KV cache.
//
// Semantics (reference: nanovllm_voxcpm/model/layers.py:266-305): for every token i whose slot s = slot_mapping[i]
// is not -1, the row k[i] (num_kv_heads * head_dim contiguous elements, rows strided by k_row_stride) is copied to
// k_cache.flat[s * row .. (s + 1) * row), and likewise v[i] to v_cache. Bit-exact copy, no arithmetic.
//
// Layout on gfx950: one slot row is 2 * 128 bf16 = 512 bytes for the production shape, i.e. 32 lanes x 16 bytes.
// Each lane moves 16 bytes with one dwordx4 load and one dwordx4 store, so a wave stores two full, aligned 512-byte
// cache rows per instruction. Work is flattened over (token, tensor, 16-byte piece) so any row width that is a
// multiple of 8 elements is covered, and a grid-stride loop keeps the grid small for large N.
#include <type_traits>

#include "vox_common.h"

namespace vox {

// VEC = elements per lane access: 8 (16-byte path, all addresses 16-byte aligned) or 1 (2-byte fallback).
template <int VEC>
__global__ __launch_bounds__(256) void store_kvcache_kernel(const uint16_t* __restrict__ k,
                                                            const uint16_t* __restrict__ v, int64_t k_row_stride,
                                                            int64_t v_row_stride, uint16_t* __restrict__ k_cache,
                                                            uint16_t* __restrict__ v_cache, int64_t num_slots,
                                                            const int32_t* __restrict__ slot_mapping, int64_t n,
                                                            int row_elems) {
  const int pieces = row_elems / VEC;          // per token per tensor
  const int64_t total = n * 2 * (int64_t)pieces;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int64_t tok;
    int rem;
    if (total <= 0x7fffffff) {  // 32-bit index arithmetic whenever it fits (every real step)
      const int i32 = (int)idx;
      tok = i32 / (2 * pieces);
      rem = i32 - (int)tok * 2 * pieces;
    } else {
      tok = idx / (2 * pieces);
      rem = (int)(idx - tok * 2 * pieces);
    }
    const int which = rem >= pieces;  // 0: key, 1: value
    const int piece = rem - which * pieces;
    // The source row and the slot load together (the row index is always valid), so the copy costs one round trip.
    const uint16_t* src = (which ? v + tok * v_row_stride : k + tok * k_row_stride) + piece * VEC;
    typedef typename std::conditional<VEC == 8, u32x4, uint16_t>::type Unit;
    const Unit val = *reinterpret_cast<const Unit*>(src);
    const int64_t slot = slot_mapping[tok];
    asm volatile("" ::"v"(val), "v"(slot));  // keeps the row load ahead of the branch below (not sunk into it)
    // -1 marks a padded row (graph-captured batches); the range check keeps a bad slot from writing outside the
    // cache (the reference would write out of bounds there).
    if (slot < 0 || slot >= num_slots) continue;
    uint16_t* dst = (which ? v_cache : k_cache) + slot * row_elems + piece * VEC;
    *reinterpret_cast<Unit*>(dst) = val;
  }
}

hipError_t launch_store_kvcache(const void* k, const void* v, int64_t k_row_stride, int64_t v_row_stride,
                                void* k_cache, void* v_cache, int64_t num_slots, const int32_t* slot_mapping,
                                int64_t n, int row_elems, bool vec16, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const int threads = 256;
  const int vec = vec16 ? 8 : 1;
  const int64_t total = n * 2 * (int64_t)(row_elems / vec);
  int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 65536) blocks = 65536;  // grid-stride loop covers the rest
  if (vec16) {
    store_kvcache_kernel<8><<<dim3((unsigned)blocks), dim3(threads), 0, stream>>>(
        (const uint16_t*)k, (const uint16_t*)v, k_row_stride, v_row_stride, (uint16_t*)k_cache, (uint16_t*)v_cache,
        num_slots, slot_mapping, n, row_elems);
  } else {
    store_kvcache_kernel<1><<<dim3((unsigned)blocks), dim3(threads), 0, stream>>>(
        (const uint16_t*)k, (const uint16_t*)v, k_row_stride, v_row_stride, (uint16_t*)k_cache, (uint16_t*)v_cache,
        num_slots, slot_mapping, n, row_elems);
  }
  return hipGetLastError();
}

}  // namespace vox
