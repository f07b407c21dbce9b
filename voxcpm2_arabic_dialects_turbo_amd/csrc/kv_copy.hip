// Kernel 4: copy the first n token slots of KV-cache blocks, in every (layer, K/V) plane, in one launch.
//
// Semantics (reference: nanovllm_voxcpm/kernels/kv_copy.py:17-41, copy_kv_block_prefix): the engine keeps all
// causal layers' K/V in one tensor [layers, 2, blocks, block_size, kv_heads, head_dim]; for every entry
// (src, dst, n) and every plane, the first n slots of block src are copied over the first n slots of block dst
// (n clipped to block_size; entries with n <= 0 do nothing). A block's first n slots are one contiguous run of
// n * per_token elements in each plane. Bit-exact copy. Entries whose src or dst is outside the cache are skipped
// (the reference would read or write out of bounds); entries that write a block another entry reads race, as in the
// reference's single launch.
//
// gfx950 mapping: workgroup (entry, plane, chunk of 16 KiB); each lane moves 16 bytes per access, all four of its
// loads issue before its stores. A full 256-slot bf16 block plane of the model (128 KiB) is eight workgroups, so
// one entry over 72 planes is 576 workgroups: enough to cover the chip even for a single prefix copy.
#include <type_traits>

#include "vox_common.h"
#include "vox_kernels.h"

namespace vox {

namespace {

constexpr int kThreadsCopy = 256;
constexpr int kPerLane = 4;                                  // 16-byte pieces per lane per chunk
constexpr int kChunkPieces = kThreadsCopy * kPerLane;        // 16 KiB per workgroup

template <int VEC>
__global__ __launch_bounds__(kThreadsCopy) void copy_block_prefix_kernel(CopyArgs a) {
  const int e = blockIdx.x;
  const int64_t plane = blockIdx.y;
  const int chunk = blockIdx.z;
  const int32_t src = a.entries[3 * e];
  const int32_t dst = a.entries[3 * e + 1];
  const int n = min(a.entries[3 * e + 2], a.block_size);
  if (n <= 0 || src < 0 || src >= a.num_blocks || dst < 0 || dst >= a.num_blocks) return;
  // in units of VEC elements (16 bytes when VEC == 8)
  const int64_t run = (int64_t)n * a.per_token / VEC;
  const int64_t block_units = (int64_t)a.block_size * a.per_token / VEC;
  const int64_t plane_units = a.num_blocks * block_units;
  const int64_t base = (int64_t)chunk * kChunkPieces;
  if (base >= run) return;
  typedef typename std::conditional<VEC == 8, u32x4, uint16_t>::type Unit;
  const Unit* s = reinterpret_cast<const Unit*>(a.kv) + plane * plane_units + src * block_units;
  Unit* d = reinterpret_cast<Unit*>(a.kv) + plane * plane_units + dst * block_units;
  Unit v[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int64_t off = base + i * kThreadsCopy + threadIdx.x;
    if (off < run) v[i] = s[off];
  }
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int64_t off = base + i * kThreadsCopy + threadIdx.x;
    if (off < run) d[off] = v[i];
  }
}

}  // namespace

hipError_t launch_copy_block_prefix(const CopyArgs& a, int max_tokens, bool vec16, hipStream_t stream) {
  const int vec = vec16 ? 8 : 1;
  const int64_t max_units = (int64_t)max_tokens * a.per_token / vec;
  const int64_t chunks = (max_units + kChunkPieces - 1) / kChunkPieces;
  if (a.num_entries <= 0 || a.num_planes <= 0 || chunks <= 0) return hipSuccess;
  const dim3 grid((unsigned)a.num_entries, (unsigned)a.num_planes, (unsigned)chunks);
  if (vec16)
    copy_block_prefix_kernel<8><<<grid, dim3(kThreadsCopy), 0, stream>>>(a);
  else
    copy_block_prefix_kernel<1><<<grid, dim3(kThreadsCopy), 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace vox
