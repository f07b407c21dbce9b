// Shared device helpers for the gfx950 paged-KV attention kernels.
//
// Everything here is written for CDNA4 (gfx950, wave64): bf16 MFMA 16x16x32, 16-byte vector memory
// operations and cross-lane reductions within one 64-lane wavefront.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vox {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// D(16x16 fp32) += A(16x32 bf16) * B(32x16 bf16).
// Lane l holds A[row = l%16][k = 8*(l/16) .. +8), B[k = 8*(l/16) .. +8)[col = l%16] and
// D[row = 4*(l/16) .. +4][col = l%16]. Which physical k a register slot stands for is free as long as A and B
// agree, which the kernels use to feed operands straight from memory.
__device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

// 16-byte global load (one dwordx4 per lane).
__device__ __forceinline__ u32x4 ld_g16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// The same load marked non-temporal (streaming): for data read once per launch, such as the decode kernel's KV cache
// tiles, so that the stream does not evict from L2 what the launch reads again (its partials, plan records, block
// tables, query rows). Measured on the 28-layer decode step of 150 sequences: 1.103 -> 1.045 ms.
__device__ __forceinline__ u32x4 ld_g16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Round-to-nearest-even fp32 -> bf16 of two values packed low/high into one dword.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));  // one v_cvt_pk_bf16_f32
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// Max / sum over the four lanes {l, l^16, l^32, l^48} that share l%16 (one MFMA column).
// Cross-row exchanges of a wavefront without LDS: v_permlane32_swap exchanges the two 32-lane halves between its
// operands, v_permlane16_swap the odd 16-lane rows of one with the even rows of the other. Called with the same
// value twice, the two results hold (in some order) x of each lane and x of its partner 32 (16) lanes away, so the
// max or sum of the pair is the same in both partners whichever operand the hardware swaps.
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xrow_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xrow_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Max / sum over the four lanes l % 16 + 16 j (j = 0..3): an MFMA D column spread over the four 16-lane rows.
__device__ __forceinline__ float col_max4(float x) { return xrow_max(xhalf_max(x)); }
__device__ __forceinline__ float col_sum4(float x) { return xrow_sum(xhalf_sum(x)); }

// Max over the 64 lanes of a wavefront: row_ror DPP steps (8, 4, 2, 1) within each 16-lane row, then the four rows
// through col_max4. No LDS (the __shfl_xor form goes through ds_bpermute, one LDS round trip per step).
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xF, 0xF, false)));
  return col_max4(x);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Inclusive prefix sum over the 64 lanes of a wavefront.
__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  return x;
}

// s_waitcnt vmcnt(0): every vector memory load of this wave has landed. Placed after loads whose registers stay live
// across a software-pipelined loop (the query operands), it lets the compiler's wait analysis see them as complete
// at the loop header; otherwise it falls back to a full vmcnt(0) inside the loop, which also waits for the
// next tile's prefetch.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Orders this wavefront's LDS writes before its later LDS reads of other lanes' data (wave-private buffers).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Transposed LDS read (ds_read_b64_tr_b16): within each 16-lane group, lane j returns element j%4 of the 8-byte
// chunks that lanes 4r + j/4 (r = 0..3) address, i.e. four rows of one column when lanes 4r + q point at row r,
// column 4q. Turns a row-major [row][col] bf16 tile into MFMA A-operand columns.
__device__ __forceinline__ s16x4 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

}  // namespace vox
