/* libvoxprobe: memory-rate probes that bench.py runs beside the attention kernels (MI355X, gfx950), C ABI.
 *
 * Measurement only: no reference counterpart, and nothing in the attention path calls them. They load and discard
 * (an XOR that is stored only on an impossible value), so their rate is what the HBM path delivers to plain vector
 * loads. Return 0 on success, 1 for a bad argument, 2 when the launch fails. Stream-ordered on `stream`.
 */
#ifndef VOX_PROBE_H_
#define VOX_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (multiple of 16, 16-byte aligned) of `buf` once with `grid` workgroups of 256 threads, grid-stride,
 * four 16-byte loads in flight per thread. `sink`: 1 KiB of device memory that is written only on an impossible
 * value. */
int vox_probe_stream_read(const void* buf, int64_t bytes, void* sink, int grid, void* stream);

/* The decode kernel's loads without its arithmetic: for each of `n_tiles` byte offsets, 16 contiguous 512-byte slot
 * rows of the K plane and the same rows of the V plane, read with the decode kernel's per-wave load layout; the
 * tiles are cut into `grid` equal contiguous ranges, one per 4-wave workgroup, `depth` (1 or 2) tiles in flight per
 * wave. Every offset + 8 KiB must lie inside both planes. */
int vox_probe_tile_read(const void* k_plane, const void* v_plane, const int64_t* tile_offsets, int64_t n_tiles,
                        void* sink, int grid, int depth, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VOX_PROBE_H_ */
