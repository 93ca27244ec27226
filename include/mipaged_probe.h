/*
 * mipaged_probe.h — measurement helper shipped in libmipaged.so; not part of the drop-in ABI
 * (include/mipaged.h) and with no reference counterpart.
 */
#ifndef MIPAGED_PROBE_H_
#define MIPAGED_PROBE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * HBM read probe: reads chunk c = chunk_ids[i] (bytes [c * chunk_bytes, (c + 1) * chunk_bytes)
 * of `base`) for every i < n_chunks, 1 KiB per wavefront load (64 lanes x 16 bytes), with `grid`
 * workgroups of 256 threads, and stores one folded word per thread to `sink`
 * (grid * 256 uint32): the XOR of every 32-bit word the thread read, so the XOR of the whole
 * sink is that of every word of the chunks. `mode` picks the read path:
 *   MIP_PROBE_GRID_STRIDE  wavefront w of W takes 1 KiB units w, w + W, ..., 8 register loads
 *                          in flight per lane;
 *   MIP_PROBE_SPAN_LDS     wavefront w takes the contiguous units [w U / W, (w + 1) U / W) of
 *                          the list through a 3-stage ring of 4 KiB in LDS, filled by direct
 *                          global-to-LDS loads (the paged decode kernel's read path); each
 *                          wavefront's units must lie within 128 chunks (MIP_EINVAL otherwise);
 *   MIP_PROBE_SPAN_LDS_NT  the same with the nontemporal cache policy on the loads, as the
 *                          decode kernel's K/V loads.
 * Every chunk id must satisfy (c + 1) * chunk_bytes <= base_bytes (not checked on the device).
 * chunk_bytes must be a multiple of 1024, `base` 16-byte aligned, and
 * n_chunks * chunk_bytes / 1024 + 32 * grid < 2^31. Returns MIP_OK, MIP_EINVAL or a hipError_t. Used by
 * bench.py to report the achievable read rate of each pattern.
 */
enum mip_probe_mode { MIP_PROBE_GRID_STRIDE = 0, MIP_PROBE_SPAN_LDS = 1, MIP_PROBE_SPAN_LDS_NT = 2 };
int mip_hbm_read_probe(const void* base, int64_t base_bytes, const int32_t* chunk_ids, int64_t n_chunks,
                       int32_t chunk_bytes, uint32_t* sink, int32_t grid, int32_t mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MIPAGED_PROBE_H_ */
