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
 * workgroups of 256 threads in a grid-stride loop over the 1 KiB units, and stores one folded
 * word per thread to `sink` (grid * 256 uint32). Every chunk id must satisfy
 * (c + 1) * chunk_bytes <= base_bytes (not checked on the device). chunk_bytes must be a
 * multiple of 1024, `base` 16-byte aligned, and n_chunks * chunk_bytes / 1024 < 2^31.
 * Returns MIP_OK, MIP_EINVAL or a hipError_t. Used by bench.py to report the achievable
 * random-chunk read rate.
 */
int mip_hbm_read_probe(const void* base, int64_t base_bytes, const int32_t* chunk_ids, int64_t n_chunks,
                       int32_t chunk_bytes, uint32_t* sink, int32_t grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MIPAGED_PROBE_H_ */
