// HBM read probe (measurement only, no reference counterpart): how fast this GPU streams a
// given number of bytes when they arrive as randomly placed chunks, the access pattern of the
// paged decode kernels (one 2 KiB (block, kv head) tile of K or V at a time at the Qwen2.5-0.5B
// shape). bench.py times it beside the decode call so that each run reports the achievable
// read rate next to the 8 TB/s data-sheet peak.
//
// Work unit: 1 KiB of one chunk, read by one wavefront with one 16-byte load per lane. Wavefront w
// of W takes units w, w + W, ...; the unit's chunk id and offset are wave-uniform (scalar loads
// and arithmetic), and each lane keeps kProbeUnroll loads in flight, folding what it read into
// one word that is stored at the end (so no load is optimised away).
#include "mip_common.h"
#include "mipaged_probe.h"

namespace mip {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;

__global__ __launch_bounds__(kProbeThreads) void hbm_read_probe_kernel(const char* __restrict__ base,
                                                                       const int32_t* __restrict__ chunk_ids,
                                                                       int n_units, int units_per_chunk,
                                                                       int chunk_bytes, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * (kProbeThreads / kWave) +
                                                  static_cast<int>(threadIdx.x) / kWave);
  const int waves = gridDim.x * (kProbeThreads / kWave);
  auto unit_ptr = [&](int64_t u) {
    const int c = static_cast<int>(u / units_per_chunk), r = static_cast<int>(u - static_cast<int64_t>(c) * units_per_chunk);
    return reinterpret_cast<const uint4*>(base + static_cast<int64_t>(load_uniform_i32(chunk_ids + c)) * chunk_bytes +
                                          r * 1024) + lane;
  };
  uint32_t acc = 0;
  int64_t u = wave;
  for (; u + static_cast<int64_t>(kProbeUnroll - 1) * waves < n_units; u += static_cast<int64_t>(kProbeUnroll) * waves) {
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int k = 0; k < kProbeUnroll; ++k) v[k] = *unit_ptr(u + static_cast<int64_t>(k) * waves);
#pragma unroll
    for (int k = 0; k < kProbeUnroll; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; u < n_units; u += waves) {
    const uint4 v = *unit_ptr(u);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  sink[static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = acc;
}

}  // namespace
}  // namespace mip

extern "C" int mip_hbm_read_probe(const void* base, int64_t base_bytes, const int32_t* chunk_ids, int64_t n_chunks,
                                  int32_t chunk_bytes, uint32_t* sink, int32_t grid, void* stream) {
  if (!base || !chunk_ids || !sink || n_chunks < 0 || grid <= 0 || chunk_bytes <= 0 || chunk_bytes % 1024)
    return MIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(base) & 15) || base_bytes < chunk_bytes) return MIP_EINVAL;
  const int64_t units = n_chunks * (chunk_bytes / 1024);
  if (units >= (int64_t{1} << 31)) return MIP_EINVAL;
  if (n_chunks == 0) return MIP_OK;
  hipLaunchKernelGGL(mip::hbm_read_probe_kernel, dim3(grid), dim3(mip::kProbeThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const char*>(base), chunk_ids,
                     static_cast<int>(units), chunk_bytes / 1024, chunk_bytes, sink);
  return mip::status_from_hip(hipGetLastError());
}
