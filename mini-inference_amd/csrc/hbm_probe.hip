// HBM read probe (measurement only, no reference counterpart): how fast this GPU streams a
// given number of bytes when they arrive as given chunks (randomly placed, as the paged decode
// kernels read one (block, kv head) tile of K or V at a time, or one contiguous run). bench.py
// times it beside the decode call so that each run reports the achievable read rate next to
// the 8 TB/s data-sheet peak.
//
// Three read paths, all over 1 KiB units (one 16-byte load per lane of a wavefront):
//   * grid stride (MIP_PROBE_GRID_STRIDE): wavefront w of W takes units w, w + W, ...; the
//     unit's chunk id and offset are wave-uniform (scalar loads), and each lane keeps
//     kProbeUnroll loads in flight, folding what it read into one word stored at the end.
//   * span through an LDS ring (MIP_PROBE_SPAN_LDS, MIP_PROBE_SPAN_LDS_NT): the paged decode
//     kernel's own path. Wavefront w takes the contiguous units [w U / W, (w + 1) U / W) of the
//     chunk list, through a ring of kRingStages stages of kRingLoads direct global-to-LDS loads
//     (global_load_lds_dwordx4), the loads of stage i + kRingStages - 1 issued before stage i
//     is read; _NT sets the nontemporal cache policy on the loads, as the decode kernel's K/V
//     loads do. The wavefront's chunk ids sit in two registers (128 chunks at most).
// Every path folds each lane's 16 bytes of every unit into its word of `sink`, so the XOR of
// the whole sink is the XOR of every 32-bit word read, whatever the path.
#include "mip_common.h"
#include "mipaged_probe.h"

namespace mip {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;
constexpr int kRingStages = 3;
constexpr int kRingLoads = 4;  // 1 KiB direct loads per stage
constexpr int kRingBytes = kProbeThreads / kWave * kRingStages * kRingLoads * 1024;  // per workgroup
constexpr int kSpanChunks = 2 * kWave;  // chunk ids one wavefront holds in registers

typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;
typedef __attribute__((address_space(3))) char lchar_t;

__global__ __launch_bounds__(kProbeThreads) void hbm_read_probe_kernel(const char* __restrict__ base,
                                                                       const int32_t* __restrict__ chunk_ids,
                                                                       int n_units, int units_per_chunk,
                                                                       int chunk_bytes, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * (kProbeThreads / kWave) +
                                                  static_cast<int>(threadIdx.x) / kWave);
  const int waves = gridDim.x * (kProbeThreads / kWave);
  // 32-bit unit indices (n_units < 2^31, host-checked; with the grids used the sums below stay
  // far from the limit): a 64-bit division per unit would cost more issue slots than the load.
  auto unit_ptr = [&](int u) {
    const int c = u / units_per_chunk, r = u - c * units_per_chunk;
    return reinterpret_cast<const uint4*>(base + static_cast<int64_t>(load_uniform_i32(chunk_ids + c)) * chunk_bytes +
                                          r * 1024) + lane;
  };
  uint32_t acc = 0;
  int u = wave;
  for (; u < n_units - (kProbeUnroll - 1) * waves; u += kProbeUnroll * waves) {
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int k = 0; k < kProbeUnroll; ++k) v[k] = *unit_ptr(u + k * waves);
#pragma unroll
    for (int k = 0; k < kProbeUnroll; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; u < n_units; u += waves) {
    const uint4 v = *unit_ptr(u);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  sink[static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = acc;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int CPOL>
__global__ __launch_bounds__(kProbeThreads) void hbm_read_probe_ring_kernel(const char* __restrict__ base,
                                                                            const int32_t* __restrict__ chunk_ids,
                                                                            int n_units, int units_per_chunk,
                                                                            int chunk_bytes, uint32_t* __restrict__ sink) {
  extern __shared__ __attribute__((aligned(16))) char ring_mem[];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * (kProbeThreads / kWave) + w);
  const int waves = gridDim.x * (kProbeThreads / kWave);
  const int lo = static_cast<int>(static_cast<int64_t>(n_units) * wave / waves);
  const int hi = static_cast<int>(static_cast<int64_t>(n_units) * (wave + 1) / waves);
  const int n_chunks = n_units / units_per_chunk;
  const int cbase = lo / units_per_chunk;  // this wavefront's chunks: cbase .. cbase + 127 (host-checked)
  int id0 = cbase + lane < n_chunks ? chunk_ids[cbase + lane] : 0;
  int id1 = cbase + kWave + lane < n_chunks ? chunk_ids[cbase + kWave + lane] : 0;
  lchar_t* ring = (lchar_t*)(ring_mem) + w * kRingStages * kRingLoads * 1024;
  const uint32_t ring_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring));
  // Stage s <- units us .. us + kRingLoads - 1 (those below hi).
  auto produce = [&](int s, int us) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kRingLoads; ++j) {
      const int u = us + j;
      if (u < hi) {
        const int c = u / units_per_chunk, r = u - c * units_per_chunk, k = c - cbase;
        const int cid = k < kWave ? __builtin_amdgcn_readlane(id0, k) : __builtin_amdgcn_readlane(id1, k - kWave);
        const char* g = base + static_cast<int64_t>(cid) * chunk_bytes + r * 1024 + lane * 16;
        __builtin_amdgcn_global_load_lds((gvoid_t*)g, (lvoid_t*)(ring + (s * kRingLoads + j) * 1024), 16, 0, CPOL);
      }
    }
  };
  // The chunk ids (ordinary loads into registers) are complete before any direct load is
  // issued, so the ring's waits below count direct loads only; the empty asm tells the
  // compiler so (otherwise it waits for them again before every lane read of them).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  asm volatile("" : "+v"(id0), "+v"(id1));
  uint32_t acc = 0;
  const int n_stages = (hi - lo + kRingLoads - 1) / kRingLoads;
#pragma unroll
  for (int s = 0; s < kRingStages - 1; ++s) produce(s, lo + s * kRingLoads);
  for (int i = 0; i < n_stages; ++i) {
    produce((i + kRingStages - 1) % kRingStages, lo + (i + kRingStages - 1) * kRingLoads);
    // Loads complete in issue order: with every later stage full, at most
    // (kRingStages - 1) * kRingLoads outstanding means stage i has landed.
    if (lo + (i + kRingStages) * kRingLoads <= hi) {
      wait_vmcnt<(kRingStages - 1) * kRingLoads>();
    } else {
      wait_vmcnt<0>();
    }
    const int s = i % kRingStages;
#pragma unroll
    for (int j = 0; j < kRingLoads; ++j) {
      if (lo + i * kRingLoads + j >= hi) break;  // a range's last stage may be partial
      uint4 x;
      asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                   : "=v"(x)
                   : "v"(ring_addr + (s * kRingLoads + j) * 1024 + lane * 16)
                   : "memory");
      acc ^= x.x ^ x.y ^ x.z ^ x.w;
    }
  }
  wait_vmcnt<0>();  // no direct load may land in LDS after this wavefront ends
  sink[static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = acc;
}

}  // namespace
}  // namespace mip

extern "C" int mip_hbm_read_probe(const void* base, int64_t base_bytes, const int32_t* chunk_ids, int64_t n_chunks,
                                  int32_t chunk_bytes, uint32_t* sink, int32_t grid, int32_t mode, void* stream) {
  if (!base || !chunk_ids || !sink || n_chunks < 0 || grid <= 0 || chunk_bytes <= 0 || chunk_bytes % 1024)
    return MIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(base) & 15) || base_bytes < chunk_bytes) return MIP_EINVAL;
  if (mode != MIP_PROBE_GRID_STRIDE && mode != MIP_PROBE_SPAN_LDS && mode != MIP_PROBE_SPAN_LDS_NT) return MIP_EINVAL;
  const int64_t units = n_chunks * (chunk_bytes / 1024);
  // The kernels index units in 32 bits: u + kProbeUnroll * waves must not overflow either.
  if (units + static_cast<int64_t>(grid) * mip::kProbeThreads / mip::kWave * mip::kProbeUnroll >= (int64_t{1} << 31))
    return MIP_EINVAL;
  if (n_chunks == 0) return MIP_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int upc = chunk_bytes / 1024;
  if (mode == MIP_PROBE_GRID_STRIDE) {
    hipLaunchKernelGGL(mip::hbm_read_probe_kernel, dim3(grid), dim3(mip::kProbeThreads), 0, s,
                       static_cast<const char*>(base), chunk_ids, static_cast<int>(units), upc, chunk_bytes, sink);
    return mip::status_from_hip(hipGetLastError());
  }
  // A wavefront's contiguous range must lie within the kSpanChunks chunk ids it holds: at most
  // ceil(units / waves) units, which can straddle one more chunk on each side.
  const int64_t waves = static_cast<int64_t>(grid) * (mip::kProbeThreads / mip::kWave);
  const int64_t span_units = (units + waves - 1) / waves;
  if ((span_units + upc - 1) / upc + 2 > mip::kSpanChunks) return MIP_EINVAL;
  auto kernel = mode == MIP_PROBE_SPAN_LDS_NT ? mip::hbm_read_probe_ring_kernel<2> : mip::hbm_read_probe_ring_kernel<0>;
  static const hipError_t attr = [] {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(mip::hbm_read_probe_ring_kernel<0>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, mip::kRingBytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(mip::hbm_read_probe_ring_kernel<2>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, mip::kRingBytes);
    return e;
  }();
  if (attr != hipSuccess) return mip::status_from_hip(attr);
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(mip::kProbeThreads), mip::kRingBytes, s, static_cast<const char*>(base),
                     chunk_ids, static_cast<int>(units), upc, chunk_bytes, sink);
  return mip::status_from_hip(hipGetLastError());
}
