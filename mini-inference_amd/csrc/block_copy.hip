// Block copy for copy-on-write of shared prefix blocks.
//
// No reference counterpart (the reference shares only full, never-rewritten blocks,
// engine/kv_cache.py:499-508). Semantics are a bitwise memcpy of every layer's K and V
// copy of a block:  cache[l][dst][:] = cache[l][src][:]  for l in [0, num_layers).
//
// Work split: one workgroup per (pair, layer, K|V) unit, a contiguous block_bytes run in the
// pool layout; its threads copy CHUNK bytes each, kUnroll chunks in flight per thread. The
// pair is uniform over the workgroup, so its two block ids are one scalar load: from device
// memory (mip_copy_blocks), or from the kernel arguments (mip_copy_blocks_host, up to
// kInlinePairs pairs per launch), where the copy starts without any dependent memory read.
#include "mip_common.h"

namespace mip {
namespace {

template <int CHUNK> struct CopyT;
template <> struct CopyT<16> { using T = uint4; };
template <> struct CopyT<8>  { using T = uint2; };
template <> struct CopyT<4>  { using T = uint32_t; };
template <> struct CopyT<2>  { using T = uint16_t; };
template <> struct CopyT<1>  { using T = uint8_t; };

#ifndef MIP_COPY_THREADS
#define MIP_COPY_THREADS 256
#endif
constexpr int kCopyThreads = MIP_COPY_THREADS;  // threads per (pair, layer, K|V) unit
constexpr int kUnroll = 4;
constexpr int kInlinePairs = MIP_COPY_INLINE_PAIRS;

struct CopyArgs {
  char* k;
  char* v;
  const int64_t* pairs;  // device [n][2] (src, dst); null for pairs in InlinePairs
  int64_t ncb;           // blocks per layer (pool size including the scratch block)
  int64_t block_bytes;
  int num_layers;
};

// (src, dst) block ids of up to kInlinePairs pairs; -1 marks an id outside the pool.
struct InlinePairs {
  int32_t id[2 * kInlinePairs];
};
struct NoPairs {};  // pairs in device memory

template <int CHUNK, class P>
__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(CopyArgs a, P ip) {
  constexpr bool INLINE = sizeof(P) == sizeof(InlinePairs);
  using V = typename CopyT<CHUNK>::T;
  const int64_t u = blockIdx.x;  // (pair, layer, side), side fastest
  const int side = static_cast<int>(u & 1);
  const int64_t pl = u >> 1;
  const int64_t pair = pl / a.num_layers;
  const int64_t layer = pl - pair * a.num_layers;
  int64_t src, dst;
  if constexpr (INLINE) {
    src = ip.id[2 * pair];
    dst = ip.id[2 * pair + 1];
  } else {
    src = load_uniform_i64(a.pairs + 2 * pair);
    dst = load_uniform_i64(a.pairs + 2 * pair + 1);
  }
  if (src < 0 || src >= a.ncb || dst < 0 || dst >= a.ncb) return;
  char* base = (side ? a.v : a.k) + layer * a.ncb * a.block_bytes;
  const char* from = base + src * a.block_bytes;
  char* to = base + dst * a.block_bytes;
  constexpr int64_t kStep = static_cast<int64_t>(kCopyThreads) * CHUNK;
  int64_t byte = static_cast<int64_t>(threadIdx.x) * CHUNK;
  // Rounds of kUnroll chunks: every load of a round is issued before its stores (source and
  // destination are distinct blocks, but the compiler cannot know that).
  for (; byte + (kUnroll - 1) * kStep < a.block_bytes; byte += kUnroll * kStep) {
    V r[kUnroll];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) r[j] = *reinterpret_cast<const V*>(from + byte + j * kStep);
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) *reinterpret_cast<V*>(to + byte + j * kStep) = r[j];
  }
  for (; byte < a.block_bytes; byte += kStep) *reinterpret_cast<V*>(to + byte) = *reinterpret_cast<const V*>(from + byte);
}

// Picks the widest chunk the block size and the pool bases allow and fills CopyArgs (the
// caller has checked the arguments); returns the chunk width.
int copy_setup(void* k_cache, void* v_cache, int32_t num_layers, int64_t num_cache_blocks, int64_t block_bytes,
               CopyArgs& a) {
  const uint64_t align_bits = static_cast<uint64_t>(block_bytes) | reinterpret_cast<uintptr_t>(k_cache) |
                              reinterpret_cast<uintptr_t>(v_cache);
  int chunk = 16;
  while (chunk > 1 && (align_bits & (chunk - 1))) chunk >>= 1;
  a.k = static_cast<char*>(k_cache);
  a.v = static_cast<char*>(v_cache);
  a.pairs = nullptr;
  a.ncb = num_cache_blocks;
  a.block_bytes = block_bytes;
  a.num_layers = num_layers;
  return chunk;
}

// A launch's grid holds fewer than 2^32 work-items (HIP's limit on gridDim.x * blockDim.x),
// so one launch copies at most this many (pair, layer, K|V) units.
constexpr int64_t kMaxUnitsPerLaunch = ((int64_t{1} << 32) - 1) / kCopyThreads;

// Pairs one launch may take at this layer count (0: not even one pair fits).
int64_t pairs_per_launch(int32_t num_layers) { return kMaxUnitsPerLaunch / (2 * static_cast<int64_t>(num_layers)); }

template <class P>
int copy_launch(const CopyArgs& a, const P& ip, int64_t n_pairs, int chunk, hipStream_t s) {
  const int64_t units = n_pairs * a.num_layers * 2;
  if (units > kMaxUnitsPerLaunch) return MIP_EINVAL;
  const dim3 grid(static_cast<unsigned>(units)), block(kCopyThreads);
  switch (chunk) {
    case 16: hipLaunchKernelGGL((copy_blocks_kernel<16, P>), grid, block, 0, s, a, ip); break;
    case 8:  hipLaunchKernelGGL((copy_blocks_kernel<8, P>), grid, block, 0, s, a, ip); break;
    case 4:  hipLaunchKernelGGL((copy_blocks_kernel<4, P>), grid, block, 0, s, a, ip); break;
    case 2:  hipLaunchKernelGGL((copy_blocks_kernel<2, P>), grid, block, 0, s, a, ip); break;
    default: hipLaunchKernelGGL((copy_blocks_kernel<1, P>), grid, block, 0, s, a, ip); break;
  }
  return status_from_hip(hipGetLastError());
}

}  // namespace
}  // namespace mip

using namespace mip;

extern "C" int mip_copy_blocks(void* k_cache, void* v_cache, const int64_t* pairs, int32_t n_pairs,
                               int32_t num_layers, int64_t num_cache_blocks, int64_t block_bytes, void* stream) {
  if (n_pairs < 0 || num_layers <= 0 || num_cache_blocks <= 0 || block_bytes <= 0) return MIP_EINVAL;
  if (n_pairs == 0) return MIP_OK;
  if (!k_cache || !v_cache || !pairs) return MIP_EINVAL;
  const int64_t per_launch = pairs_per_launch(num_layers);
  if (per_launch < 1) return MIP_EINVAL;
  CopyArgs a;
  const int chunk = copy_setup(k_cache, v_cache, num_layers, num_cache_blocks, block_bytes, a);
  // One launch per per_launch pairs (a single one unless n_pairs * num_layers reaches 2^23).
  for (int64_t p0 = 0; p0 < n_pairs; p0 += per_launch) {
    const int64_t n = n_pairs - p0 < per_launch ? n_pairs - p0 : per_launch;
    a.pairs = pairs + 2 * p0;
    const int st = copy_launch(a, NoPairs{}, n, chunk, static_cast<hipStream_t>(stream));
    if (st) return st;
  }
  return MIP_OK;
}

extern "C" int mip_copy_blocks_host(void* k_cache, void* v_cache, const int64_t* pairs, int32_t n_pairs,
                                    int32_t num_layers, int64_t num_cache_blocks, int64_t block_bytes,
                                    void* stream) {
  if (n_pairs < 0 || num_layers <= 0 || num_cache_blocks <= 0 || block_bytes <= 0) return MIP_EINVAL;
  if (n_pairs == 0) return MIP_OK;
  if (!k_cache || !v_cache || !pairs) return MIP_EINVAL;
  const int64_t fit = pairs_per_launch(num_layers);
  if (fit < 1) return MIP_EINVAL;
  const int32_t per_launch = fit < kInlinePairs ? static_cast<int32_t>(fit) : kInlinePairs;
  CopyArgs a;
  const int chunk = copy_setup(k_cache, v_cache, num_layers, num_cache_blocks, block_bytes, a);
  // One launch per kInlinePairs pairs (fewer if the layer count is large), their ids copied into
  // the kernel arguments (an id outside [0, num_cache_blocks) becomes -1, which the kernel skips
  // like the device variant).
  InlinePairs ip;
  for (int32_t p0 = 0; p0 < n_pairs; p0 += per_launch) {
    const int32_t n = n_pairs - p0 < per_launch ? n_pairs - p0 : per_launch;
    for (int32_t i = 0; i < 2 * n; ++i) {
      const int64_t id = pairs[2 * static_cast<int64_t>(p0) + i];
      ip.id[i] = id >= 0 && id < num_cache_blocks && id <= INT32_MAX ? static_cast<int32_t>(id) : -1;
    }
    const int st = copy_launch(a, ip, n, chunk, static_cast<hipStream_t>(stream));
    if (st) return st;
  }
  return MIP_OK;
}

extern "C" int mip_version(void) { return (0 << 16) | 1; }

extern "C" const char* mip_status_string(int status) {
  switch (status) {
    case MIP_OK: return "ok";
    case MIP_EINVAL: return "invalid argument";
    case MIP_E2BIG: return "the call needs more scratch than the library's static array holds";
    case MIP_EUNSUPPORTED: return "unsupported shape (no compiled kernel)";
    default: return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown status";
  }
}
