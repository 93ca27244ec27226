// Block copy for copy-on-write of shared prefix blocks.
//
// No reference counterpart (the reference shares only full, never-rewritten blocks,
// engine/kv_cache.py:499-508). Semantics are a bitwise memcpy of every layer's K and V
// copy of a block:  cache[l][dst][:] = cache[l][src][:]  for l in [0, num_layers).
//
// Work split: one lane per CHUNK bytes; the flat index runs over
// (pair, layer, K|V, chunk) with chunks fastest, so each wavefront streams contiguous
// bytes of one block (a (block, layer) unit is contiguous in the pool layout).
#include "mip_common.h"

namespace mip {
namespace {

template <int CHUNK> struct CopyT;
template <> struct CopyT<16> { using T = uint4; };
template <> struct CopyT<8>  { using T = uint2; };
template <> struct CopyT<4>  { using T = uint32_t; };
template <> struct CopyT<2>  { using T = uint16_t; };
template <> struct CopyT<1>  { using T = uint8_t; };

struct CopyArgs {
  char* k;
  char* v;
  const int64_t* pairs;
  int64_t ncb;           // blocks per layer (pool size including the scratch block)
  int64_t block_bytes;
  int64_t chunks_per_block;
  int64_t total;         // n_pairs * num_layers * 2 * chunks_per_block
  int num_layers;
};

template <int CHUNK>
__global__ __launch_bounds__(256) void copy_blocks_kernel(CopyArgs a) {
  using V = typename CopyT<CHUNK>::T;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < a.total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = i % a.chunks_per_block;
    const int64_t u = i / a.chunks_per_block;       // (pair, layer, side)
    const int side = static_cast<int>(u & 1);
    const int64_t pl = u >> 1;
    const int64_t layer = pl % a.num_layers;
    const int64_t pair = pl / a.num_layers;
    const int64_t src = a.pairs[2 * pair];
    const int64_t dst = a.pairs[2 * pair + 1];
    if (src < 0 || src >= a.ncb || dst < 0 || dst >= a.ncb) continue;
    char* base = (side ? a.v : a.k) + layer * a.ncb * a.block_bytes;
    const int64_t byte = c * CHUNK;
    *reinterpret_cast<V*>(base + dst * a.block_bytes + byte) =
        *reinterpret_cast<const V*>(base + src * a.block_bytes + byte);
  }
}

}  // namespace
}  // namespace mip

using namespace mip;

extern "C" int mip_copy_blocks(void* k_cache, void* v_cache, const int64_t* pairs, int32_t n_pairs,
                               int32_t num_layers, int64_t num_cache_blocks, int64_t block_bytes, void* stream) {
  if (n_pairs < 0 || num_layers <= 0 || num_cache_blocks <= 0 || block_bytes <= 0) return MIP_EINVAL;
  if (n_pairs == 0) return MIP_OK;
  if (!k_cache || !v_cache || !pairs) return MIP_EINVAL;
  const uint64_t align_bits = static_cast<uint64_t>(block_bytes) | reinterpret_cast<uintptr_t>(k_cache) |
                              reinterpret_cast<uintptr_t>(v_cache);
  int chunk = 16;
  while (chunk > 1 && (align_bits & (chunk - 1))) chunk >>= 1;
  CopyArgs a;
  a.k = static_cast<char*>(k_cache);
  a.v = static_cast<char*>(v_cache);
  a.pairs = pairs;
  a.ncb = num_cache_blocks;
  a.block_bytes = block_bytes;
  a.chunks_per_block = block_bytes / chunk;
  a.num_layers = num_layers;
  a.total = static_cast<int64_t>(n_pairs) * num_layers * 2 * a.chunks_per_block;
  const int threads = 256;
  const int64_t want = (a.total + threads - 1) / threads;
  const int blocks = static_cast<int>(want < 8192 ? want : 8192);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (chunk) {
    case 16: hipLaunchKernelGGL(copy_blocks_kernel<16>, dim3(blocks), dim3(threads), 0, s, a); break;
    case 8:  hipLaunchKernelGGL(copy_blocks_kernel<8>, dim3(blocks), dim3(threads), 0, s, a); break;
    case 4:  hipLaunchKernelGGL(copy_blocks_kernel<4>, dim3(blocks), dim3(threads), 0, s, a); break;
    case 2:  hipLaunchKernelGGL(copy_blocks_kernel<2>, dim3(blocks), dim3(threads), 0, s, a); break;
    default: hipLaunchKernelGGL(copy_blocks_kernel<1>, dim3(blocks), dim3(threads), 0, s, a); break;
  }
  return status_from_hip(hipGetLastError());
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
