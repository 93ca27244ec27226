// KV append: scatter new K/V rows into the paged pool through a flat slot mapping.
//
// Reference semantics (engine/kv_cache.py:613-614 decode, :286-289 packed prefill):
//     k_layer[slot // bs, h, slot % bs, :] = k_src[token, h, :]      for every token, head
// implemented as pure data movement, so the pool bytes equal the source bytes exactly.
//
// Work split: one lane per CHUNK-byte piece of one (K|V, token, head) row, lanes of a row
// adjacent, rows of a token adjacent: a wavefront reads and writes whole rows with 16-byte
// global_load/store_dwordx4 when the row and every stride allow it.
#include "mip_common.h"

namespace mip {
namespace {

template <int CHUNK> struct ChunkT;
template <> struct ChunkT<16> { using T = uint4; };
template <> struct ChunkT<8>  { using T = uint2; };
template <> struct ChunkT<4>  { using T = uint32_t; };
template <> struct ChunkT<2>  { using T = uint16_t; };

struct AppendArgs {
  const char* k_src;
  const char* v_src;
  int64_t k_st, k_sh, v_st, v_sh;  // bytes
  char* k_cache;
  char* v_cache;
  const int64_t* slots;
  int64_t n_slots;                 // num_cache_blocks * block_size
  int n_tokens, hkv, block_size, row_bytes;
  int log2_bs;
};

// An empty asm that takes a loaded chunk and its slot as operands: both loads are issued
// before it and waited for together.
__device__ __forceinline__ void pin(uint4& v, int64_t& s) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w), "+v"(s));
}
__device__ __forceinline__ void pin(uint2& v, int64_t& s) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(s)); }
__device__ __forceinline__ void pin(uint32_t& v, int64_t& s) { asm volatile("" : "+v"(v), "+v"(s)); }
__device__ __forceinline__ void pin(uint16_t& v, int64_t& s) {
  uint32_t w = v;
  asm volatile("" : "+v"(w), "+v"(s));
  v = static_cast<uint16_t>(w);
}

// The slot list and the source rows come as leading arguments, preloaded into scalar
// registers at wave launch (the build's kernel-argument preloading for this file), and each
// lane reads its source chunk before its slot is tested: the source does not depend on the
// slot, so the slot and the row arrive in the same memory round trip and only the store waits
// for both.
template <int CHUNK>
__global__ __launch_bounds__(256) void kv_append_kernel(const int64_t* __restrict__ slots,
                                                        const char* __restrict__ k_src,
                                                        const char* __restrict__ v_src, AppendArgs a) {
  using V = typename ChunkT<CHUNK>::T;
  const uint32_t cpr = static_cast<uint32_t>(a.row_bytes / CHUNK);  // chunks per (token, head) row
  const uint32_t per_side = static_cast<uint32_t>(a.n_tokens) * a.hkv * cpr;
  const uint32_t total = 2u * per_side;  // < 2^31, checked on the host
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const bool is_v = i >= per_side;
    const uint32_t j = is_v ? i - per_side : i;
    const uint32_t c = j % cpr;
    const uint32_t th = j / cpr;
    const uint32_t h = th % static_cast<uint32_t>(a.hkv);
    const int64_t tok = th / static_cast<uint32_t>(a.hkv);
    const char* src = (is_v ? v_src + tok * a.v_st + h * a.v_sh : k_src + tok * a.k_st + h * a.k_sh) +
                      static_cast<int64_t>(c) * CHUNK;
    V val = *reinterpret_cast<const V*>(src);
    int64_t slot = slots[tok];
    // Both values pass through an empty asm before the slot is tested: the compiler issues
    // both loads and waits once, instead of sinking the source load into the store's branch
    // (its only use) and reading it one round trip after the slot.
    pin(val, slot);
    if (slot < 0 || slot >= a.n_slots) continue;  // padding row or invalid slot: no write
    const int64_t blk = slot >> a.log2_bs;
    const int64_t off = slot & (a.block_size - 1);
    const int64_t dst_row = (blk * a.hkv + h) * a.block_size + off;
    char* dst = (is_v ? a.v_cache : a.k_cache) + dst_row * a.row_bytes + static_cast<int64_t>(c) * CHUNK;
    *reinterpret_cast<V*>(dst) = val;
  }
}

}  // namespace
}  // namespace mip

using namespace mip;

extern "C" int mip_kv_append(const void* k_src, const void* v_src, int64_t k_stride_tok, int64_t k_stride_head,
                             int64_t v_stride_tok, int64_t v_stride_head, void* k_cache, void* v_cache,
                             int64_t num_cache_blocks, const int64_t* slot_mapping, int32_t n_tokens,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t dtype,
                             void* stream) {
  if (dtype != MIP_F32 && dtype != MIP_F16 && dtype != MIP_BF16) return MIP_EINVAL;
  if (n_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_cache_blocks <= 0) return MIP_EINVAL;
  if (!is_pow2(block_size) || block_size > 4096) return MIP_EINVAL;
  if (n_tokens == 0) return MIP_OK;
  if (!k_src || !v_src || !k_cache || !v_cache || !slot_mapping) return MIP_EINVAL;
  const int64_t es = dtype == MIP_F32 ? 4 : 2;
  AppendArgs a;
  a.k_src = static_cast<const char*>(k_src);
  a.v_src = static_cast<const char*>(v_src);
  a.k_st = k_stride_tok * es;
  a.k_sh = k_stride_head * es;
  a.v_st = v_stride_tok * es;
  a.v_sh = v_stride_head * es;
  a.k_cache = static_cast<char*>(k_cache);
  a.v_cache = static_cast<char*>(v_cache);
  a.slots = slot_mapping;
  a.n_slots = num_cache_blocks * block_size;
  a.n_tokens = n_tokens;
  a.hkv = num_kv_heads;
  a.block_size = block_size;
  a.log2_bs = ilog2_exact(block_size);
  a.row_bytes = static_cast<int>(head_dim * es);

  // Widest chunk that divides the row, every stride and every base address.
  uint64_t align_bits = static_cast<uint64_t>(a.row_bytes) | static_cast<uint64_t>(a.k_st) |
                        static_cast<uint64_t>(a.k_sh) | static_cast<uint64_t>(a.v_st) |
                        static_cast<uint64_t>(a.v_sh) | reinterpret_cast<uintptr_t>(k_src) |
                        reinterpret_cast<uintptr_t>(v_src) | reinterpret_cast<uintptr_t>(k_cache) |
                        reinterpret_cast<uintptr_t>(v_cache);
  int chunk = 16;
  while (chunk > 2 && (align_bits & (chunk - 1))) chunk >>= 1;
  if (align_bits & 1) return MIP_EINVAL;

  const int64_t total = 2LL * n_tokens * num_kv_heads * (a.row_bytes / chunk);
  if (total >= (int64_t{1} << 31)) return MIP_EINVAL;
  const int threads = 256;
  const int64_t blocks64 = (total + threads - 1) / threads;
  const int blocks = static_cast<int>(blocks64 < 65536 ? blocks64 : 65536);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (chunk) {
    case 16: hipLaunchKernelGGL(kv_append_kernel<16>, dim3(blocks), dim3(threads), 0, s, a.slots, a.k_src, a.v_src, a); break;
    case 8:  hipLaunchKernelGGL(kv_append_kernel<8>, dim3(blocks), dim3(threads), 0, s, a.slots, a.k_src, a.v_src, a); break;
    case 4:  hipLaunchKernelGGL(kv_append_kernel<4>, dim3(blocks), dim3(threads), 0, s, a.slots, a.k_src, a.v_src, a); break;
    default: hipLaunchKernelGGL(kv_append_kernel<2>, dim3(blocks), dim3(threads), 0, s, a.slots, a.k_src, a.v_src, a); break;
  }
  return status_from_hip(hipGetLastError());
}
