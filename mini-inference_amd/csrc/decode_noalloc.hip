// mip_paged_decode_append_noalloc: the fused append + decode call with its scratch memory in a
// static device array of this library instead of a caller-provided workspace, for callers that
// cannot allocate device memory (code under HIP graph capture, serving loops or harnesses that
// forbid hipMalloc). No reference counterpart.
//
// The array `scratch` holds kNoAllocScratchBytes on every device the library runs on, for the
// life of the process. Its device address is looked up once per device (hipGetSymbolAddress,
// with that device current) and kept; the host-side name `scratch` is never passed to a kernel
// or a copy. Every call on one device shares that device's array and leaves its contents
// undefined (the decode kernels need no initialised scratch), so calls that can overlap on one
// device (different streams, concurrent host threads) race; calls ordered on one stream do not.
#include <mutex>

#include "mip_common.h"

namespace mip {
namespace {

constexpr size_t kNoAllocScratchBytes = MIP_NOALLOC_SCRATCH_BYTES;  // 32 MiB per device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on device `dev` (the current device); nullptr on failure.
void* scratch_on(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace mip

extern "C" int mip_paged_decode_append_noalloc(const void* k_new, const void* v_new, int64_t k_stride_tok,
                                               int64_t k_stride_head, int64_t v_stride_tok, int64_t v_stride_head,
                                               const int64_t* slot_mapping, void* out, int64_t out_stride_b,
                                               int64_t out_stride_h, const void* q, int64_t q_stride_b,
                                               int64_t q_stride_h, void* k_cache, void* v_cache,
                                               int64_t num_cache_blocks, const int32_t* block_tables,
                                               int64_t bt_stride, const int32_t* context_lens, int32_t batch,
                                               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                               int32_t block_size, int32_t max_blocks_per_seq, float scale,
                                               const void* plan, size_t plan_bytes, int32_t dtype, void* stream) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0)
    return MIP_EINVAL;
  if (batch == 0) return MIP_OK;
  const size_t need = mip_paged_decode_workspace(batch, num_heads, num_kv_heads, head_dim, block_size,
                                                 max_blocks_per_seq, dtype);
  if (need > mip::kNoAllocScratchBytes) return MIP_E2BIG;
  void* ws = nullptr;
  if (need > 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= mip::kMaxDevices) return MIP_EINVAL;
    ws = mip::scratch_on(dev);
    if (!ws) return MIP_EINVAL;
  }
  return mip_paged_decode_append(k_new, v_new, k_stride_tok, k_stride_head, v_stride_tok, v_stride_head, slot_mapping,
                                 out, out_stride_b, out_stride_h, q, q_stride_b, q_stride_h, k_cache, v_cache,
                                 num_cache_blocks, block_tables, bt_stride, context_lens, batch, num_heads,
                                 num_kv_heads, head_dim, block_size, max_blocks_per_seq, scale, ws,
                                 ws ? mip::kNoAllocScratchBytes : 0, plan, plan_bytes, dtype, stream);
}
