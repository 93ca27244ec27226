// Rotary position embedding of q and k fused with the KV append.
//
// Reference semantics, one decoder layer (engine/model.py:216-224 apply_rope / _rotate_half,
// called at engine/model.py:249, then the scatter of engine/kv_cache.py:613-614 or :286-289):
//     q, k = q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin
//     k_layer[slot // bs, h, slot % bs, :] = k[token, h, :];  same for v
// with rotate_half(x) = cat(-x[D/2:], x[:D/2]). Each torch op rounds to the tensor dtype, so
// element j < D/2 of a row is
//     rnd(rnd(x[j] * cos[j]) + rnd(-x[j + D/2] * sin[j]))
// and element j >= D/2 is
//     rnd(rnd(x[j] * cos[j]) + rnd(x[j - D/2] * sin[j])),
// products and the sum in fp32, rnd = round to nearest even into the dtype (identity for
// fp32). The kernel evaluates exactly that, never contracting a product and the sum into one
// fma (which would skip the product's rounding in fp32), so its q, k and
// pool rows are bit-identical to the torch sequence.
//
// Work split: one lane per (row, chunk) where a row is one (token, head) of q, k or v and a
// chunk is CHUNK bytes of the first half of the row together with the matching CHUNK bytes of
// the second half, so each lane owns both elements of every rotation pair it touches and the
// in-place update of q and k has no hazard. Lanes of a row are adjacent and the rows of a
// token are adjacent, so a wavefront reads and writes whole rows with wide accesses.
#include "mip_common.h"

namespace mip {
namespace {

template <int BYTES> struct Chunk;
template <> struct Chunk<16> { using T = uint4; };
template <> struct Chunk<8>  { using T = uint2; };
template <> struct Chunk<4>  { using T = uint32_t; };
template <> struct Chunk<2>  { using T = uint16_t; };

struct RopeArgs {
  char* q;
  char* k;
  const char* v;
  const char* cos;
  const char* sin;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, cs_st;  // bytes
  char* k_cache;
  char* v_cache;
  const int64_t* slots;
  int64_t n_slots;  // num_cache_blocks * block_size
  int n_tokens, hq, hkv, half_bytes, row_bytes, block_size, log2_bs;
};

template <int DT> __device__ __forceinline__ float widen(typename Elem<DT>::S s);
template <> __device__ __forceinline__ float widen<MIP_F32>(float s) { return s; }
template <> __device__ __forceinline__ float widen<MIP_F16>(uint16_t s) { return f16_bits_to_f32(s); }
template <> __device__ __forceinline__ float widen<MIP_BF16>(uint16_t s) { return __uint_as_float(uint32_t{s} << 16); }

// Round an fp32 value to the dtype and back (the value a torch op on dtype tensors stores).
template <int DT> __device__ __forceinline__ float rnd(float f) { return widen<DT>(from_f32<DT>(f)); }

// fp32 multiply and add that are never contracted into an fma (each rounds on its own, as
// torch's separate elementwise kernels do).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

template <int DT, int CHUNK>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeArgs a) {
  using S = typename Elem<DT>::S;
  using V = typename Chunk<CHUNK>::T;
  constexpr int N = CHUNK / Elem<DT>::kBytes;  // elements per chunk
  static_assert(N >= 1 && N * Elem<DT>::kBytes == CHUNK, "chunk must hold whole elements");
  const uint32_t lanes_row = static_cast<uint32_t>(a.half_bytes / CHUNK);
  const uint32_t rows = static_cast<uint32_t>(a.hq + 2 * a.hkv);
  const uint32_t total = static_cast<uint32_t>(a.n_tokens) * rows * lanes_row;  // < 2^31, host-checked
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const uint32_t c = i % lanes_row;
    const uint32_t tr = i / lanes_row;
    const uint32_t r = tr % rows;
    const int64_t tok = tr / rows;
    const int64_t lo_off = static_cast<int64_t>(c) * CHUNK;
    const int64_t hi_off = lo_off + a.half_bytes;
    const bool is_q = r < static_cast<uint32_t>(a.hq);
    const bool is_v = r >= static_cast<uint32_t>(a.hq + a.hkv);
    const int h = static_cast<int>(is_q ? r : (is_v ? r - a.hq - a.hkv : r - a.hq));
    // The slot is loaded first so its latency overlaps the row loads (k and v rows only).
    const int64_t slot = is_q ? -1 : a.slots[tok];

    V lo, hi;
    char* row = nullptr;
    if (is_v) {
      const char* src = a.v + tok * a.v_st + h * a.v_sh;
      lo = *reinterpret_cast<const V*>(src + lo_off);
      hi = *reinterpret_cast<const V*>(src + hi_off);
    } else {
      row = is_q ? a.q + tok * a.q_st + h * a.q_sh : a.k + tok * a.k_st + h * a.k_sh;
      lo = *reinterpret_cast<const V*>(row + lo_off);
      hi = *reinterpret_cast<const V*>(row + hi_off);
      const char* cs = a.cos + tok * a.cs_st;
      const char* sn = a.sin + tok * a.cs_st;
      const V c_lo = *reinterpret_cast<const V*>(cs + lo_off);
      const V c_hi = *reinterpret_cast<const V*>(cs + hi_off);
      const V s_lo = *reinterpret_cast<const V*>(sn + lo_off);
      const V s_hi = *reinterpret_cast<const V*>(sn + hi_off);
      S xl[N], xh[N], cl[N], ch[N], sl[N], sh[N];
      __builtin_memcpy(xl, &lo, CHUNK);
      __builtin_memcpy(xh, &hi, CHUNK);
      __builtin_memcpy(cl, &c_lo, CHUNK);
      __builtin_memcpy(ch, &c_hi, CHUNK);
      __builtin_memcpy(sl, &s_lo, CHUNK);
      __builtin_memcpy(sh, &s_hi, CHUNK);
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float x0 = widen<DT>(xl[e]);
        const float x1 = widen<DT>(xh[e]);
        const float y0 = add_rn(rnd<DT>(mul_rn(x0, widen<DT>(cl[e]))), rnd<DT>(mul_rn(-x1, widen<DT>(sl[e]))));
        const float y1 = add_rn(rnd<DT>(mul_rn(x1, widen<DT>(ch[e]))), rnd<DT>(mul_rn(x0, widen<DT>(sh[e]))));
        xl[e] = from_f32<DT>(y0);
        xh[e] = from_f32<DT>(y1);
      }
      __builtin_memcpy(&lo, xl, CHUNK);
      __builtin_memcpy(&hi, xh, CHUNK);
      *reinterpret_cast<V*>(row + lo_off) = lo;
      *reinterpret_cast<V*>(row + hi_off) = hi;
    }
    if (slot < 0 || slot >= a.n_slots) continue;  // q row, padding row or invalid slot: no pool write
    const int64_t blk = slot >> a.log2_bs;
    const int64_t off = slot & (a.block_size - 1);
    char* dst = (is_v ? a.v_cache : a.k_cache) + ((blk * a.hkv + h) * a.block_size + off) * a.row_bytes;
    *reinterpret_cast<V*>(dst + lo_off) = lo;
    *reinterpret_cast<V*>(dst + hi_off) = hi;
  }
}

template <int DT>
int launch(const RopeArgs& a, int chunk, int blocks, hipStream_t s) {
  if constexpr (DT == MIP_F32) {
    switch (chunk) {
      case 16: hipLaunchKernelGGL((rope_append_kernel<DT, 16>), dim3(blocks), dim3(256), 0, s, a); break;
      case 8:  hipLaunchKernelGGL((rope_append_kernel<DT, 8>), dim3(blocks), dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL((rope_append_kernel<DT, 4>), dim3(blocks), dim3(256), 0, s, a); break;
    }
  } else {
    switch (chunk) {
      case 16: hipLaunchKernelGGL((rope_append_kernel<DT, 16>), dim3(blocks), dim3(256), 0, s, a); break;
      case 8:  hipLaunchKernelGGL((rope_append_kernel<DT, 8>), dim3(blocks), dim3(256), 0, s, a); break;
      case 4:  hipLaunchKernelGGL((rope_append_kernel<DT, 4>), dim3(blocks), dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL((rope_append_kernel<DT, 2>), dim3(blocks), dim3(256), 0, s, a); break;
    }
  }
  return status_from_hip(hipGetLastError());
}

}  // namespace
}  // namespace mip

using namespace mip;

extern "C" int mip_rope_kv_append(void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                  void* k, int64_t k_stride_tok, int64_t k_stride_head,
                                  const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                                  const void* cos, const void* sin, int64_t cs_stride_tok,
                                  void* k_cache, void* v_cache, int64_t num_cache_blocks,
                                  const int64_t* slot_mapping, int32_t n_tokens, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                  int32_t dtype, void* stream) {
  if (dtype != MIP_F32 && dtype != MIP_F16 && dtype != MIP_BF16) return MIP_EINVAL;
  if (n_tokens < 0 || num_heads < 0 || num_kv_heads <= 0 || num_cache_blocks <= 0) return MIP_EINVAL;
  if (head_dim <= 0 || head_dim % 2 != 0) return MIP_EINVAL;
  if (!is_pow2(block_size) || block_size > 4096) return MIP_EINVAL;
  if (n_tokens == 0) return MIP_OK;
  if ((num_heads > 0 && !q) || !k || !v || !cos || !sin || !k_cache || !v_cache || !slot_mapping) return MIP_EINVAL;
  const int64_t es = dtype == MIP_F32 ? 4 : 2;
  RopeArgs a;
  a.q = static_cast<char*>(q);
  a.k = static_cast<char*>(k);
  a.v = static_cast<const char*>(v);
  a.cos = static_cast<const char*>(cos);
  a.sin = static_cast<const char*>(sin);
  a.q_st = q_stride_tok * es;
  a.q_sh = q_stride_head * es;
  a.k_st = k_stride_tok * es;
  a.k_sh = k_stride_head * es;
  a.v_st = v_stride_tok * es;
  a.v_sh = v_stride_head * es;
  a.cs_st = cs_stride_tok * es;
  a.k_cache = static_cast<char*>(k_cache);
  a.v_cache = static_cast<char*>(v_cache);
  a.slots = slot_mapping;
  a.n_slots = num_cache_blocks * block_size;
  a.n_tokens = n_tokens;
  a.hq = num_heads;
  a.hkv = num_kv_heads;
  a.row_bytes = static_cast<int>(head_dim * es);
  a.half_bytes = a.row_bytes / 2;
  a.block_size = block_size;
  a.log2_bs = ilog2_exact(block_size);

  // Widest chunk that divides the half row, every stride and every base address.
  uint64_t align_bits = static_cast<uint64_t>(a.half_bytes) | static_cast<uint64_t>(a.k_st) |
                        static_cast<uint64_t>(a.k_sh) | static_cast<uint64_t>(a.v_st) |
                        static_cast<uint64_t>(a.v_sh) | static_cast<uint64_t>(a.cs_st) |
                        reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                        reinterpret_cast<uintptr_t>(cos) | reinterpret_cast<uintptr_t>(sin) |
                        reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache);
  if (num_heads > 0)
    align_bits |= static_cast<uint64_t>(a.q_st) | static_cast<uint64_t>(a.q_sh) | reinterpret_cast<uintptr_t>(q);
  int chunk = 16;
  while (chunk > es && (align_bits & (chunk - 1))) chunk >>= 1;
  if (align_bits & (es - 1)) return MIP_EINVAL;  // an address or stride splits an element

  const int64_t total = static_cast<int64_t>(n_tokens) * (num_heads + 2 * num_kv_heads) * (a.half_bytes / chunk);
  if (total >= (int64_t{1} << 31)) return MIP_EINVAL;
  const int64_t blocks64 = (total + 255) / 256;
  const int blocks = static_cast<int>(blocks64 < 65536 ? blocks64 : 65536);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MIP_F32: return launch<MIP_F32>(a, chunk, blocks, s);
    case MIP_F16: return launch<MIP_F16>(a, chunk, blocks, s);
    default:      return launch<MIP_BF16>(a, chunk, blocks, s);
  }
}
