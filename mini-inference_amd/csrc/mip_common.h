// Shared device helpers for the paged KV-cache kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mipaged.h"

namespace mip {

constexpr int kWave = 64;

// Element storage per dtype tag. 16-bit types are carried as raw uint16_t bits so that
// append and copy stay pure data movement (bit-exact by construction).
template <int DT> struct Elem;
template <> struct Elem<MIP_F32>  { using S = float;    static constexpr int kBytes = 4; };
template <> struct Elem<MIP_F16>  { using S = uint16_t; static constexpr int kBytes = 2; };
template <> struct Elem<MIP_BF16> { using S = uint16_t; static constexpr int kBytes = 2; };

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// Low / high element of a dword holding two 16-bit values, as fp32.
template <int DT> __device__ __forceinline__ float lo16(uint32_t w);
template <int DT> __device__ __forceinline__ float hi16(uint32_t w);
template <> __device__ __forceinline__ float lo16<MIP_BF16>(uint32_t w) { return bf16_lo(w); }
template <> __device__ __forceinline__ float hi16<MIP_BF16>(uint32_t w) { return bf16_hi(w); }
template <> __device__ __forceinline__ float lo16<MIP_F16>(uint32_t w) { return f16_bits_to_f32(w & 0xffffu); }
template <> __device__ __forceinline__ float hi16<MIP_F16>(uint32_t w) { return f16_bits_to_f32(w >> 16); }

// fp32 -> 16-bit with round-to-nearest-even (the rounding torch's .to(bfloat16/float16) uses).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT> __device__ __forceinline__ typename Elem<DT>::S from_f32(float f);
template <> __device__ __forceinline__ float from_f32<MIP_F32>(float f) { return f; }
template <> __device__ __forceinline__ uint16_t from_f32<MIP_F16>(float f) { return f32_to_f16_rne(f); }
template <> __device__ __forceinline__ uint16_t from_f32<MIP_BF16>(float f) { return f32_to_bf16_rne(f); }

// 2-term dot product of packed 16-bit pairs accumulated in fp32 (v_dot2_f32_{bf16,f16}).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <int DT> __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c);
template <> __device__ __forceinline__ float dot2<MIP_BF16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}
template <> __device__ __forceinline__ float dot2<MIP_F16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
}

// Read a wave-uniform int32 through the constant address space, so it becomes a scalar load
// (its own counter) even in kernels that store to global memory. Only for inputs that no
// kernel writes while it runs (block tables).
__device__ __forceinline__ int load_uniform_i32(const int32_t* p) {
  return *(const __attribute__((address_space(4))) int32_t*)(p);
}

__device__ __forceinline__ int64_t load_uniform_i64(const int64_t* p) {
  return *(const __attribute__((address_space(4))) int64_t*)(p);
}

// A vector load issued where it is written. A relaxed atomic load is not sunk into the branch
// that uses it and not reordered behind another one, so a group of them written back to back
// goes out back to back and costs one memory round trip, however its values are tested
// afterwards. (Plain loads of a prologue were sunk past an early-exit test and issued one
// round trip after another.) The atomic is wavefront-scope: a plain global_load.
__device__ __forceinline__ uint64_t load_now_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

// The two 32-bit halves of a wave-uniform 64-bit value, in scalar registers.
__device__ __forceinline__ int uniform_lo(uint64_t x) {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(x)));
}
__device__ __forceinline__ int uniform_hi(uint64_t x) {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(x >> 32)));
}

__host__ __device__ constexpr int ilog2_exact(int x) { return x <= 1 ? 0 : 1 + ilog2_exact(x >> 1); }

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

inline int status_from_hip(hipError_t e) { return e == hipSuccess ? MIP_OK : static_cast<int>(e); }

}  // namespace mip
