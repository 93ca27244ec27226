// Definitions shared by the paged decode-attention kernels (partition and stream-K).
#pragma once

#include <cmath>

#include "mip_common.h"

namespace mip {
namespace decode {

constexpr int kNW = 4;                  // wavefronts per workgroup
constexpr float kRescaleLog2 = 8.0f;    // lazy-rescale threshold, log2 units (p <= 256)

struct DecodeArgs {
  char* out;
  int64_t out_sb, out_sh;  // elements
  const char* q;
  int64_t q_sb, q_sh;      // elements
  const char* k;
  const char* v;
  int64_t ncb;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* lens;
  int hq, hkv, bs, log2_bs, max_blocks;
  // VALU kernel: workgroups per kv head (0 or 1: one). With gsplit > 1 workgroup y of the grid
  // reads kv head y / gsplit and serves query heads kvh * group + (y % gsplit) * G .. + G - 1
  // of its group of `group` heads; the last workgroup of a group masks the heads past its end
  // (G = ceil(group / gsplit), so the split need not divide the group).
  int gsplit;
  int group;
  int part_tokens;
  int nparts;
  float scale_log2;
  float* ws_acc;  // [B][Hq][nparts][D]
  float* ws_ml;   // [B][Hq][nparts][2]
  // Packed prefill rows (cu_q != nullptr, VALU kernel only): workgroup x of the grid
  // (num_seqs * max_q_len, kv heads) is new token i = x % max_q_len of sequence s =
  // x / max_q_len, packed row cu_q[s] + i (absent past cu_q[s + 1]); it attends keys
  // 0 .. ctx_start[s] + i through table row s. One partition per row (no merge).
  const int32_t* cu_q;
  const int32_t* ctx_start;
  int max_q_len;
};

// The step's new K/V rows, appended by the stream kernel itself (mip_paged_decode_append).
// slots == nullptr: no append.
struct AppendRows {
  const char* k;               // row (b, h) at k + b * k_st + h * k_sh (bytes), head_dim elements
  const char* v;
  int32_t k_st, k_sh, v_st, v_sh;
  const int64_t* slots;        // [batch] flat pool slot of sequence b's new token
  char* k_cache;               // the pool (same as DecodeArgs k / v, writable)
  char* v_cache;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v_t __attribute__((ext_vector_type(2)));

template <int DT> struct MfmaOps;
template <> struct MfmaOps<MIP_BF16> {
  static __device__ __forceinline__ f32x4_t qk(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t pv(uint2 a, uint2 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b),
                                                     c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t round16(float x) { return f32_to_bf16_rne(x); }
  static __device__ __forceinline__ float widen16(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
  // Two floats -> packed pair (x in the low half), round to nearest even (v_cvt_pk_bf16_f32).
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{x, y}), bf16x2v_t));
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};
template <> struct MfmaOps<MIP_F16> {
  static __device__ __forceinline__ f32x4_t qk(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t pv(uint2 a, uint2 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a), __builtin_bit_cast(f16x4_t, b), c,
                                                 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t round16(float x) { return f32_to_f16_rne(x); }
  static __device__ __forceinline__ float widen16(uint16_t h) { return f16_bits_to_f32(h); }
  // Two floats -> packed pair (x in the low half), round to nearest even (v_cvt_pk_f16_f32).
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{x, y}), f16x2v_t));
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return f16_bits_to_f32(w & 0xffffu); }
  static __device__ __forceinline__ float hi(uint32_t w) { return f16_bits_to_f32(w >> 16); }
};

struct StreamArgs {
  DecodeArgs a;
  int batch;
  int group;
  int tw;          // wavefronts in the grid
  int min_tiles;   // fewest tiles an active wavefront takes
  int max_pieces;  // most wavefronts per segment, on average (caps W at segments * max_pieces)
  // The records sit next to the fields the merge kernel reads first (batch, tw), in the same
  // 64-byte line of the kernel arguments, so reading them costs no further argument load.
  int rec_stride;  // floats per record: m[16] | l[16] | acc[group][D]
  float* ws_rec;   // [tw][2][rec_stride]
  AppendRows app;
  const int32_t* plan;  // stream work plan for these context lengths (nullptr: derive it in-kernel)
  // 32-bit copies of the 64-bit strides / sizes of DecodeArgs (the host checks they fit), so
  // the stream kernel's loop state stays within the scalar register file.
  int32_t q_sb, q_sh, out_sb, out_sh, bt_stride, ncb;
  uint32_t nrows;  // rows of one layer's pool (num_cache_blocks * kv heads * block size)
  int32_t plan_seg_off, plan_tile_off;  // word offsets of the plan's segment records / tile descriptors
  int32_t plan_wave_cap;                // descriptor slots per wavefront in the plan
  int* ws_prefix;  // [batch + 1] tile prefix over sequences (written by workgroup 0)
  // Calls with few segments: the merge cuts a segment of many pieces into `parts` runs (one
  // workgroup each) and leaves their states here, [batch * kv heads][parts][rec_stride], for
  // the fold kernel. parts = 1: the merge combines every segment whole.
  float* ws_part;
  int parts;
};

template <int D>
struct SShape {
  static constexpr int KC = D / 32;
  static constexpr int MT = D / 16;
  static constexpr int TILE_BYTES = 16 * D * 2;
};

// Layout of a stream work plan (int32 words), written once per step by the plan kernel
// (block size >= 16 only):
//   header [kPlanHeader]: T total tiles, W active wavefronts, batch, kv heads, word offset of
//     the tile descriptors, word offset of the segment records, C descriptor slots per
//     wavefront, 0;
//   tw wavefront records of kPlanWave words (the first W written): lo, hi (global tile range);
//   batch * kv heads segment records of kPlanSeg words: g_lo (first wavefront holding a piece),
//     R (pieces), lo_split (the first piece sits in that wavefront's "last segment" slot), L;
//   tw * C + kWave tile descriptor slots of 2 words (8-byte aligned), wavefront-major: tile x
//     of wavefront g's range [lo, hi) sits in slot g * C + (x - lo), so a wavefront finds its
//     first descriptors without reading lo first; C >= hi - lo for every wavefront, and the
//     kWave spare slots keep a wavefront's 64-slot window inside the plan. A descriptor is
//     the pool row of the tile's first key, (block * kv heads + kv head) * block size + offset
//     (0xffffffff for a block id outside the pool), and meta = b | kv head << 16 |
//     valid keys << 24 | first << 29 | last << 30 (first / last: tile 0 / the last tile of its
//     segment).
constexpr int kPlanHeader = 8;
constexpr int kPlanWave = 2;
constexpr int kPlanSeg = 4;
constexpr int kPlanTileOffWord = 4;
constexpr int kPlanSegOffWord = 5;
constexpr int kPlanWaveCapWord = 6;
constexpr uint32_t kTileNoRow = 0xffffffffu;

__device__ __forceinline__ int wave_inclusive_scan(int x, int lane) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  return x;
}

// Active wavefronts W of the stream split: at most the grid's tw, at least min_tiles tiles
// each, and at most max_pieces per segment on average, so that a few long sequences are not
// cut into hundreds of pieces each (the merge combines a segment's pieces serially).
__device__ __forceinline__ int stream_active_waves(int tw, int total_tiles, int min_tiles, int64_t segments,
                                                   int max_pieces) {
  const int want = (total_tiles + min_tiles - 1) / min_tiles;
  int w = want < tw ? want : tw;
  const int64_t cap = segments * max_pieces;
  if (cap < w) w = static_cast<int>(cap);
  return w > 0 ? w : 1;
}

// Launch the stream-K kernel and its merge (paged_decode_stream.hip). grid = workgroups;
// returns 0 or a hipError_t.
struct StreamConfig {
  bool ok;          // a stream kernel exists for this (dtype, head_dim, group)
  int grid;         // workgroups of the persistent grid (device capacity)
  int tw;           // wavefronts in the grid
  int lds_bytes;    // dynamic LDS per workgroup
  int64_t rec_floats;
};
StreamConfig stream_config(int dtype, int d, int group, int batch);
// Floats of second-level merge records a call of this shape needs (0: it merges in one pass).
int64_t stream_part_floats(const StreamConfig& cfg, int batch, int num_kv_heads);
int stream_launch(const StreamConfig& cfg, const StreamArgs& sa, int dtype, int d, int group, int num_kv_heads,
                  int batch, hipStream_t stream);
// Bytes of a work plan for this launch shape (0: no plan, block size < 16), and the plan kernel.
int64_t stream_plan_bytes(const StreamConfig& cfg, int batch, int num_kv_heads, int block_size, int max_blocks);
// Word offsets of a plan's segment records and tile descriptors, and its descriptor slots per
// wavefront (the same the plan kernel writes).
void stream_plan_offsets(const StreamConfig& cfg, int batch, int num_kv_heads, int block_size, int max_blocks,
                         int32_t* seg_off, int32_t* tile_off, int32_t* wave_cap);
int stream_plan_launch(const StreamConfig& cfg, const int32_t* lens, const int32_t* block_tables, int64_t bt_stride,
                       int batch, int num_kv_heads, int block_size, int max_blocks, int32_t* plan, hipStream_t stream);

// Tuning knobs of the stream split, read from the environment once per process
// (MIP_STREAM_MIN_TILES, MIP_STREAM_MAX_PIECES; 0 = the built-in choice).
int stream_min_tiles();
int stream_max_pieces_env();

// Packed prefill attention on the VALU decode kernel (paged_decode.hip), for the shapes the
// MFMA prefill kernel does not cover: fp32, head sizes other than 64 / 128 (8 .. 256, powers
// of two), up to 8 query heads per kv head. Arguments as mip_paged_prefill, checked there.
int valu_prefill_launch(void* out, int64_t out_stride_tok, int64_t out_stride_head, const void* q,
                        int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache, const void* v_cache,
                        int64_t num_cache_blocks, const int32_t* block_tables, int64_t bt_stride, const int32_t* cu_q,
                        const int32_t* ctx_start, int32_t num_seqs, int32_t max_q_len, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                        float scale, int32_t dtype, hipStream_t stream);

}  // namespace decode
}  // namespace mip
