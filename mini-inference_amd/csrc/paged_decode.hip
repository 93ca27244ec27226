// Paged decode attention for gfx950 (wave64), GQA, one query token per sequence.
//
// Reference semantics: engine/kv_cache.py:615-620 (gather each sequence's blocks through its
// table, hide keys j > positions[b] with a mask) followed by engine/model.py:126-147
// (decode_attention: query head h uses kv head h // G, G = num_heads / num_kv_heads,
// softmax(q.k * scale) @ v with scale = 1/sqrt(head_dim)).
//
// Design
//   * Grid = (partitions, kv heads, batch). A workgroup of kNW wavefronts owns one
//     (sequence, kv head, partition of part_tokens keys) and computes all G query heads of
//     that kv head, so each K/V row is read from HBM once for the whole GQA group.
//     Workgroups whose partition starts past the sequence's context exit at once; the grid
//     therefore depends only on max_blocks_per_seq (graph-capturable).
//   * Within a workgroup the wavefronts take turns on "passes" of RPP consecutive keys.
//     QK: lane (row r, chunk c) holds CH contiguous elements of key r (32-byte loads) and
//     the matching q slice for all G heads; partial dot products (v_dot2_f32_{bf16,f16} for
//     16-bit data) are summed across the LPR lanes of a row with xor shuffles.
//     PV: probabilities and row indices go through a per-wave LDS slot; the value rows are
//     then read with one dword per lane (a wavefront covers TPI whole rows per load) and
//     accumulated in fp32 for all G heads.
//   * Softmax is online in base 2 with a wave-uniform running max per head that is only
//     raised when some key exceeds it by more than kRescaleLog2 (then all partial sums are
//     rescaled), so most passes need no cross-lane max.
//   * Partials of a multi-partition sequence (running max m, sum l, unnormalised
//     accumulator) go to the workspace; the last workgroup of a (sequence, kv head) to
//     finish (agent-scope counter) merges them and writes the output, then re-arms the
//     counter to zero. One launch does the whole operation.
#include <cstdlib>
#include <cmath>

#include "mip_common.h"

namespace mip {
namespace {

constexpr int kNW = 4;                  // wavefronts per workgroup
constexpr float kRescaleLog2 = 8.0f;    // lazy-rescale threshold, log2 units (p <= 256)
constexpr int kDefaultPartTokens = 512;

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
  int part_tokens;
  int nparts;
  float scale_log2;
  float* ws_acc;  // [B][Hq][nparts][D]
  float* ws_ml;   // [B][Hq][nparts][2]
  int* ws_cnt;    // [B][Hkv]
};

template <int DT, int D, int G>
struct Shape {
  static constexpr int ES = Elem<DT>::kBytes;
  static constexpr int CH = (D < 32 / ES) ? D : 32 / ES;           // key elements per lane
  static constexpr int LPR = D / CH;                                 // lanes per key row
  static constexpr int RPP = kWave / LPR;                            // keys per pass
  static constexpr int KDW = CH * ES / 4;                            // key dwords per lane
  static constexpr int ROWDW = D * ES / 4;                           // dwords per row
  static constexpr int VPL = ROWDW > kWave ? ROWDW / kWave : 1;      // value dwords per lane
  static constexpr int LPT = ROWDW / VPL;                            // lanes per value row
  static constexpr int TPI = kWave / LPT;                            // value rows per load
  static constexpr int VEPL = VPL * 4 / ES;                          // value elements per lane
  static constexpr int GP = (G + 3) & ~3;                            // LDS stride of p rows
  static constexpr int QW = (DT == MIP_F32) ? CH : CH / 2;           // q registers per head
  static constexpr int PASS_ALIGN = kNW * RPP;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int N>
__device__ __forceinline__ void load_dwords(uint32_t (&dst)[N], const char* p) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const uint4 t = reinterpret_cast<const uint4*>(p)[i];
      dst[4 * i] = t.x; dst[4 * i + 1] = t.y; dst[4 * i + 2] = t.z; dst[4 * i + 3] = t.w;
    }
  } else if constexpr (N == 2) {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    dst[0] = t.x; dst[1] = t.y;
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) dst[i] = reinterpret_cast<const uint32_t*>(p)[i];
  }
}

__device__ __forceinline__ float ws_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ws_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT, int D, int G>
__global__ __launch_bounds__(kNW * kWave) void paged_decode_valu(DecodeArgs a) {
  using Sh = Shape<DT, D, G>;
  constexpr int ES = Sh::ES, CH = Sh::CH, LPR = Sh::LPR, RPP = Sh::RPP, KDW = Sh::KDW;
  constexpr int ROWDW = Sh::ROWDW, VPL = Sh::VPL, LPT = Sh::LPT, TPI = Sh::TPI, VEPL = Sh::VEPL;
  constexpr int GP = Sh::GP, QW = Sh::QW;
  using S = typename Elem<DT>::S;

  __shared__ float sh_p[kNW][RPP][GP];
  __shared__ int sh_row[kNW][RPP];
  __shared__ float sh_m[kNW][G];
  __shared__ float sh_l[kNW][G];
  __shared__ float sh_acc[kNW][G][D];
  __shared__ int sh_last;

  const int part = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int h0 = kvh * G;

  int ctx = a.lens[b];
  const int cap = a.max_blocks * a.bs;
  ctx = ctx < cap ? ctx : cap;
  const int np_b = ctx > 0 ? (ctx + a.part_tokens - 1) / a.part_tokens : 1;
  if (part >= np_b) return;

  S* out_base = reinterpret_cast<S*>(a.out);
  if (ctx <= 0) {
    for (int i = tid; i < G * D; i += kNW * kWave) {
      const int g = i / D, d = i % D;
      out_base[b * a.out_sb + (h0 + g) * a.out_sh + d] = from_f32<DT>(0.0f);
    }
    return;
  }
  const int t0 = part * a.part_tokens;
  const int t1 = (t0 + a.part_tokens < ctx) ? t0 + a.part_tokens : ctx;

  // ---- q slice for all G heads of this kv head: lane (r, c) holds elements [c*CH, c*CH+CH).
  const int r = lane / LPR, c = lane % LPR;
  uint32_t qreg[G][QW];
  {
    const char* qb = a.q + (static_cast<int64_t>(b) * a.q_sb + static_cast<int64_t>(c) * CH) * ES;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint32_t* qp = reinterpret_cast<const uint32_t*>(qb + static_cast<int64_t>(h0 + g) * a.q_sh * ES);
#pragma unroll
      for (int i = 0; i < QW; ++i) qreg[g][i] = qp[i];
    }
  }

  float m[G], l[G], acc[G][VEPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEPL; ++e) acc[g][e] = 0.0f;
  }

  const int32_t* table = a.bt + static_cast<int64_t>(b) * a.bt_stride;
  const int ts = lane / LPT, u = lane % LPT;

  for (int base = t0 + w * RPP; base < t1; base += kNW * RPP) {
    // ---- keys: lane (r, c)
    const int tok = base + r;
    bool valid = tok < t1;
    int row = -1;
    if (valid) {
      const int blk = table[tok >> a.log2_bs];
      if (blk >= 0 && blk < a.ncb) {
        row = (blk * a.hkv + kvh) * a.bs + (tok & (a.bs - 1));
      } else {
        valid = false;
      }
    }
    uint32_t kw[KDW];
    if (valid) {
      load_dwords<KDW>(kw, a.k + (static_cast<int64_t>(row) * D + c * CH) * ES);
    } else {
#pragma unroll
      for (int i = 0; i < KDW; ++i) kw[i] = 0u;
    }

    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc_s = 0.0f;
      if constexpr (DT == MIP_F32) {
#pragma unroll
        for (int i = 0; i < KDW; ++i) acc_s = fmaf(__uint_as_float(qreg[g][i]), __uint_as_float(kw[i]), acc_s);
      } else {
#pragma unroll
        for (int i = 0; i < KDW; ++i) acc_s = dot2<DT>(qreg[g][i], kw[i], acc_s);
      }
      s[g] = acc_s;
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) {
#pragma unroll
      for (int g = 0; g < G; ++g) s[g] += __shfl_xor(s[g], o);
    }
    bool need = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s[g] = valid ? s[g] * a.scale_log2 : -INFINITY;
      need |= s[g] > m[g] + kRescaleLog2;
    }
    if (__any(need)) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = s[g];
#pragma unroll
        for (int o = LPR; o < kWave; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float mn = fmaxf(m[g], mx);
        const float alpha = (m[g] == -INFINITY) ? 0.0f : fast_exp2(m[g] - mn);
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < VEPL; ++e) acc[g][e] *= alpha;
        m[g] = mn;
      }
    }
    float p[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      p[g] = valid ? fast_exp2(s[g] - m[g]) : 0.0f;
      l[g] += p[g];
    }
    if (c == 0) {
      sh_row[w][r] = valid ? row : -1;
#pragma unroll
      for (int g = 0; g < GP; ++g) sh_p[w][r][g] = g < G ? p[g] : 0.0f;
    }
    __builtin_amdgcn_wave_barrier();

    // ---- values: lane (ts, u) covers dwords [u*VPL, u*VPL+VPL) of row i*TPI + ts
#pragma unroll
    for (int i = 0; i < RPP / TPI; ++i) {
      const int tl = i * TPI + ts;
      const int vrow = sh_row[w][tl];
      float pv[GP];
#pragma unroll
      for (int g4 = 0; g4 < GP / 4; ++g4) {
        const float4 t = *reinterpret_cast<const float4*>(&sh_p[w][tl][4 * g4]);
        pv[4 * g4] = t.x; pv[4 * g4 + 1] = t.y; pv[4 * g4 + 2] = t.z; pv[4 * g4 + 3] = t.w;
      }
      uint32_t vw[VPL];
      if (vrow >= 0) {
        load_dwords<VPL>(vw, a.v + (static_cast<int64_t>(vrow) * ROWDW + u * VPL) * 4);
      } else {
#pragma unroll
        for (int k2 = 0; k2 < VPL; ++k2) vw[k2] = 0u;
      }
      float vf[VEPL];
#pragma unroll
      for (int k2 = 0; k2 < VPL; ++k2) {
        if constexpr (DT == MIP_F32) {
          vf[k2] = __uint_as_float(vw[k2]);
        } else {
          vf[2 * k2] = lo16<DT>(vw[k2]);
          vf[2 * k2 + 1] = hi16<DT>(vw[k2]);
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < VEPL; ++e) acc[g][e] = fmaf(pv[g], vf[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- wave reduction: l over key rows, acc over value-row slots.
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int o = LPR; o < kWave; o <<= 1) l[g] += __shfl_xor(l[g], o);
#pragma unroll
    for (int o = LPT; o < kWave; o <<= 1) {
#pragma unroll
      for (int e = 0; e < VEPL; ++e) acc[g][e] += __shfl_xor(acc[g][e], o);
    }
  }
  if (lane < LPT) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < VEPL; ++e) sh_acc[w][g][u * VEPL + e] = acc[g][e];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      sh_m[w][g] = m[g];
      sh_l[w][g] = l[g];
    }
  }
  __syncthreads();

  // ---- merge the kNW wavefronts of this workgroup.
  for (int i = tid; i < G * D; i += kNW * kWave) {
    const int g = i / D, d = i % D;
    float mx = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kNW; ++ww) mx = fmaxf(mx, sh_m[ww][g]);
    float A = 0.0f, Ls = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kNW; ++ww) {
      const float mw = sh_m[ww][g];
      const float wt = (mw == -INFINITY) ? 0.0f : fast_exp2(mw - mx);
      A = fmaf(wt, sh_acc[ww][g][d], A);
      Ls = fmaf(wt, sh_l[ww][g], Ls);
    }
    if (np_b == 1) {
      out_base[b * a.out_sb + (h0 + g) * a.out_sh + d] = from_f32<DT>(Ls > 0.0f ? A / Ls : 0.0f);
    } else {
      const int64_t slot = (static_cast<int64_t>(b) * a.hq + h0 + g) * a.nparts + part;
      ws_store(a.ws_acc + slot * D + d, A);
      if (d == 0) {
        ws_store(a.ws_ml + slot * 2, mx);
        ws_store(a.ws_ml + slot * 2 + 1, Ls);
      }
    }
  }
  if (np_b == 1) return;

  // ---- cross-workgroup merge by the last partition to finish.
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(a.ws_cnt + b * a.hkv + kvh, 1);
    sh_last = (prev == np_b - 1);
  }
  __syncthreads();
  if (!sh_last) return;
  __threadfence();
  for (int i = tid; i < G * D; i += kNW * kWave) {
    const int g = i / D, d = i % D;
    const int64_t slot0 = (static_cast<int64_t>(b) * a.hq + h0 + g) * a.nparts;
    float mx = -INFINITY;
    for (int pp = 0; pp < np_b; ++pp) mx = fmaxf(mx, ws_load(a.ws_ml + (slot0 + pp) * 2));
    float A = 0.0f, Ls = 0.0f;
    for (int pp = 0; pp < np_b; ++pp) {
      const float mp = ws_load(a.ws_ml + (slot0 + pp) * 2);
      const float wt = (mp == -INFINITY) ? 0.0f : fast_exp2(mp - mx);
      A = fmaf(wt, ws_load(a.ws_acc + (slot0 + pp) * D + d), A);
      Ls = fmaf(wt, ws_load(a.ws_ml + (slot0 + pp) * 2 + 1), Ls);
    }
    out_base[b * a.out_sb + (h0 + g) * a.out_sh + d] = from_f32<DT>(Ls > 0.0f ? A / Ls : 0.0f);
  }
  if (tid == 0) __hip_atomic_store(a.ws_cnt + b * a.hkv + kvh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ host side

inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

int rows_per_pass(int dtype, int d) {
  const int es = dtype == MIP_F32 ? 4 : 2;
  const int ch = d < 32 / es ? d : 32 / es;
  return kWave / (d / ch);
}

int part_tokens_for(int dtype, int d) {
  const int align = kNW * rows_per_pass(dtype, d);
  int want = kDefaultPartTokens;
  if (const char* env = std::getenv("MIP_PART_TOKENS")) {
    const int v = std::atoi(env);
    if (v > 0) want = v;
  }
  return static_cast<int>(align_up(want, align));
}

struct WsLayout {
  int nparts;
  int64_t cnt_off, ml_off, acc_off, bytes;
};

WsLayout ws_layout(int batch, int hq, int hkv, int d, int bs, int max_blocks, int dtype) {
  WsLayout w{};
  const int pt = part_tokens_for(dtype, d);
  const int64_t max_ctx = static_cast<int64_t>(max_blocks) * bs;
  w.nparts = static_cast<int>((max_ctx + pt - 1) / pt);
  if (w.nparts < 1) w.nparts = 1;
  if (w.nparts == 1) return w;
  w.cnt_off = 0;
  w.ml_off = align_up(static_cast<int64_t>(batch) * hkv * 4, 256);
  w.acc_off = w.ml_off + align_up(static_cast<int64_t>(batch) * hq * w.nparts * 2 * 4, 256);
  w.bytes = w.acc_off + align_up(static_cast<int64_t>(batch) * hq * w.nparts * d * 4, 256);
  return w;
}

using KernelFn = void (*)(DecodeArgs);

template <int DT, int D>
KernelFn pick_g(int g) {
  switch (g) {
    case 1: return paged_decode_valu<DT, D, 1>;
    case 2: return paged_decode_valu<DT, D, 2>;
    case 3: return paged_decode_valu<DT, D, 3>;
    case 4: return paged_decode_valu<DT, D, 4>;
    case 5: return paged_decode_valu<DT, D, 5>;
    case 6: return paged_decode_valu<DT, D, 6>;
    case 7: return paged_decode_valu<DT, D, 7>;
    case 8: return paged_decode_valu<DT, D, 8>;
    default: return nullptr;
  }
}

template <int DT>
KernelFn pick_d(int d, int g) {
  switch (d) {
    case 8: return pick_g<DT, 8>(g);
    case 16: return pick_g<DT, 16>(g);
    case 32: return pick_g<DT, 32>(g);
    case 64: return pick_g<DT, 64>(g);
    case 128: return pick_g<DT, 128>(g);
    case 256: return pick_g<DT, 256>(g);
    default: return nullptr;
  }
}

KernelFn pick_kernel(int dtype, int d, int g) {
  switch (dtype) {
    case MIP_F32: return pick_d<MIP_F32>(d, g);
    case MIP_F16: return pick_d<MIP_F16>(d, g);
    case MIP_BF16: return pick_d<MIP_BF16>(d, g);
    default: return nullptr;
  }
}

}  // namespace
}  // namespace mip

using namespace mip;

extern "C" size_t mip_paged_decode_workspace(int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                             int32_t block_size, int32_t max_blocks_per_seq, int32_t dtype) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0)
    return 0;
  return static_cast<size_t>(
      ws_layout(batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, dtype).bytes);
}

extern "C" int mip_paged_decode(void* out, int64_t out_stride_b, int64_t out_stride_h, const void* q,
                                int64_t q_stride_b, int64_t q_stride_h, const void* k_cache, const void* v_cache,
                                int64_t num_cache_blocks, const int32_t* block_tables, int64_t bt_stride,
                                const int32_t* context_lens, int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq, float scale,
                                void* workspace, size_t workspace_bytes, int32_t dtype, void* stream) {
  if (dtype != MIP_F32 && dtype != MIP_F16 && dtype != MIP_BF16) return MIP_EINVAL;
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return MIP_EINVAL;
  if (num_heads % num_kv_heads != 0) return MIP_EINVAL;
  if (!is_pow2(block_size) || block_size > 4096 || max_blocks_per_seq <= 0 || bt_stride < max_blocks_per_seq)
    return MIP_EINVAL;
  if (num_cache_blocks <= 0 || num_cache_blocks * num_kv_heads * block_size >= (int64_t{1} << 31)) return MIP_EINVAL;
  if (static_cast<int64_t>(max_blocks_per_seq) * block_size >= (int64_t{1} << 30)) return MIP_EINVAL;
  if (batch == 0) return MIP_OK;
  if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens) return MIP_EINVAL;
  if (!std::isfinite(scale)) return MIP_EINVAL;
  const int group = num_heads / num_kv_heads;
  KernelFn fn = pick_kernel(dtype, head_dim, group);
  if (!fn) return MIP_EUNSUPPORTED;
  const int64_t es = dtype == MIP_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15) return MIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(q) | static_cast<uint64_t>(q_stride_b * es) |
       static_cast<uint64_t>(q_stride_h * es)) & 3)
    return MIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(out) | static_cast<uint64_t>(out_stride_b * es) |
       static_cast<uint64_t>(out_stride_h * es)) & (es - 1))
    return MIP_EINVAL;

  const WsLayout wl = ws_layout(batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, dtype);
  DecodeArgs a{};
  if (wl.nparts > 1) {
    if (!workspace || workspace_bytes < static_cast<size_t>(wl.bytes) ||
        (reinterpret_cast<uintptr_t>(workspace) & 255))
      return MIP_EINVAL;
    char* ws = static_cast<char*>(workspace);
    a.ws_cnt = reinterpret_cast<int*>(ws + wl.cnt_off);
    a.ws_ml = reinterpret_cast<float*>(ws + wl.ml_off);
    a.ws_acc = reinterpret_cast<float*>(ws + wl.acc_off);
  }
  a.out = static_cast<char*>(out);
  a.out_sb = out_stride_b;
  a.out_sh = out_stride_h;
  a.q = static_cast<const char*>(q);
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.k = static_cast<const char*>(k_cache);
  a.v = static_cast<const char*>(v_cache);
  a.ncb = num_cache_blocks;
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  a.lens = context_lens;
  a.hq = num_heads;
  a.hkv = num_kv_heads;
  a.bs = block_size;
  a.log2_bs = ilog2_exact(block_size);
  a.max_blocks = max_blocks_per_seq;
  a.part_tokens = part_tokens_for(dtype, head_dim);
  a.nparts = wl.nparts;
  a.scale_log2 = scale * 1.4426950408889634f;
  if (batch > 65535) return MIP_EINVAL;
  hipLaunchKernelGGL(fn, dim3(wl.nparts, num_kv_heads, batch), dim3(kNW * kWave), 0,
                     static_cast<hipStream_t>(stream), a);
  return status_from_hip(hipGetLastError());
}
