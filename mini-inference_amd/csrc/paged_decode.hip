// Paged decode attention for gfx950 (wave64), GQA, one query token per sequence.
//
// Reference semantics: engine/kv_cache.py:615-620 (gather each sequence's blocks through its
// table, hide keys j > positions[b] with a mask) followed by engine/model.py:126-147
// (decode_attention: query head h uses kv head h // G, G = num_heads / num_kv_heads,
// softmax(q.k * scale) @ v with scale = 1/sqrt(head_dim)).
//
// Design
//   * Two launches. The partition kernel's grid is (partitions, kv heads, batch): a
//     workgroup of kNW wavefronts owns one (sequence, kv head, partition of part_tokens
//     keys) and computes all G query heads of that kv head, so each K/V row is read from HBM
//     once for the whole GQA group. Workgroups whose partition starts past the sequence's
//     context exit at once, so the grid depends only on max_blocks_per_seq
//     (graph-capturable). A sequence that fits one partition is finished by that
//     workgroup; otherwise each partition writes (running max m, sum l, unnormalised
//     accumulator) to the workspace and the merge kernel, grid (kv heads, batch), combines
//     them. The kernel boundary orders the two, so no device-scope fence (an L2 writeback
//     on this chip) is needed inside a kernel.
//   * Within a workgroup the wavefronts take turns on "passes" of RPP consecutive keys,
//     and each wavefront keeps the next pass's K and V loads in flight while it computes
//     the current one (two register fragments, ping-pong, no copies).
//     QK: lane (row r, chunk c) holds CH contiguous elements of key r (32-byte loads) and
//     the matching q slice for all G heads; partial dot products (v_dot2_f32_{bf16,f16} for
//     16-bit data) are summed across the LPR lanes of a row with xor shuffles.
//     PV: lane (slot ts, dword u) loads dword u of value rows i*TPI + ts straight from the
//     pool (a wavefront covers TPI whole rows per load); the probabilities of those rows
//     come through a per-wavefront LDS slot; accumulation is fp32 for all G heads.
//   * When a block holds a whole pass (block_size >= RPP) the pass's block id is one scalar
//     load; otherwise each lane looks its rows up in the table.
//   * Softmax is online in base 2 with a wave-uniform running max per head that is only
//     raised when some key exceeds it by more than kRescaleLog2 (then the partial sums are
//     rescaled), so most passes need no cross-lane max.
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "paged_decode_common.h"

namespace mip {
namespace {

using namespace decode;

constexpr int kDefaultPartTokens = 256;

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
  static constexpr int NV = RPP / TPI;                               // value loads per pass
  static constexpr int VEPL = VPL * 4 / ES;                          // value elements per lane
  static constexpr int GP = (G + 3) & ~3;                            // LDS stride of p rows
  static constexpr int QW = (DT == MIP_F32) ? CH : CH / 2;           // q registers per head
};

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

// One pass worth of this lane's K/V data (in flight while the previous pass is computed).
template <int KDW, int NV, int VPL>
struct PassFrag {
  uint32_t kw[KDW];
  uint32_t vw[NV][VPL];
  bool kvalid;      // this lane's key row is a key of the partition
  uint32_t vmask;   // bit i: value row i of this lane is a key of the partition
};

template <int DT, int D, int G>
struct Pass {
  using Sh = Shape<DT, D, G>;
  using Frag = PassFrag<Sh::KDW, Sh::NV, Sh::VPL>;

  // Issue the loads of the pass starting at key `base` (< t1). Rows past t1 are clamped to
  // the pass's first row (always a key) and flagged invalid; a block id outside the pool
  // reads block 0 and is flagged invalid, so every address stays inside the pool.
  static __device__ __forceinline__ void load(Frag& f, const DecodeArgs& a, const int32_t* table, int kvh, int base,
                                              int t1, int r, int c, int ts, int u) {
    constexpr int ES = Sh::ES, CH = Sh::CH, RPP = Sh::RPP, KDW = Sh::KDW, ROWDW = Sh::ROWDW;
    constexpr int VPL = Sh::VPL, TPI = Sh::TPI, NV = Sh::NV;
    f.vmask = 0u;
    if (a.bs >= RPP) {
      const int blk = load_uniform_i32(table + (base >> a.log2_bs));
      const bool bok = blk >= 0 && blk < a.ncb;
      const int row0 = ((bok ? blk : 0) * a.hkv + kvh) * a.bs + (base & (a.bs - 1));
      const bool kin = base + r < t1;
      f.kvalid = bok && kin;
      load_dwords<KDW>(f.kw, a.k + (static_cast<int64_t>(row0 + (kin ? r : 0)) * D + c * CH) * ES);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int tl = i * TPI + ts;
        const bool vin = base + tl < t1;
        f.vmask |= static_cast<uint32_t>(bok && vin) << i;
        load_dwords<VPL>(f.vw[i], a.v + (static_cast<int64_t>(row0 + (vin ? tl : 0)) * ROWDW + u * VPL) * 4);
      }
    } else {
      {
        const int tok = base + r < t1 ? base + r : base;
        const int blk = table[tok >> a.log2_bs];
        const bool bok = blk >= 0 && blk < a.ncb;
        f.kvalid = bok && (base + r < t1);
        const int row = ((bok ? blk : 0) * a.hkv + kvh) * a.bs + (tok & (a.bs - 1));
        load_dwords<KDW>(f.kw, a.k + (static_cast<int64_t>(row) * D + c * CH) * ES);
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int tl = i * TPI + ts;
        const int tok = base + tl < t1 ? base + tl : base;
        const int blk = table[tok >> a.log2_bs];
        const bool bok = blk >= 0 && blk < a.ncb;
        f.vmask |= static_cast<uint32_t>(bok && (base + tl < t1)) << i;
        const int row = ((bok ? blk : 0) * a.hkv + kvh) * a.bs + (tok & (a.bs - 1));
        load_dwords<VPL>(f.vw[i], a.v + (static_cast<int64_t>(row) * ROWDW + u * VPL) * 4);
      }
    }
  }
};

template <int DT, int D, int G>
__global__ __launch_bounds__(kNW * kWave) void paged_decode_part(DecodeArgs a) {
  using Sh = Shape<DT, D, G>;
  using P = Pass<DT, D, G>;
  using Frag = typename P::Frag;
  constexpr int ES = Sh::ES, CH = Sh::CH, LPR = Sh::LPR, RPP = Sh::RPP, KDW = Sh::KDW;
  constexpr int VPL = Sh::VPL, LPT = Sh::LPT, TPI = Sh::TPI, NV = Sh::NV, VEPL = Sh::VEPL;
  constexpr int GP = Sh::GP, QW = Sh::QW;
  using S = typename Elem<DT>::S;

  __shared__ float sh_p[kNW][RPP][GP];
  __shared__ float sh_m[kNW][G];
  __shared__ float sh_l[kNW][G];
  __shared__ float sh_acc[kNW][G][D];

  // Query heads h0 .. h0 + nh - 1 of kv head kvh (a group of more than 8 heads is split over
  // a.gsplit workgroups, each holding G of them in registers; the last one of a group holds
  // nh <= G live heads, and its other register slots shadow head h0, whose results it drops).
  const int y = static_cast<int>(blockIdx.y);
  const int kvh = a.gsplit > 1 ? y / a.gsplit : y;
  const int h0 = a.gsplit > 1 ? kvh * a.group + (y - kvh * a.gsplit) * G : y * G;
  const int nh = a.gsplit > 1 ? min(G, a.group - (y - kvh * a.gsplit) * G) : G;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);

  // Decode: (partition, kv head, sequence). Packed prefill: (sequence x new token, kv head),
  // one partition; the row's keys are its sequence's keys up to its own position.
  int part, b, ctx, trow;
  if (a.cu_q) {
    const int x = blockIdx.x, s = x / a.max_q_len, i = x - s * a.max_q_len;
    const int r0 = a.cu_q[s];
    if (r0 + i >= a.cu_q[s + 1]) return;
    part = 0;
    b = r0 + i;
    trow = s;
    ctx = a.ctx_start[s] + i + 1;
  } else {
    part = blockIdx.x;
    b = blockIdx.z;
    trow = b;
    ctx = a.lens[b];
  }
  const int cap = a.max_blocks * a.bs;
  ctx = ctx < cap ? ctx : cap;
  const int np_b = ctx > 0 ? (ctx + a.part_tokens - 1) / a.part_tokens : 1;
  if (part >= np_b) return;

  S* out_base = reinterpret_cast<S*>(a.out);
  if (ctx <= 0) {
    for (int i = tid; i < nh * D; i += kNW * kWave) {
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
      const int hg = h0 + (g < nh ? g : 0);
      const uint32_t* qp = reinterpret_cast<const uint32_t*>(qb + static_cast<int64_t>(hg) * a.q_sh * ES);
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

  const int32_t* table = a.bt + static_cast<int64_t>(trow) * a.bt_stride;
  const int ts = lane / LPT, u = lane % LPT;

  auto compute = [&](const Frag& f) {
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc_s = 0.0f;
      if constexpr (DT == MIP_F32) {
#pragma unroll
        for (int i = 0; i < KDW; ++i) acc_s = fmaf(__uint_as_float(qreg[g][i]), __uint_as_float(f.kw[i]), acc_s);
      } else {
#pragma unroll
        for (int i = 0; i < KDW; ++i) acc_s = dot2<DT>(qreg[g][i], f.kw[i], acc_s);
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
      s[g] = f.kvalid ? s[g] * a.scale_log2 : -INFINITY;
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
      p[g] = f.kvalid ? fast_exp2(s[g] - m[g]) : 0.0f;
      l[g] += p[g];
    }
    if (c == 0) {
#pragma unroll
      for (int g = 0; g < GP; ++g) sh_p[w][r][g] = g < G ? p[g] : 0.0f;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int tl = i * TPI + ts;
      float pv[GP];
#pragma unroll
      for (int g4 = 0; g4 < GP / 4; ++g4) {
        const float4 t = *reinterpret_cast<const float4*>(&sh_p[w][tl][4 * g4]);
        pv[4 * g4] = t.x; pv[4 * g4 + 1] = t.y; pv[4 * g4 + 2] = t.z; pv[4 * g4 + 3] = t.w;
      }
      const bool ok = (f.vmask >> i) & 1u;
      float vf[VEPL];
#pragma unroll
      for (int k2 = 0; k2 < VPL; ++k2) {
        const uint32_t wv = ok ? f.vw[i][k2] : 0u;
        if constexpr (DT == MIP_F32) {
          vf[k2] = __uint_as_float(wv);
        } else {
          vf[2 * k2] = lo16<DT>(wv);
          vf[2 * k2 + 1] = hi16<DT>(wv);
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < VEPL; ++e) acc[g][e] = fmaf(pv[g], vf[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- software-pipelined pass loop: fragment A/B ping-pong. The next pass is always
  // loaded (past the end it re-reads the current pass, which stays inside the partition),
  // so the number of loads in flight is the same on every path and the compiler waits only
  // for the fragment being computed.
  constexpr int kStep = kNW * RPP;
  int base = t0 + w * RPP;
  if (base < t1) {
    Frag fa, fb;
    P::load(fa, a, table, kvh, base, t1, r, c, ts, u);
    while (true) {
      int nb = base + kStep;
      P::load(fb, a, table, kvh, nb < t1 ? nb : base, t1, r, c, ts, u);
      compute(fa);
      base = nb;
      if (base >= t1) break;
      nb = base + kStep;
      P::load(fa, a, table, kvh, nb < t1 ? nb : base, t1, r, c, ts, u);
      compute(fb);
      base = nb;
      if (base >= t1) break;
    }
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

  // ---- merge the kNW wavefronts; finish the sequence or hand the partition to the merge kernel.
  for (int i = tid; i < nh * D; i += kNW * kWave) {
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
      a.ws_acc[slot * D + d] = A;
      if (d == 0) {
        a.ws_ml[slot * 2] = mx;
        a.ws_ml[slot * 2 + 1] = Ls;
      }
    }
  }
}

// ---------------------------------------------------------------- MFMA partition kernel
//
// For 16-bit K/V with head_dim 64 or 128 and up to 16 query heads per kv head. Same grid,
// partitions, workspace and merge kernel as the VALU kernel; the inner tile is different.
// A tile is 16 consecutive keys of one wavefront:
//   S^T[16 keys x 16 heads] = K[16 x D] . Q^T[D x 16]       v_mfma_f32_16x16x32_{bf16,f16}
//       A = key rows as loaded (lane l: key l%16, dims 8*(l/16)+32*kc .. +7, one 16-byte load),
//       B = q (lane l: head l%16, same dims), zero for heads >= G;
//       out: lane l holds keys 4*(l/16)+i (i = 0..3) of head l%16.
//   O^T[D x 16 heads] += V^T[D x 16 keys] . P^T[16 keys x 16 heads]   v_mfma_f32_16x16x16_*
//       B = P^T is exactly the S^T output layout, so probabilities stay in registers;
//       A = V^T: lane l needs keys 4*(l/16)+i at dim l%16 (+16 per M-tile), read from a
//       per-wavefront LDS copy of the value tile (written from the 16-byte row loads);
//       P is split into hi + lo 16-bit parts (two MFMAs) so PV keeps ~fp32 precision.
// Every (dim, head) accumulator lives in exactly one lane, and a lane only ever rescales
// its own head, so the running max/sum need no cross-lane traffic except on a rescale.

template <int D>
struct MShape {
  static constexpr int KC = D / 32;                 // 16-byte loads per lane per tile row, QK K-steps
  static constexpr int MT = D / 16;                 // O^T M-tiles
  static constexpr int TPW = D <= 64 ? 2 : 1;       // tiles per pass (8 KB of K+V per pass in flight)
  static constexpr int PASS = 16 * TPW;             // keys per pass
  static constexpr int TILE_BYTES = 16 * D * 2;
};

template <int D>
struct MFrag {
  uint4 k[MShape<D>::TPW][MShape<D>::KC];
  uint4 v[MShape<D>::TPW][MShape<D>::KC];
  uint32_t rowok;  // bit t: this lane's row (key l%16) of tile t is a key of the partition
};

// Load one pass (TPW tiles) starting at key `base` (< t1). Lane l loads key row l%16 of each
// tile; rows past t1 re-read the tile's first key, rows of an invalid block id read block 0,
// so every address stays inside the pool; both are flagged in rowok.
template <int D>
__device__ __forceinline__ void mfma_load_rows(MFrag<D>& f, const DecodeArgs& a, int t, int64_t row, int grp) {
  const char* kp = a.k + row * (D * 2) + 16 * grp;
  const char* vp = a.v + row * (D * 2) + 16 * grp;
#pragma unroll
  for (int kc = 0; kc < MShape<D>::KC; ++kc) {
    f.k[t][kc] = *reinterpret_cast<const uint4*>(kp + 64 * kc);
    f.v[t][kc] = *reinterpret_cast<const uint4*>(vp + 64 * kc);
  }
}

template <int D>
__device__ __forceinline__ void mfma_load(MFrag<D>& f, const DecodeArgs& a, const int32_t* table, int kvh, int base,
                                          int t1, int i16, int grp) {
  using MS = MShape<D>;
  f.rowok = 0u;
  if (a.bs >= 16) {
    // A tile never crosses a block: one scalar table load per tile, so the row loads wait
    // only on the scalar counter and the previous pass's loads stay in flight.
#pragma unroll
    for (int t = 0; t < MS::TPW; ++t) {
      const int tb = __builtin_amdgcn_readfirstlane(base + 16 * t < t1 ? base + 16 * t : base);
      const int blk = load_uniform_i32(table + (tb >> a.log2_bs));
      const bool bok = blk >= 0 && blk < a.ncb;
      const int tok = base + 16 * t + i16;
      const bool in = tok < t1;
      const int off = ((in ? tok : tb) & (a.bs - 1));
      f.rowok |= static_cast<uint32_t>(in && bok) << t;
      mfma_load_rows<D>(f, a, t, static_cast<int64_t>(((bok ? blk : 0) * a.hkv + kvh) * a.bs + off), grp);
    }
  } else {
#pragma unroll
    for (int t = 0; t < MS::TPW; ++t) {
      const int tb = base + 16 * t;
      const int tok = tb + i16;
      const bool in = tok < t1;
      const int tk = in ? tok : (tb < t1 ? tb : base);
      const int blk = table[tk >> a.log2_bs];
      const bool bok = blk >= 0 && blk < a.ncb;
      f.rowok |= static_cast<uint32_t>(in && bok) << t;
      mfma_load_rows<D>(f, a, t, static_cast<int64_t>(((bok ? blk : 0) * a.hkv + kvh) * a.bs + (tk & (a.bs - 1))),
                        grp);
    }
  }
}

template <int DT, int D, int G>
__global__ __launch_bounds__(kNW * kWave) void paged_decode_part_mfma(DecodeArgs a) {
  using MS = MShape<D>;
  using Ops = MfmaOps<DT>;
  using S = typename Elem<DT>::S;
  constexpr int KC = MS::KC, MT = MS::MT, TPW = MS::TPW, PASS = MS::PASS;
  constexpr int LDS_TILES = kNW * TPW * MS::TILE_BYTES;
  constexpr int LDS_MERGE = (kNW * G * D + 2 * kNW * 16) * 4;
  constexpr int LDS_BYTES = LDS_TILES > LDS_MERGE ? LDS_TILES : LDS_MERGE;
  __shared__ __attribute__((aligned(16))) char smem[LDS_BYTES];

  const int part = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int i16 = lane & 15, grp = lane >> 4;
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

  // Q^T operand: lane l holds q[head l%16][dims 32*kc + 8*(l/16) .. +7], zero past G.
  uint4 qb[KC];
  {
    const char* qrow = a.q + (static_cast<int64_t>(b) * a.q_sb + static_cast<int64_t>(h0 + i16) * a.q_sh) * 2;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      qb[kc] = i16 < G ? *reinterpret_cast<const uint4*>(qrow + 64 * kc + 16 * grp) : make_uint4(0, 0, 0, 0);
  }

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m = -INFINITY, l = 0.0f;
  const bool head_live = i16 < G;
  const int32_t* table = a.bt + static_cast<int64_t>(b) * a.bt_stride;
  char* my_tiles = smem + w * TPW * MS::TILE_BYTES;

  auto compute = [&](const MFrag<D>& f, int base) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tb = base + 16 * t;
      const bool ok_row = (f.rowok >> t) & 1u;
      // Value rows into this wavefront's LDS tile (zeros for rows that are not keys).
      char* tile = my_tiles + t * MS::TILE_BYTES;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const uint4 vv = ok_row ? f.v[t][kc] : make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(tile + i16 * (D * 2) + 64 * kc + 16 * grp) = vv;
      }
      // Keys valid as rows of the S^T output: row j = 4*grp + i is a key iff lane j's row was.
      const uint32_t okmask = static_cast<uint32_t>(__ballot(ok_row)) & 0xffffu;
      f32x4_t st = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) st = Ops::qk(f.k[t][kc], qb[kc], st);
      float sv[4];
      bool need = false;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = head_live && ((okmask >> (4 * grp + i)) & 1u) && (tb + 4 * grp + i < t1);
        sv[i] = ok ? st[i] * a.scale_log2 : -INFINITY;
        need |= sv[i] > m + kRescaleLog2;
      }
      if (__any(need)) {
        float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float alpha = (m == -INFINITY) ? 0.0f : fast_exp2(m - mn);
        l *= alpha;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] *= alpha;
        m = mn;
      }
      uint32_t ph[2], pl[2];
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float p0 = sv[i] == -INFINITY ? 0.0f : fast_exp2(sv[i] - m);
        const float p1 = sv[i + 1] == -INFINITY ? 0.0f : fast_exp2(sv[i + 1] - m);
        l += p0 + p1;
        const uint16_t h0b = Ops::round16(p0), h1b = Ops::round16(p1);
        const uint16_t l0b = Ops::round16(p0 - Ops::widen16(h0b)), l1b = Ops::round16(p1 - Ops::widen16(h1b));
        ph[i / 2] = static_cast<uint32_t>(h0b) | (static_cast<uint32_t>(h1b) << 16);
        pl[i / 2] = static_cast<uint32_t>(l0b) | (static_cast<uint32_t>(l1b) << 16);
      }
      __builtin_amdgcn_wave_barrier();
      // V^T operand: lane l takes keys 4*grp + i at dim 16*mt + i16.
      const uint16_t* tv = reinterpret_cast<const uint16_t*>(tile) + (4 * grp) * D + i16;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint32_t e0 = tv[16 * mt], e1 = tv[D + 16 * mt], e2 = tv[2 * D + 16 * mt], e3 = tv[3 * D + 16 * mt];
        const uint2 va = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
        acc[mt] = Ops::pv(va, make_uint2(ph[0], ph[1]), acc[mt]);
        acc[mt] = Ops::pv(va, make_uint2(pl[0], pl[1]), acc[mt]);
      }
      __builtin_amdgcn_wave_barrier();
    }
  };

  constexpr int kStep = kNW * PASS;
  int base = t0 + w * PASS;
  if (base < t1) {
    MFrag<D> fa, fb;
    mfma_load<D>(fa, a, table, kvh, base, t1, i16, grp);
    while (true) {
      int nb = base + kStep;
      mfma_load<D>(fb, a, table, kvh, nb < t1 ? nb : base, t1, i16, grp);
      compute(fa, base);
      base = nb;
      if (base >= t1) break;
      nb = base + kStep;
      mfma_load<D>(fa, a, table, kvh, nb < t1 ? nb : base, t1, i16, grp);
      compute(fb, base);
      base = nb;
      if (base >= t1) break;
    }
  }

  // ---- per-wave totals: l summed over the 4 lane groups; acc needs no reduction.
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  __syncthreads();  // the merge area overlaps other wavefronts' value tiles
  float* sh_acc = reinterpret_cast<float*>(smem);          // [kNW][G][D]
  float* sh_m = sh_acc + kNW * G * D;                       // [kNW][16]
  float* sh_l = sh_m + kNW * 16;                            // [kNW][16]
  if (head_live) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sh_acc[(w * G + i16) * D + 16 * mt + 4 * grp + i] = acc[mt][i];
    }
    if (grp == 0) {
      sh_m[w * 16 + i16] = m;
      sh_l[w * 16 + i16] = l;
    }
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kNW * kWave) {
    const int g = i / D, d = i % D;
    float mx = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kNW; ++ww) mx = fmaxf(mx, sh_m[ww * 16 + g]);
    float A = 0.0f, Ls = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kNW; ++ww) {
      const float mw = sh_m[ww * 16 + g];
      const float wt = (mw == -INFINITY) ? 0.0f : fast_exp2(mw - mx);
      A = fmaf(wt, sh_acc[(ww * G + g) * D + d], A);
      Ls = fmaf(wt, sh_l[ww * 16 + g], Ls);
    }
    if (np_b == 1) {
      out_base[b * a.out_sb + (h0 + g) * a.out_sh + d] = from_f32<DT>(Ls > 0.0f ? A / Ls : 0.0f);
    } else {
      const int64_t slot = (static_cast<int64_t>(b) * a.hq + h0 + g) * a.nparts + part;
      a.ws_acc[slot * D + d] = A;
      if (d == 0) {
        a.ws_ml[slot * 2] = mx;
        a.ws_ml[slot * 2 + 1] = Ls;
      }
    }
  }
}

// Combine the partitions of every sequence that needed more than one. Grid (groups of G query
// heads, batch): kv heads, or kv heads x a.gsplit for a split VALU group.
template <int DT, int D, int G>
__global__ __launch_bounds__(256) void paged_decode_merge(DecodeArgs a) {
  using S = typename Elem<DT>::S;
  const int hg = blockIdx.x, b = blockIdx.y;
  int ctx = a.lens[b];
  const int cap = a.max_blocks * a.bs;
  ctx = ctx < cap ? ctx : cap;
  const int np_b = ctx > 0 ? (ctx + a.part_tokens - 1) / a.part_tokens : 1;
  if (np_b <= 1) return;
  S* out_base = reinterpret_cast<S*>(a.out);
  // The heads of workgroup y of the partition kernel (see paged_decode_part).
  const int kvh = a.gsplit > 1 ? hg / a.gsplit : hg;
  const int h0 = a.gsplit > 1 ? kvh * a.group + (hg - kvh * a.gsplit) * G : hg * G;
  const int nh = a.gsplit > 1 ? min(G, a.group - (hg - kvh * a.gsplit) * G) : G;
  for (int i = threadIdx.x; i < nh * D; i += blockDim.x) {
    const int g = i / D, d = i % D;
    const int64_t slot0 = (static_cast<int64_t>(b) * a.hq + h0 + g) * a.nparts;
    float mx = -INFINITY;
    for (int pp = 0; pp < np_b; ++pp) mx = fmaxf(mx, a.ws_ml[(slot0 + pp) * 2]);
    float A = 0.0f, Ls = 0.0f;
    for (int pp = 0; pp < np_b; ++pp) {
      const float mp = a.ws_ml[(slot0 + pp) * 2];
      const float wt = (mp == -INFINITY) ? 0.0f : fast_exp2(mp - mx);
      A = fmaf(wt, a.ws_acc[(slot0 + pp) * D + d], A);
      Ls = fmaf(wt, a.ws_ml[(slot0 + pp) * 2 + 1], Ls);
    }
    out_base[b * a.out_sb + (h0 + g) * a.out_sh + d] = from_f32<DT>(Ls > 0.0f ? A / Ls : 0.0f);
  }
}

// ------------------------------------------------------------------ host side

inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

enum class Algo { kValu, kMfma, kStream };

bool mfma_eligible(int dtype, int d, int g) {
  return (dtype == MIP_BF16 || dtype == MIP_F16) && (d == 64 || d == 128) && g >= 1 && g <= 16;
}

// Forced algorithm (mip_set_decode_algo; MIP_ALGO_AUTO = the default choice below). Its
// first value comes from MIP_DECODE_ALGO=valu|mfma|stream, read once.
int algo_from_env() {
  const char* env = std::getenv("MIP_DECODE_ALGO");
  const char f = env ? env[0] : 0;
  return f == 'v' ? MIP_ALGO_VALU : f == 'm' ? MIP_ALGO_MFMA : f == 's' ? MIP_ALGO_STREAM : MIP_ALGO_AUTO;
}
std::atomic<int>& forced_algo() {
  static std::atomic<int> v{algo_from_env()};
  return v;
}

// Default: the stream-K MFMA kernel for 16-bit data at head_dim 64/128 (balanced persistent
// work split, the fastest under rocprof at the Qwen shapes) while its per-sequence scan fits
// in LDS (batch <= 4096); otherwise the per-partition MFMA kernel; the VALU kernel for fp32
// and the other head sizes. A forced algorithm applies where its kernel exists.
Algo choose_algo(int dtype, int d, int g, int batch) {
  const int f = forced_algo().load(std::memory_order_relaxed);
  const bool mfma_ok = mfma_eligible(dtype, d, g);
  const bool stream_ok = mfma_ok && stream_config(dtype, d, g, batch).ok;
  if (f == MIP_ALGO_VALU) return Algo::kValu;
  if (f == MIP_ALGO_MFMA && mfma_ok) return Algo::kMfma;
  if (f == MIP_ALGO_STREAM && stream_ok) return Algo::kStream;
  return stream_ok ? Algo::kStream : mfma_ok ? Algo::kMfma : Algo::kValu;
}

int pass_tokens(Algo algo, int dtype, int d) {
  if (algo != Algo::kValu) return d <= 64 ? 32 : 16;
  const int es = dtype == MIP_F32 ? 4 : 2;
  const int ch = d < 32 / es ? d : 32 / es;
  return kWave / (d / ch);
}

// Keys per partition of the partition kernels (MIP_PART_TOKENS, read once).
int part_tokens_env() {
  static const int v = [] {
    const char* env = std::getenv("MIP_PART_TOKENS");
    const int x = env ? std::atoi(env) : 0;
    return x > 0 ? x : kDefaultPartTokens;
  }();
  return v;
}

int part_tokens_for(Algo algo, int dtype, int d) {
  const int align = kNW * pass_tokens(algo, dtype, d);
  return static_cast<int>(align_up(part_tokens_env(), align));
}

struct WsLayout {
  Algo algo;
  int part_tokens;
  int nparts;
  int64_t ml_off, acc_off, bytes;
  StreamConfig stream;          // stream kernel launch shape
  int64_t prefix_off, rec_off, part_off;  // stream kernel workspace
};

WsLayout ws_layout(int batch, int hq, int hkv, int d, int bs, int max_blocks, int dtype) {
  WsLayout w{};
  w.algo = choose_algo(dtype, d, hq / hkv, batch);
  if (w.algo == Algo::kStream) {
    w.stream = stream_config(dtype, d, hq / hkv, batch);
    if (!w.stream.ok) {
      w.algo = Algo::kMfma;
    } else {
      w.prefix_off = 0;
      w.rec_off = align_up(static_cast<int64_t>(batch + 1) * 4, 256);
      w.part_off = w.rec_off + align_up(static_cast<int64_t>(w.stream.tw) * 2 * w.stream.rec_floats * 4, 256);
      w.bytes = w.part_off + align_up(stream_part_floats(w.stream, batch, hkv) * 4, 256);
      w.nparts = 1;
      return w;
    }
  }
  w.part_tokens = part_tokens_for(w.algo, dtype, d);
  const int64_t max_ctx = static_cast<int64_t>(max_blocks) * bs;
  w.nparts = static_cast<int>((max_ctx + w.part_tokens - 1) / w.part_tokens);
  if (w.nparts < 1) w.nparts = 1;
  if (w.nparts == 1) return w;
  w.ml_off = 0;
  w.acc_off = align_up(static_cast<int64_t>(batch) * hq * w.nparts * 2 * 4, 256);
  w.bytes = w.acc_off + align_up(static_cast<int64_t>(batch) * hq * w.nparts * d * 4, 256);
  return w;
}

// Workgroups per kv head of the VALU kernel: ceil(g / 8), so each holds at most 8 query heads
// (a workgroup keeps q, the running maxima and sums and the accumulators of all its heads in
// registers). Each of them reads the kv head's keys and values, so the K/V traffic grows by
// this factor. valu_heads is the register slots per workgroup, ceil(g / split); the last
// workgroup of a group masks the slots past the group's end.
int valu_split(int g) { return g > 8 ? (g + 7) / 8 : 1; }
int valu_heads(int g) {
  const int s = valu_split(g);
  return (g + s - 1) / s;
}

using KernelFn = void (*)(DecodeArgs);
struct KernelPair {
  KernelFn part = nullptr;
  KernelFn merge = nullptr;
};

template <int DT, int D, int G>
KernelPair valu_pair() {
  return {paged_decode_part<DT, D, G>, paged_decode_merge<DT, D, G>};
}

template <int DT, int D>
KernelPair pick_valu_g(int g) {
  switch (g) {
    case 1: return valu_pair<DT, D, 1>();
    case 2: return valu_pair<DT, D, 2>();
    case 3: return valu_pair<DT, D, 3>();
    case 4: return valu_pair<DT, D, 4>();
    case 5: return valu_pair<DT, D, 5>();
    case 6: return valu_pair<DT, D, 6>();
    case 7: return valu_pair<DT, D, 7>();
    case 8: return valu_pair<DT, D, 8>();
    default: return {};
  }
}

template <int DT>
KernelPair pick_valu_d(int d, int g) {
  switch (d) {
    case 8: return pick_valu_g<DT, 8>(g);
    case 16: return pick_valu_g<DT, 16>(g);
    case 32: return pick_valu_g<DT, 32>(g);
    case 64: return pick_valu_g<DT, 64>(g);
    case 128: return pick_valu_g<DT, 128>(g);
    case 256: return pick_valu_g<DT, 256>(g);
    default: return {};
  }
}

template <int DT, int D, int G>
KernelPair mfma_pair() {
  return {paged_decode_part_mfma<DT, D, G>, paged_decode_merge<DT, D, G>};
}

template <int DT, int D>
KernelPair pick_mfma_g(int g) {
  switch (g) {
    case 1: return mfma_pair<DT, D, 1>();
    case 2: return mfma_pair<DT, D, 2>();
    case 3: return mfma_pair<DT, D, 3>();
    case 4: return mfma_pair<DT, D, 4>();
    case 5: return mfma_pair<DT, D, 5>();
    case 6: return mfma_pair<DT, D, 6>();
    case 7: return mfma_pair<DT, D, 7>();
    case 8: return mfma_pair<DT, D, 8>();
    case 9: return mfma_pair<DT, D, 9>();
    case 10: return mfma_pair<DT, D, 10>();
    case 11: return mfma_pair<DT, D, 11>();
    case 12: return mfma_pair<DT, D, 12>();
    case 13: return mfma_pair<DT, D, 13>();
    case 14: return mfma_pair<DT, D, 14>();
    case 15: return mfma_pair<DT, D, 15>();
    case 16: return mfma_pair<DT, D, 16>();
    default: return {};
  }
}

template <int DT>
KernelPair pick_mfma_d(int d, int g) {
  switch (d) {
    case 64: return pick_mfma_g<DT, 64>(g);
    case 128: return pick_mfma_g<DT, 128>(g);
    default: return {};
  }
}

KernelPair pick_kernel(Algo algo, int dtype, int d, int g) {
  if (algo == Algo::kMfma) {
    switch (dtype) {
      case MIP_F16: return pick_mfma_d<MIP_F16>(d, g);
      case MIP_BF16: return pick_mfma_d<MIP_BF16>(d, g);
      default: return {};
    }
  }
  switch (dtype) {
    case MIP_F32: return pick_valu_d<MIP_F32>(d, g);
    case MIP_F16: return pick_valu_d<MIP_F16>(d, g);
    case MIP_BF16: return pick_valu_d<MIP_BF16>(d, g);
    default: return {};
  }
}

}  // namespace

namespace decode {

int valu_prefill_launch(void* out, int64_t out_stride_tok, int64_t out_stride_head, const void* q,
                        int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache, const void* v_cache,
                        int64_t num_cache_blocks, const int32_t* block_tables, int64_t bt_stride, const int32_t* cu_q,
                        const int32_t* ctx_start, int32_t num_seqs, int32_t max_q_len, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                        float scale, int32_t dtype, hipStream_t stream) {
  const int group = num_heads / num_kv_heads;
  const int vsplit = valu_split(group);
  const KernelPair kp = pick_kernel(Algo::kValu, dtype, head_dim, valu_heads(group));
  if (!kp.part) return MIP_EUNSUPPORTED;
  const int64_t es = dtype == MIP_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15) return MIP_EINVAL;
  // q is read 4 bytes at a time, outputs are written one element at a time.
  if ((reinterpret_cast<uintptr_t>(q) | static_cast<uint64_t>(q_stride_tok * es) |
       static_cast<uint64_t>(q_stride_head * es)) & 3)
    return MIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(out) | static_cast<uint64_t>(out_stride_tok * es) |
       static_cast<uint64_t>(out_stride_head * es)) & (es - 1))
    return MIP_EINVAL;
  const int64_t cap = static_cast<int64_t>(max_blocks_per_seq) * block_size;
  if (cap >= (int64_t{1} << 30)) return MIP_EINVAL;
  if (num_cache_blocks * num_kv_heads * block_size >= (int64_t{1} << 31)) return MIP_EINVAL;
  const int64_t grid_x = static_cast<int64_t>(num_seqs) * max_q_len;
  if (grid_x >= (int64_t{1} << 31) || static_cast<int64_t>(num_kv_heads) * vsplit > 65535) return MIP_EUNSUPPORTED;
  DecodeArgs a{};
  a.out = static_cast<char*>(out);
  a.out_sb = out_stride_tok;
  a.out_sh = out_stride_head;
  a.q = static_cast<const char*>(q);
  a.q_sb = q_stride_tok;
  a.q_sh = q_stride_head;
  a.k = static_cast<const char*>(k_cache);
  a.v = static_cast<const char*>(v_cache);
  a.ncb = num_cache_blocks;
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  a.hq = num_heads;
  a.hkv = num_kv_heads;
  a.bs = block_size;
  a.log2_bs = ilog2_exact(block_size);
  a.max_blocks = max_blocks_per_seq;
  // One partition covers the longest row (at most max_blocks_per_seq * block_size keys).
  a.part_tokens = static_cast<int>(align_up(cap, kNW * pass_tokens(Algo::kValu, dtype, head_dim)));
  a.nparts = 1;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.cu_q = cu_q;
  a.ctx_start = ctx_start;
  a.max_q_len = max_q_len;
  a.gsplit = vsplit;
  a.group = group;
  hipLaunchKernelGGL(kp.part, dim3(static_cast<unsigned>(grid_x), num_kv_heads * vsplit, 1), dim3(kNW * kWave), 0,
                     stream, a);
  return status_from_hip(hipGetLastError());
}

}  // namespace decode
}  // namespace mip

using namespace mip;

extern "C" int mip_set_decode_algo(int32_t algo) {
  if (algo < MIP_ALGO_AUTO || algo > MIP_ALGO_STREAM) return MIP_EINVAL;
  return forced_algo().exchange(algo);
}

extern "C" size_t mip_paged_decode_workspace(int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                             int32_t block_size, int32_t max_blocks_per_seq, int32_t dtype) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0)
    return 0;
  return static_cast<size_t>(
      ws_layout(batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, dtype).bytes);
}

namespace {

// Decode attention; with app.slots set, the stream kernel also appends the step's new K/V
// rows (the caller has checked their 16-byte alignment and that the stream kernel runs).
int paged_decode_impl(void* out, int64_t out_stride_b, int64_t out_stride_h, const void* q, int64_t q_stride_b,
                      int64_t q_stride_h, const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
                      const int32_t* block_tables, int64_t bt_stride, const int32_t* context_lens, int32_t batch,
                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                      int32_t max_blocks_per_seq, float scale, void* workspace, size_t workspace_bytes,
                      const void* plan, size_t plan_bytes, int32_t dtype, void* stream, const AppendRows& app) {
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
  const WsLayout wl = ws_layout(batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, dtype);
  const int vsplit = wl.algo == Algo::kValu ? valu_split(group) : 1;
  const KernelPair kp = pick_kernel(wl.algo == Algo::kStream ? Algo::kMfma : wl.algo, dtype, head_dim,
                                    wl.algo == Algo::kValu ? valu_heads(group) : group);
  if (!kp.part) return MIP_EUNSUPPORTED;
  const int64_t es = dtype == MIP_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15) return MIP_EINVAL;
  const uint64_t q_align = wl.algo == Algo::kValu ? 3 : 15;  // MFMA kernels read q rows with 16-byte loads
  if ((reinterpret_cast<uintptr_t>(q) | static_cast<uint64_t>(q_stride_b * es) |
       static_cast<uint64_t>(q_stride_h * es)) & q_align)
    return MIP_EINVAL;
  const uint64_t out_align = wl.algo == Algo::kStream ? 7 : es - 1;  // the stream kernel stores 4 outputs at once
  if ((reinterpret_cast<uintptr_t>(out) | static_cast<uint64_t>(out_stride_b * es) |
       static_cast<uint64_t>(out_stride_h * es)) & out_align)
    return MIP_EINVAL;

  DecodeArgs a{};
  if (wl.nparts > 1 || wl.algo == Algo::kStream) {
    if (!workspace || workspace_bytes < static_cast<size_t>(wl.bytes) ||
        (reinterpret_cast<uintptr_t>(workspace) & 255))
      return MIP_EINVAL;
    char* ws = static_cast<char*>(workspace);
    if (wl.algo != Algo::kStream) {
      a.ws_ml = reinterpret_cast<float*>(ws + wl.ml_off);
      a.ws_acc = reinterpret_cast<float*>(ws + wl.acc_off);
    }
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
  a.part_tokens = wl.part_tokens;
  a.nparts = wl.nparts;
  a.scale_log2 = scale * 1.4426950408889634f;
  if (batch > 65535) return MIP_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (wl.algo == Algo::kStream) {
    StreamArgs sa{};
    sa.a = a;
    sa.batch = batch;
    sa.group = group;
    sa.ws_prefix = reinterpret_cast<int*>(static_cast<char*>(workspace) + wl.prefix_off);
    sa.ws_rec = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.rec_off);
    sa.ws_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.part_off);
    sa.app = app;
    // A plan drives the tile-descriptor kernel, which needs tiles inside one block and 32-bit
    // lane offsets into the q head rows; otherwise the kernel derives its split itself.
    const int64_t plan_need = stream_plan_bytes(wl.stream, batch, num_kv_heads, block_size, max_blocks_per_seq);
    const bool use_plan = plan != nullptr && plan_need > 0 && q_stride_h >= 0 &&
                          q_stride_h * 2 * 16 < (int64_t{1} << 31);
    if (plan && (reinterpret_cast<uintptr_t>(plan) & 7)) return MIP_EINVAL;
    // The kernel reads the plan at offsets of this shape's layout before it checks the header.
    if (use_plan && plan_bytes < static_cast<size_t>(plan_need)) return MIP_EINVAL;
    sa.plan = use_plan ? static_cast<const int32_t*>(plan) : nullptr;
    if (use_plan)
      stream_plan_offsets(wl.stream, batch, num_kv_heads, block_size, max_blocks_per_seq, &sa.plan_seg_off,
                          &sa.plan_tile_off, &sa.plan_wave_cap);
    sa.nrows = static_cast<uint32_t>(num_cache_blocks * num_kv_heads * block_size);
    const int64_t lim = int64_t{1} << 31;
    for (const int64_t x : {q_stride_b, q_stride_h, out_stride_b, out_stride_h, bt_stride, num_cache_blocks})
      if (x <= -lim || x >= lim) return MIP_EUNSUPPORTED;
    sa.q_sb = static_cast<int32_t>(q_stride_b);
    sa.q_sh = static_cast<int32_t>(q_stride_h);
    sa.out_sb = static_cast<int32_t>(out_stride_b);
    sa.out_sh = static_cast<int32_t>(out_stride_h);
    sa.bt_stride = static_cast<int32_t>(bt_stride);
    sa.ncb = static_cast<int32_t>(num_cache_blocks);
    const int st = stream_launch(wl.stream, sa, dtype, head_dim, group, num_kv_heads, batch, s);
    return st == 0 ? MIP_OK : st;
  }
  if (app.slots) return MIP_EUNSUPPORTED;  // callers fuse only into the stream kernel
  if (static_cast<int64_t>(num_kv_heads) * vsplit > 65535) return MIP_EUNSUPPORTED;
  a.gsplit = vsplit;
  a.group = group;
  hipLaunchKernelGGL(kp.part, dim3(wl.nparts, num_kv_heads * vsplit, batch), dim3(kNW * kWave), 0, s, a);
  if (wl.nparts > 1) hipLaunchKernelGGL(kp.merge, dim3(num_kv_heads * vsplit, batch), dim3(256), 0, s, a);
  return status_from_hip(hipGetLastError());
}

}  // namespace

extern "C" int mip_paged_decode(void* out, int64_t out_stride_b, int64_t out_stride_h, const void* q,
                                int64_t q_stride_b, int64_t q_stride_h, const void* k_cache, const void* v_cache,
                                int64_t num_cache_blocks, const int32_t* block_tables, int64_t bt_stride,
                                const int32_t* context_lens, int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq, float scale,
                                void* workspace, size_t workspace_bytes, const void* plan, size_t plan_bytes,
                                int32_t dtype, void* stream) {
  return paged_decode_impl(out, out_stride_b, out_stride_h, q, q_stride_b, q_stride_h, k_cache, v_cache,
                           num_cache_blocks, block_tables, bt_stride, context_lens, batch, num_heads, num_kv_heads,
                           head_dim, block_size, max_blocks_per_seq, scale, workspace, workspace_bytes, plan,
                           plan_bytes, dtype, stream, AppendRows{});
}

extern "C" int mip_paged_decode_append(const void* k_new, const void* v_new, int64_t k_stride_tok,
                                       int64_t k_stride_head, int64_t v_stride_tok, int64_t v_stride_head,
                                       const int64_t* slot_mapping, void* out, int64_t out_stride_b,
                                       int64_t out_stride_h, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                       void* k_cache, void* v_cache, int64_t num_cache_blocks,
                                       const int32_t* block_tables, int64_t bt_stride, const int32_t* context_lens,
                                       int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                       int32_t block_size, int32_t max_blocks_per_seq, float scale, void* workspace,
                                       size_t workspace_bytes, const void* plan, size_t plan_bytes, int32_t dtype,
                                       void* stream) {
  if (dtype != MIP_F32 && dtype != MIP_F16 && dtype != MIP_BF16) return MIP_EINVAL;
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return MIP_EINVAL;
  if (batch == 0) return MIP_OK;
  if (!k_new || !v_new || !slot_mapping) return MIP_EINVAL;
  const int64_t es = dtype == MIP_F32 ? 4 : 2;
  const uint64_t align = reinterpret_cast<uintptr_t>(k_new) | reinterpret_cast<uintptr_t>(v_new) |
                         static_cast<uint64_t>(k_stride_tok * es) | static_cast<uint64_t>(k_stride_head * es) |
                         static_cast<uint64_t>(v_stride_tok * es) | static_cast<uint64_t>(v_stride_head * es) |
                         static_cast<uint64_t>(head_dim * es);
  const WsLayout wl = ws_layout(batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, dtype);
  const int64_t lim = int64_t{1} << 31;
  bool strides_fit = true;
  for (const int64_t x : {k_stride_tok * es, k_stride_head * es, v_stride_tok * es, v_stride_head * es})
    strides_fit = strides_fit && x > -lim && x < lim;
  if (wl.algo == Algo::kStream && (align & 15) == 0 && strides_fit && batch <= 65535) {
    AppendRows app{};
    app.k = static_cast<const char*>(k_new);
    app.v = static_cast<const char*>(v_new);
    app.k_st = static_cast<int32_t>(k_stride_tok * es);
    app.k_sh = static_cast<int32_t>(k_stride_head * es);
    app.v_st = static_cast<int32_t>(v_stride_tok * es);
    app.v_sh = static_cast<int32_t>(v_stride_head * es);
    app.slots = slot_mapping;
    app.k_cache = static_cast<char*>(k_cache);
    app.v_cache = static_cast<char*>(v_cache);
    return paged_decode_impl(out, out_stride_b, out_stride_h, q, q_stride_b, q_stride_h, k_cache, v_cache,
                             num_cache_blocks, block_tables, bt_stride, context_lens, batch, num_heads,
                             num_kv_heads, head_dim, block_size, max_blocks_per_seq, scale, workspace,
                             workspace_bytes, plan, plan_bytes, dtype, stream, app);
  }
  // Not fusable here: the append kernel, then the decode, in stream order.
  const int st = mip_kv_append(k_new, v_new, k_stride_tok, k_stride_head, v_stride_tok, v_stride_head, k_cache,
                               v_cache, num_cache_blocks, slot_mapping, batch, num_kv_heads, head_dim, block_size,
                               dtype, stream);
  if (st != MIP_OK) return st;
  return mip_paged_decode(out, out_stride_b, out_stride_h, q, q_stride_b, q_stride_h, k_cache, v_cache,
                          num_cache_blocks, block_tables, bt_stride, context_lens, batch, num_heads, num_kv_heads,
                          head_dim, block_size, max_blocks_per_seq, scale, workspace, workspace_bytes, plan,
                          plan_bytes, dtype, stream);
}

extern "C" size_t mip_paged_decode_plan_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                              int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                                              int32_t dtype) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0 || num_heads % num_kv_heads != 0)
    return 0;
  const WsLayout wl = ws_layout(batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, dtype);
  if (wl.algo != Algo::kStream) return 0;
  return static_cast<size_t>(stream_plan_bytes(wl.stream, batch, num_kv_heads, block_size, max_blocks_per_seq));
}

extern "C" int mip_paged_decode_plan(const int32_t* context_lens, const int32_t* block_tables, int64_t bt_stride,
                                     int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t block_size, int32_t max_blocks_per_seq, int32_t dtype, void* plan,
                                     size_t plan_bytes, void* stream) {
  if (dtype != MIP_F32 && dtype != MIP_F16 && dtype != MIP_BF16) return MIP_EINVAL;
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return MIP_EINVAL;
  if (num_heads % num_kv_heads != 0) return MIP_EINVAL;
  if (!is_pow2(block_size) || block_size > 4096 || max_blocks_per_seq <= 0 || bt_stride < max_blocks_per_seq)
    return MIP_EINVAL;
  if (static_cast<int64_t>(max_blocks_per_seq) * block_size >= (int64_t{1} << 30)) return MIP_EINVAL;
  if (!context_lens || !block_tables || !plan || (reinterpret_cast<uintptr_t>(plan) & 7)) return MIP_EINVAL;
  const WsLayout wl = ws_layout(batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, dtype);
  if (wl.algo != Algo::kStream) return MIP_EUNSUPPORTED;
  const int64_t need = stream_plan_bytes(wl.stream, batch, num_kv_heads, block_size, max_blocks_per_seq);
  if (need == 0) return MIP_EUNSUPPORTED;
  if (plan_bytes < static_cast<size_t>(need)) return MIP_EINVAL;
  const int st = stream_plan_launch(wl.stream, context_lens, block_tables, bt_stride, batch, num_kv_heads, block_size,
                                    max_blocks_per_seq, static_cast<int32_t*>(plan), static_cast<hipStream_t>(stream));
  return st == 0 ? MIP_OK : st;
}
