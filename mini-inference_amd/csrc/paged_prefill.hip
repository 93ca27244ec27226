// Paged varlen prefill attention over a cached prefix (gfx950, MFMA).
//
// Reference semantics (engine/kv_cache.py:268-294 PackedPrefillContext with a prefix hit,
// engine/model.py:101-123 sdpa_attention): several sequences' new tokens are packed end to
// end; new token i of sequence s sits at position p = ctx_start[s] + i and attends every key
// 0..p of its own sequence (the cached prefix and the new tokens before it, already appended
// to the pool). The reference reads all those keys back out of the pool and runs SDPA with a
// dense [N, total keys] mask; here the keys are read in place through the block table and
// only each sequence's own causal range is computed. With ctx_start = 0 this is the packed
// block-diagonal causal prefill of engine/kv_cache.py:290-294.
//
// Work split: an item is (kv head, sequence, block of TQ new tokens), done by a workgroup of
// 4 wavefronts owning NC 16-row column blocks each. The item's query rows are its (token,
// head of the kv head's group) pairs, packed token-major with no padding: row r is head
// r % G of token r / G, and TQ = 64 NC / G tokens fill all but 64 NC mod G rows (252 of 256
// at G = 7). The grid is persistent and walks a longest-first work list
// (paged_prefill_kernel).
//
// Per 32-key tile: all 256 threads copy the K and V rows (found through the block table) into
// an LDS stage (two stages: the next tile's rows are fetched into registers while the current
// one is computed); then each wavefront computes, for each 16-key half,
//   S^T[16 keys x 16 rows] = K . Q^T      v_mfma_f32_16x16x32, D/32 steps (Q^T in registers)
// and then, over all 32 keys,
//   O^T[D x 16 rows]      += V^T . P^T    v_mfma_f32_16x16x32, D/16 tiles (fp16 P; bf16 V staged as fp16)
// with a base-2 online softmax per row, as in the decode kernels. Rows whose position is below
// a key mask it out; a wavefront skips tiles that lie beyond all of its rows' positions, and a
// column block skips the masking in steps whose keys all of its live rows see (most of them).
// The kernel is VALU-bound, so the softmax step is kept short: the rescale test on each lane's
// maximum, the scale folded into the exponent's fma, and the row sums taken on the matrix
// cores (the weights against a block of ones, one more 16x16x32 product per column block);
// V^T comes from transposing LDS reads.
#include "paged_decode_common.h"

namespace mip {
namespace prefill {
namespace {

using decode::f32x4_t;
using decode::fast_exp2;
using decode::kRescaleLog2;
using decode::MfmaOps;

#ifndef MIP_PREFILL_KT
#define MIP_PREFILL_KT 32
#endif
// Column blocks per wavefront: 4 at head_dim 64 (fewer barriers and K/V reads per row; 2
// wavefronts per SIMD), 2 at head_dim 128 (register file).
#ifndef MIP_PREFILL_NC
#define MIP_PREFILL_NC 0
#endif
constexpr int kPW = 4;                 // wavefronts per workgroup
constexpr int kKT = MIP_PREFILL_KT;    // keys per LDS tile (a multiple of 32)
static_assert(kKT % 32 == 0, "tiles are whole 32-key PV steps");

struct PrefillArgs {
  char* out;
  int64_t out_st, out_sh;  // elements
  const char* q;
  int64_t q_st, q_sh;      // elements
  const char* k;
  const char* v;
  int64_t ncb;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* cu_q;       // [S + 1] packed row offsets of each sequence's new tokens
  const int32_t* ctx_start;  // [S] tokens cached before this pass (position of token 0)
  int hkv, group, bs, log2_bs, max_blocks;
  int tq;                  // new tokens per work item: query rows per item / group
  int num_seqs, zb;        // sequences; blocks of tq new tokens the longest one can have
  float scale_log2;
};

// Maxima by IEEE 754-2019 maximum (v_maximum3_f32 on gfx950). fmaxf (maxNum) has to quiet
// signalling NaNs in IEEE mode, which costs one extra v_max per operand that is not the
// result of arithmetic (MFMA outputs, lane exchanges); maximum needs no such step. The two
// differ only on NaN operands, which scores never are.
__device__ __forceinline__ float fmax2(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fmax3(float a, float b, float c) { return fmax2(fmax2(a, b), c); }
__device__ __forceinline__ float max4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = fmax2(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return fmax2(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// P = exp2(s - m) lies in [0, 2^kRescaleLog2]. fp16 holds it to 2^-11 relative, enough for
// the 2e-3 bound on outputs that are convex combinations of the values; bf16 (2^-8) is not.
// bf16 items therefore first run with V converted to fp16 as it is staged (bf16x8_to_f16x8:
// exact for every value fp16 can hold), so P stays fp16 and the PV product is one fp16
// MFMA; an item that meets a value fp16 cannot hold (|v| >= 65536, inf, NaN) runs again with
// bf16 V and P split into a rounded part and its remainder, each multiplied by V^T.
template <int DT, bool VF16> constexpr bool kSplitP = DT == MIP_BF16 && !VF16;

// Eight bf16 values -> fp16 in place. bf16 has 8 significand bits and fp16 11, so the
// conversion is exact down to 2^-17 (smaller magnitudes land on fp16's subnormal grid of
// 2^-24, a change of at most 2^-25) and up to 65280, the largest bf16 value below 65536;
// 65536 and more become inf (round to nearest even), inf and NaN stay what they are.
__device__ __forceinline__ void bf16x8_to_f16x8(uint4& v) {
  auto cv = [](uint32_t x) __attribute__((always_inline)) {
    return MfmaOps<MIP_F16>::pack2(__uint_as_float(x << 16), __uint_as_float(x & 0xffff0000u));
  };
  v = make_uint4(cv(v.x), cv(v.y), cv(v.z), cv(v.w));
}

// ds_read_b64_tr_b16: within each 16-lane group, lane j supplies 4 consecutive 16-bit
// elements A[j][0..3]; lane i receives A[i / 4][i % 4], A[4 + i / 4][i % 4],
// A[8 + i / 4][i % 4], A[12 + i / 4][i % 4] (as measured on gfx950).
typedef short v4i16_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_tr16(const char* p) {
  typedef __attribute__((address_space(3))) v4i16_t lv4_t;
  const v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lv4_t*)(p));
  return __builtin_bit_cast(uint2, r);
}

template <int D>
struct PShape {
  static constexpr int RB = 2 * D;                 // bytes per K / V row
  static constexpr int CPR = RB / 16;              // 16-byte chunks per row
  static constexpr int KC = D / 32;                // QK k-steps
  static constexpr int MT = D / 16;                // PV output tiles
  static constexpr int TILE = kKT * RB;            // bytes of one K (or V) tile
  static constexpr int STAGE = 2 * TILE;           // K | V
  static constexpr int NLD = kKT * CPR / (kPW * kWave);  // 16-byte chunks per thread per tile, each of K and V
  // V row r keeps its 16-byte chunk c at c ^ vsw(r). The XOR is even, so each 32-byte segment a
  // transposing read takes stays whole, and the rows one such read touches (4 grp + 0..3 per
  // 16 lanes, 8 rows per 32 lanes) start their segment in distinct banks of a 128-byte or a
  // 256-byte bank window.
  static __device__ __forceinline__ int vsw(int r) { return CPR >= 16 ? 2 * (r & 7) : 2 * ((r + (r >> 2)) & 3); }
  static_assert(NLD >= 1 && NLD * kPW * kWave == kKT * CPR, "tile must split evenly over the workgroup");
};

// One work item: new tokens [tok_lo, tok_end) of sequence s against kv head kvh, at most
// TQ = 64 NC / G of them (the rows of NC column blocks per wavefront). smem holds the two
// K | V stages, s_ok[stage][key] whether a key row is a real key (valid block id), byte w of
// s_wok[stage] whether every key row wavefront w loaded is. Called by the whole workgroup
// (the barriers inside are workgroup-wide).
// q0, n_s and start are cu_q[s], cu_q[s + 1] - cu_q[s] and ctx_start[s] (the caller reads them).
// VF16 (bf16 only): V is converted to fp16 as it is staged. A V value fp16 cannot hold is inf
// there, and the PV product multiplies every key of a tile into every row of the wavefront
// (0 * inf = NaN), so a wavefront that reached such a key holds a non-finite accumulator; a
// wavefront that did not has no row that sees it. A wavefront with a non-finite accumulator
// stores tag in *s_big; the item then writes nothing and returns true, and the caller runs it
// again without VF16 (so do items whose inputs are inf or NaN). tag differs between the items
// a workgroup runs.
template <int DT, int D, int NC, bool VF16>
__device__ __forceinline__ bool prefill_item(const PrefillArgs& a, int kvh, int s, int q0, int n_s, int start_in,
                                             int tok_lo, int tok_end, uint32_t tag, char* smem,
                                             uint8_t (*s_ok)[kKT], uint32_t* s_wok, uint32_t* s_big) {
  static_assert(!VF16 || DT == MIP_BF16, "V is converted from bf16 only");
  using P = PShape<D>;
  using Ops = MfmaOps<DT>;                     // Q, K and the output
  using OpsV = MfmaOps<VF16 ? MIP_F16 : DT>;  // V and P
  constexpr int RB = P::RB, CPR = P::CPR, KC = P::KC, MT = P::MT;
  const int TQ = kPW * NC * 16 / a.group;  // token capacity of the item's rows

  if (tok_lo >= n_s) return false;
  const int tok_hi = tok_end < n_s ? tok_end : n_s;
  const int start = start_in > 0 ? start_in : 0;
  const int cap = a.max_blocks * a.bs;
  int p_last = start + tok_hi - 1;
  p_last = p_last < cap - 1 ? p_last : cap - 1;  // keys past the table are never read
  const int n_tiles = (p_last + kKT) / kKT;
  const int G = a.group;

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int i16 = lane & 15, grp = lane >> 4;
  const int32_t* table = a.bt + static_cast<int64_t>(s) * a.bt_stride;

  // ---- this lane's query row in each column block, and its Q^T operand.
  int pos[NC];
  bool live[NC];
  uint4 qreg[NC][KC];
  int wave_pmax = -1;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    // Row r = 16 (NC w + c) + i16 of the item: head g = r % G of its token r / G.
    const int r = (w * NC + c) * 16 + i16;
    const int tr = r / G, g = r - tr * G;
    const int tok = tok_lo + tr;
    live[c] = tr < TQ && tok < tok_hi;
    const int p = start + tok;
    pos[c] = live[c] ? (p < cap - 1 ? p : cap - 1) : -1;
    int last_tok = tok_lo + ((w * NC + c) * 16 + 15) / G;  // the block's last row's token
    last_tok = last_tok < tok_lo + TQ - 1 ? last_tok : tok_lo + TQ - 1;
    const int wp = start + (last_tok < tok_hi - 1 ? last_tok : tok_hi - 1);
    wave_pmax = wp > wave_pmax ? wp : wave_pmax;
    const char* qrow = a.q + ((static_cast<int64_t>(q0) + (live[c] ? tok : 0)) * a.q_st +
                              static_cast<int64_t>(kvh * G + (live[c] ? g : 0)) * a.q_sh) * 2;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      qreg[c][kc] = live[c] ? *reinterpret_cast<const uint4*>(qrow + (32 * kc + 8 * grp) * 2) : make_uint4(0, 0, 0, 0);
  }
  wave_pmax = __builtin_amdgcn_readfirstlane(wave_pmax < cap - 1 ? wave_pmax : cap - 1);
  // Per column block, the smallest position of its live rows (a key at or below it is
  // visible to every live row of the block).
  int pmin[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    int v = live[c] ? pos[c] : 0x7fffffff;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) v = min(v, __shfl_xor(v, d));
    pmin[c] = __builtin_amdgcn_readfirstlane(v);
  }
  int pmin_all = pmin[0];
#pragma unroll
  for (int c = 1; c < NC; ++c) pmin_all = pmin[c] < pmin_all ? pmin[c] : pmin_all;

  // ---- loader: this thread's K / V chunks of a tile. The block ids of a tile are read one
  // tile ahead of its rows, so the table lookup does not add a second latency per tile.
  uint4 kbuf[P::NLD], vbuf[P::NLD];
  bool okbuf[P::NLD];
  int bid[P::NLD];
  auto lookup = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < P::NLD; ++j) {
      const int r = (tid + j * kPW * kWave) / CPR;
      const int key = t * kKT + r;
      const int kk = key < p_last ? key : p_last;
      bid[j] = table[kk >> a.log2_bs];
    }
  };
  auto fetch = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < P::NLD; ++j) {
      const int idx = tid + j * kPW * kWave;
      const int r = idx / CPR, c = idx % CPR;
      const int key = t * kKT + r;
      const int kk = key < p_last ? key : p_last;
      const int b = bid[j];
      const bool bok = b >= 0 && b < a.ncb;
      const bool ok = key <= p_last && bok;
      // Keys past the last position re-read that position's row (a real key, so finite V: the
      // PV product multiplies every row of the tile, masked or not).
      // Pool row (block b, head kvh, offset): one 32 x 32 -> 64-bit multiply-add.
      const uint64_t row = static_cast<uint64_t>(bok ? static_cast<uint32_t>(b) : 0u) * static_cast<uint32_t>(a.hkv * a.bs) +
                           static_cast<uint32_t>(kvh * a.bs + (kk & (a.bs - 1)));
      kbuf[j] = *reinterpret_cast<const uint4*>(a.k + row * RB + c * 16);
      vbuf[j] = *reinterpret_cast<const uint4*>(a.v + row * RB + c * 16);
      okbuf[j] = ok;
    }
  };
  auto stash = [&](int stage) __attribute__((always_inline)) {
    char* st = smem + stage * P::STAGE;
#pragma unroll
    for (int j = 0; j < P::NLD; ++j) {
      const int idx = tid + j * kPW * kWave;
      const int r = idx / CPR, c = idx % CPR;
      uint4 vv = vbuf[j];
      if constexpr (VF16) bf16x8_to_f16x8(vv);
      *reinterpret_cast<uint4*>(st + r * RB + ((c ^ (r & (CPR - 1))) * 16)) = kbuf[j];  // K swizzled by row
      *reinterpret_cast<uint4*>(st + P::TILE + r * RB + ((c ^ P::vsw(r)) * 16)) = vv;
      if (c == 0) s_ok[stage][r] = okbuf[j];
    }
    bool wok = true;
#pragma unroll
    for (int j = 0; j < P::NLD; ++j) wok = wok && okbuf[j];
    wok = __all(wok);
    if (lane == 0) reinterpret_cast<uint8_t*>(&s_wok[stage])[w] = wok ? 1 : 0;
  };

  f32x4_t acc[NC][MT];
  f32x4_t lacc[NC];  // row sums by MFMA against a ones block: every element holds row i16's sum
  float m[NC];
  float mth[NC], nm[NC];  // the rescale threshold (m + kRescaleLog2) / scale_log2, and -m (0 while m = -inf)
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    m[c] = -INFINITY;
    mth[c] = -INFINITY;
    nm[c] = 0.0f;
    lacc[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[c][mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }

  lookup(0);
  fetch(0);
  if (n_tiles > 1) lookup(1);
  stash(0);
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int stage = t & 1;
    if (t + 1 < n_tiles) {
      fetch(t + 1);
      if (t + 2 < n_tiles) lookup(t + 2);
    }
    const char* st_tile = smem + stage * P::STAGE;
#pragma unroll
    for (int h = 0; h < kKT / 32; ++h) {
    const char* st = st_tile + h * 32 * RB;  // K rows of this 32-key step (V rows at + TILE)
    const int key0 = t * kKT + 32 * h;
    if (key0 <= wave_pmax) {  // else every row of this wavefront sits before these keys
      // K operands of the two 16-key halves (keys 16u + i16).
      uint4 kreg[2][KC];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
          const int r = 16 * u + i16, ch = 4 * kc + grp;
          kreg[u][kc] = *reinterpret_cast<const uint4*>(st + r * RB + ((ch ^ (r & (CPR - 1))) * 16));
        }
      }
      // The PV product runs over all 32 keys at once (16x16x32). Its k index 8 grp + i stands
      // for key 4 grp + i (i < 4) or 16 + 4 grp + i - 4: exactly the keys this lane's two S^T
      // halves hold, so P needs no lane exchange; V^T is read in the same key order.
      // Transposing LDS reads (ds_read_b64_tr_b16): in each 16-lane group, lane j = 4k + r
      // points at dims 16 mt + 4r .. +3 of key 4 grp + k, and lane i16 receives dim
      // 16 mt + i16 of keys 4 grp + 0..3 (then the same 16 keys later).
      uint4 vt[MT];
      const int vrow = 4 * grp + (i16 >> 2), vs = P::vsw(vrow);  // rows vrow and vrow + 16 share vsw
      const char* vb = st + P::TILE + vrow * RB + (i16 & 3) * 8;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int so = ((2 * mt) ^ vs) * 16;
        const uint2 lo = lds_tr16(vb + so);
        const uint2 hi = lds_tr16(vb + 16 * RB + so);
        vt[mt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
      // The 8 keys of this lane's S^T halves: 4 grp + kr[i]. kok[i]: that key lies in a valid
      // block (read per key only when some key of the tile does not).
      constexpr int kr[8] = {0, 1, 2, 3, 16, 17, 18, 19};
      const bool allok = __builtin_amdgcn_readfirstlane(s_wok[stage]) == 0x01010101u;
      bool kok[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) kok[i] = true;
      if (!allok) {
#pragma unroll
        for (int i = 0; i < 8; ++i) kok[i] = s_ok[stage][32 * h + 4 * grp + kr[i]] != 0;
      }
      // Every column block's raw scores first, then one wave-uniform masking test and one
      // rescale test for all of them, so that the exponentials and PV products of all blocks
      // form one straight-line region the scheduler can interleave. Masked scores become -inf;
      // only steps with a key past some row's position or in an invalid block need that.
      float sv[NC][8];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        f32x4_t s0 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
          s0 = Ops::qk(kreg[0][kc], qreg[c][kc], s0);
          s1 = Ops::qk(kreg[1][kc], qreg[c][kc], s1);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) sv[c][i] = i < 4 ? s0[i] : s1[i - 4];
      }
      if (!(allok && key0 + 31 <= pmin_all)) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          // Key key0 + kr[i] + 4 grp is visible to this lane's row when kr[i] <= lim.
          const int lim = pos[c] - key0 - 4 * grp;
#pragma unroll
          for (int i = 0; i < 8; ++i) sv[c][i] = (kok[i] && kr[i] <= lim) ? sv[c][i] : -INFINITY;
        }
      }
      // The rescale test on each lane's maximum of raw scores, against a threshold in raw
      // units (the scale is positive).
      float mx[NC];
      bool need = false;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        mx[c] = fmax3(fmax3(sv[c][0], sv[c][1], sv[c][2]), fmax3(sv[c][3], sv[c][4], sv[c][5]),
                      fmax2(sv[c][6], sv[c][7]));
        need = need || mx[c] > mth[c];
      }
      if (__any(need)) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          if (__any(mx[c] > mth[c])) {
            const float mn = fmax2(m[c], max4(mx[c]) * a.scale_log2);
            const float alpha = (m[c] == -INFINITY) ? 0.0f : fast_exp2(m[c] - mn);
            lacc[c] *= alpha;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[c][mt] *= alpha;
            m[c] = mn;
            mth[c] = (mn + kRescaleLog2) / a.scale_log2;
            // exp2(-inf - m) = 0 for any finite m; m stays -inf only while every score of the
            // row so far is -inf, and then exp2(-inf - 0) = 0 as well.
            nm[c] = mn == -INFINITY ? 0.0f : -mn;
          }
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float pr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pr[i] = fast_exp2(fmaf(sv[c][i], a.scale_log2, nm[c]));
        uint4 ph;
        ph.x = OpsV::pack2(pr[0], pr[1]);
        ph.y = OpsV::pack2(pr[2], pr[3]);
        ph.z = OpsV::pack2(pr[4], pr[5]);
        ph.w = OpsV::pack2(pr[6], pr[7]);
        // Row sums of the weights the PV product uses, on the matrix cores.
        constexpr uint32_t kOne2 = DT == MIP_BF16 && !VF16 ? 0x3f803f80u : 0x3c003c00u;
        const uint4 ones = make_uint4(kOne2, kOne2, kOne2, kOne2);
        lacc[c] = OpsV::qk(ones, ph, lacc[c]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[c][mt] = OpsV::qk(vt[mt], ph, acc[c][mt]);
        if constexpr (kSplitP<DT, VF16>) {
          // bf16 keeps only 8 bits of p: add the rounding remainder as a second product.
          uint4 pl;
          pl.x = Ops::pack2(pr[0] - Ops::lo(ph.x), pr[1] - Ops::hi(ph.x));
          pl.y = Ops::pack2(pr[2] - Ops::lo(ph.y), pr[3] - Ops::hi(ph.y));
          pl.z = Ops::pack2(pr[4] - Ops::lo(ph.z), pr[5] - Ops::hi(ph.z));
          pl.w = Ops::pack2(pr[6] - Ops::lo(ph.w), pr[7] - Ops::hi(ph.w));
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[c][mt] = Ops::qk(vt[mt], pl, acc[c][mt]);
          lacc[c] = Ops::qk(ones, pl, lacc[c]);
        }
      }
    }
    }
    if (t + 1 < n_tiles) stash(stage ^ 1);
    __syncthreads();
  }
  if constexpr (VF16) {
    // maximum() propagates NaN, so mxa < inf fails for any inf or NaN accumulator.
    float mxa = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        mxa = fmax3(mxa, fmax2(fabsf(acc[c][mt][0]), fabsf(acc[c][mt][1])),
                    fmax2(fabsf(acc[c][mt][2]), fabsf(acc[c][mt][3])));
    if (__any(!(mxa < INFINITY)) && lane == 0) *s_big = tag;
    __syncthreads();
    const bool redo = __builtin_amdgcn_readfirstlane(*s_big) == tag;
    // Every thread reads the flag before any stages the next item (which may store to it).
    __syncthreads();
    if (redo) return true;
  }

  // ---- normalise and write each live row: lane (row i16, group grp) holds d = 16 mt + 4 grp + 0..3.
  using S = typename Elem<DT>::S;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float lt = lacc[c][0];
    if (!live[c]) continue;
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int r = (w * NC + c) * 16 + i16;
    const int tr = r / G, g = r - tr * G;
    const int tok = tok_lo + tr;
    S* orow = reinterpret_cast<S*>(a.out) + (static_cast<int64_t>(q0) + tok) * a.out_st +
              static_cast<int64_t>(kvh * G + g) * a.out_sh;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint32_t w0 = Ops::pack2(acc[c][mt][0] * inv, acc[c][mt][1] * inv);
      const uint32_t w1 = Ops::pack2(acc[c][mt][2] * inv, acc[c][mt][3] * inv);
      *reinterpret_cast<uint2*>(orow + 16 * mt + 4 * grp) = make_uint2(w0, w1);
    }
  }
  return false;
}

struct ItemArgs {
  int kvh, s, q0, n_s, start, tok_lo, tok_end;
};

// One work item, as prefill_item describes: bf16 items with V staged as fp16 first, and again
// with bf16 V where that finds a value fp16 cannot hold. args() yields the item's arguments;
// it is called again for the second pass, so nothing but what args() reads stays live across
// the first.
template <int DT, int D, int NC, class Args>
__device__ __forceinline__ void run_item(const PrefillArgs& a, const Args& args, uint32_t tag, char* smem,
                                         uint8_t (*s_ok)[kKT], uint32_t* s_wok, uint32_t* s_big) {
  if constexpr (DT == MIP_BF16) {
    const ItemArgs x = args();
    if (!prefill_item<DT, D, NC, true>(a, x.kvh, x.s, x.q0, x.n_s, x.start, x.tok_lo, x.tok_end, tag, smem, s_ok,
                                       s_wok, s_big))
      return;
  }
  const ItemArgs x = args();
  prefill_item<DT, D, NC, false>(a, x.kvh, x.s, x.q0, x.n_s, x.start, x.tok_lo, x.tok_end, tag, smem, s_ok, s_wok,
                                 s_big);
}

// Work list of the persistent kernel, built in LDS by every workgroup from cu_q: sequences
// sorted by their number of TQ-token blocks (descending), and the items ordered by block
// index, highest first (later tokens see more keys), then by sorted sequence, then kv head,
// so the longest items start first. Limits: kMaxSeqs sequences, kMaxLevels blocks each.
constexpr int kMaxSeqs = 1024;
constexpr int kMaxLevels = 255;

// Two wavefronts per SIMD is the occupancy the register file allows at these tile sizes;
// saying so lets the compiler use up to 256 registers instead of spilling.
template <int DT, int D, int NC, bool PERSIST>
__global__ __launch_bounds__(kPW * kWave) __attribute__((amdgpu_waves_per_eu(2, 2))) void paged_prefill_kernel(
    PrefillArgs a) {
  using P = PShape<D>;
  const int TQ = a.tq;
  __shared__ __attribute__((aligned(16))) char smem[2 * P::STAGE];
  __shared__ uint8_t s_ok[2][kKT];
  __shared__ uint32_t s_wok[2];
  __shared__ uint32_t s_big;  // tag of an item to run again with bf16 V (bf16 only)
  static_assert(kPW == 4, "one byte per wavefront in s_wok");
  if constexpr (!PERSIST) {
    // One workgroup per (kv head, sequence, block), blocks of a sequence latest first.
    if constexpr (DT == MIP_BF16) {
      if (threadIdx.x == 0) s_big = 0;
      __syncthreads();
    }
    auto args = [&]() __attribute__((always_inline)) {
      const int blk = gridDim.z - 1 - blockIdx.z, s = blockIdx.y;
      const int q0 = a.cu_q[s];
      return ItemArgs{static_cast<int>(blockIdx.x), s, q0, a.cu_q[s + 1] - q0, a.ctx_start[s], blk * TQ, blk * TQ + TQ};
    };
    run_item<DT, D, NC>(a, args, 1u, smem, s_ok, s_wok, &s_big);
  } else {
    __shared__ int s_cu[kMaxSeqs + 1];      // cu_q
    __shared__ int s_st[kMaxSeqs];          // ctx_start
    __shared__ int s_nb[kMaxSeqs];          // blocks of sequence s
    __shared__ int s_seq[kMaxSeqs];         // sequences by blocks, descending
    __shared__ int s_cnt[kMaxLevels + 1];   // histogram: sequences with v blocks
    __shared__ int s_gt[kMaxLevels + 1];    // sequences with more than v blocks
    __shared__ int s_fill[kMaxLevels + 1];
    __shared__ int s_ipre[kMaxLevels + 1];  // first item of the k-th level, highest level first
    const int S = a.num_seqs, zb = a.zb;
    // One wavefront builds the list with wavefront scans (no workgroup barrier until it is
    // done); LDS operations of one wavefront take effect in program order.
    if (threadIdx.x < kWave) {
      const int lane = threadIdx.x;
      for (int v = lane; v <= zb; v += kWave) {
        s_cnt[v] = 0;
        s_fill[v] = 0;
      }
      for (int q = lane; q < S; q += kWave) {
        const int c0 = a.cu_q[q], c1 = a.cu_q[q + 1];
        s_cu[q] = c0;
        s_st[q] = a.ctx_start[q];
        if (q == S - 1) s_cu[S] = c1;
        const int n = c1 - c0;
        int nb = n > 0 ? (n + TQ - 1) / TQ : 0;
        nb = nb < zb ? nb : zb;
        s_nb[q] = nb;
        atomicAdd(&s_cnt[nb], 1);
      }
      // s_gt[v] = sum of s_cnt[u] over u > v, bins taken from the top (s_gt[zb] = 0).
      int carry = 0;
      for (int base = 0; base <= zb; base += kWave) {
        const int v = zb - base - lane;
        const int c = v >= 0 && v < zb ? s_cnt[v + 1] : 0;
        const int incl = decode::wave_inclusive_scan(c, lane) + carry;
        if (v >= 0) s_gt[v] = incl;
        carry = __shfl(incl, kWave - 1);
      }
      // Sequences with nb blocks take places s_gt[nb] onwards (descending by blocks).
      for (int q = lane; q < S; q += kWave) {
        const int nb = s_nb[q];
        s_seq[s_gt[nb] + atomicAdd(&s_fill[nb], 1)] = q;
      }
      // Items of level lv = zb - 1 - k (k-th from the top): one per (sequence with more than
      // lv blocks, kv head).
      carry = 0;
      for (int base = 0; base < zb; base += kWave) {
        const int k = base + lane;
        const int items = k < zb ? s_gt[zb - 1 - k] * a.hkv : 0;
        const int incl = decode::wave_inclusive_scan(items, lane) + carry;
        if (k < zb) s_ipre[k + 1] = incl;
        carry = __shfl(incl, kWave - 1);
      }
      if (lane == 0) {
        s_ipre[0] = 0;
        s_big = 0;
      }
    }
    __syncthreads();
    const int total = s_ipre[zb];
    // Item it of the list: (sequence, kv head, block of TQ tokens).
    auto item = [&](int it, int& seq, int& kvh, int& blk) __attribute__((always_inline)) {
      int lo = 0, hi = zb - 1;  // the level k with s_ipre[k] <= it < s_ipre[k + 1]
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_ipre[mid] <= it) lo = mid; else hi = mid - 1;
      }
      const int rem = it - s_ipre[lo];
      seq = __builtin_amdgcn_readfirstlane(s_seq[rem / a.hkv]);
      kvh = __builtin_amdgcn_readfirstlane(rem % a.hkv);
      blk = __builtin_amdgcn_readfirstlane(zb - 1 - lo);
    };
    // Whole rounds of gridDim.x items. Workgroups b and b + G/2 share a CU (the grid is two
    // workgroups per CU, dispatched one per CU first), and the older one, b, issues first and
    // runs faster while both are busy. Even rounds go in list order; in odd rounds the first
    // workgroups of the CUs take the longer half of the round in order, and the second ones
    // the shorter half in reverse, so a second workgroup that drew a short item before draws
    // the longest of its half.
    const int G = gridDim.x, wg = static_cast<int>(blockIdx.x), H = G / 2;
    const int full = total / G, last = total - full * G;
    // The arguments of whole item it.
    auto whole = [&](int it) __attribute__((always_inline)) {
      return [&, it]() __attribute__((always_inline)) {
        int seq, kvh, blk;
        item(it, seq, kvh, blk);
        return ItemArgs{kvh, seq, s_cu[seq], s_cu[seq + 1] - s_cu[seq], s_st[seq], blk * TQ, blk * TQ + TQ};
      };
    };
    for (int r = 0; r < full; ++r) {
      const int it = r * G + ((r & 1) && wg >= H ? G - 1 - (wg - H) : wg);
      run_item<DT, D, NC>(a, whole(it), it + 1u, smem, s_ok, s_wok, &s_big);
    }
    if (last == 0) return;
    // The last, partial round holds the shortest items (or, in a call of fewer items than
    // workgroups, all of them) and leaves G - last workgroups idle. Up to that many of its
    // items (the longest first) are cut into two halves of half the column blocks per
    // wavefront, one workgroup each, so the round ends after about half an item where it
    // can. Rows do not depend on one another: halves need no merge. A half does a little
    // more than half the work of its item (every key tile is still staged and walked), so
    // only the idle workgroups take halves; quarters were slower for that reason.
    const int u = (full & 1) ? G - 1 - wg : wg;  // this workgroup's place in the round
    constexpr int NC2 = NC / 2;
    const int tq2 = NC2 > 0 ? kPW * NC2 * 16 / a.group : 0;
    const int n_split = NC2 > 0 && 2 * tq2 >= TQ ? (last < G - last ? last : G - last) : 0;
    if (u >= last + n_split) return;
    if (u < 2 * n_split) {
      if constexpr (NC2 > 0) {
        const int it = full * G + u / 2;
        auto half = [&]() __attribute__((always_inline)) {
          int seq, kvh, blk;
          item(it, seq, kvh, blk);
          const int t0 = blk * TQ + (u & 1) * tq2, t_end = blk * TQ + TQ;
          return ItemArgs{kvh, seq, s_cu[seq], s_cu[seq + 1] - s_cu[seq], s_st[seq], t0,
                          t0 + tq2 < t_end ? t0 + tq2 : t_end};
        };
        run_item<DT, D, (NC2 > 0 ? NC2 : 1)>(a, half, it + 1u, smem, s_ok, s_wok, &s_big);
      }
      return;
    }
    const int it = full * G + u - n_split;
    run_item<DT, D, NC>(a, whole(it), it + 1u, smem, s_ok, s_wok, &s_big);
  }
}

template <int D> constexpr int kNC = MIP_PREFILL_NC > 0 ? MIP_PREFILL_NC : (D == 64 ? 4 : 2);

// Workgroups of the persistent kernel that fit on the device at once (0 on error).
template <int DT, int D, int NC>
int persistent_grid() {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void*>(paged_prefill_kernel<DT, D, NC, true>), kPW * kWave, 0) !=
      hipSuccess)
    return 0;
  return cus * (per_cu > 0 ? per_cu : 1);
}

template <int DT, int D>
int launch_shape(PrefillArgs a, int num_seqs, int max_q_len, hipStream_t s) {
  constexpr int NC = kNC<D>;
  const int TQ = kPW * NC * 16 / a.group;  // group <= 16, so at least one token per item
  const int zb = (max_q_len + TQ - 1) / TQ;
  a.tq = TQ;
  a.num_seqs = num_seqs;
  a.zb = zb;
  // Persistent grid over a longest-first work list where it fits in LDS: a grid with one
  // workgroup per (kv head, sequence, block) leaves most of the device idle when lengths vary,
  // since the workgroups past a sequence's end occupy the dispatcher.
  static const int grid_cap = persistent_grid<DT, D, NC>();
  const int64_t items = static_cast<int64_t>(a.hkv) * num_seqs * zb;
  // A call of fewer items than the device holds workgroups cuts them into halves, so the grid
  // may hold twice as many workgroups.
  const int64_t units = items * 2;
  if (grid_cap > 0 && num_seqs <= kMaxSeqs && zb <= kMaxLevels) {
    const int grid = static_cast<int>(units < grid_cap ? units : grid_cap);
    hipLaunchKernelGGL((paged_prefill_kernel<DT, D, NC, true>), dim3(grid), dim3(kPW * kWave), 0, s, a);
  } else {
    if (num_seqs > 65535 || zb > 65535) return MIP_EUNSUPPORTED;
    hipLaunchKernelGGL((paged_prefill_kernel<DT, D, NC, false>), dim3(a.hkv, num_seqs, zb), dim3(kPW * kWave), 0,
                       s, a);
  }
  return status_from_hip(hipGetLastError());
}

template <int DT>
int launch_dt(const PrefillArgs& a, int d, int num_seqs, int max_q_len, hipStream_t s) {
  return d == 64 ? launch_shape<DT, 64>(a, num_seqs, max_q_len, s) : launch_shape<DT, 128>(a, num_seqs, max_q_len, s);
}

}  // namespace
}  // namespace prefill
}  // namespace mip

using namespace mip;

extern "C" int mip_paged_prefill(void* out, int64_t out_stride_tok, int64_t out_stride_head, const void* q,
                                 int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                                 const void* v_cache, int64_t num_cache_blocks, const int32_t* block_tables,
                                 int64_t bt_stride, const int32_t* cu_q, const int32_t* ctx_start,
                                 int32_t num_seqs, int32_t max_q_len, int32_t num_heads, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq, float scale,
                                 int32_t dtype, void* stream) {
  if (dtype != MIP_F32 && dtype != MIP_F16 && dtype != MIP_BF16) return MIP_EINVAL;
  if (num_seqs < 0 || max_q_len < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return MIP_EINVAL;
  if (head_dim <= 0 || num_cache_blocks <= 0 || max_blocks_per_seq <= 0 || bt_stride < max_blocks_per_seq) return MIP_EINVAL;
  if (!is_pow2(block_size) || block_size > 4096) return MIP_EINVAL;
  if (num_seqs == 0 || max_q_len == 0) return MIP_OK;
  if (!out || !q || !k_cache || !v_cache || !block_tables || !cu_q || !ctx_start) return MIP_EINVAL;
  const int group = num_heads / num_kv_heads;
  if (dtype == MIP_F32 || (head_dim != 64 && head_dim != 128) || group > 16) {
    // Shapes without an MFMA prefill kernel: the VALU decode kernel, one workgroup per
    // (new token, kv head) over that token's keys (per group of at most 8 of its query heads).
    if (num_cache_blocks > INT32_MAX) return MIP_EINVAL;
    return decode::valu_prefill_launch(out, out_stride_tok, out_stride_head, q, q_stride_tok, q_stride_head, k_cache,
                                       v_cache, num_cache_blocks, block_tables, bt_stride, cu_q, ctx_start, num_seqs,
                                       max_q_len, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq,
                                       scale, dtype, static_cast<hipStream_t>(stream));
  }
  // q rows are read and output rows written 16 / 8 bytes at a time.
  const uint64_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
                         static_cast<uint64_t>(q_stride_tok * 2) | static_cast<uint64_t>(q_stride_head * 2) |
                         static_cast<uint64_t>(out_stride_tok * 2) | static_cast<uint64_t>(out_stride_head * 2);
  if (align & 7) return MIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(q) | static_cast<uint64_t>(q_stride_tok * 2) |
       static_cast<uint64_t>(q_stride_head * 2)) & 15)
    return MIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15) return MIP_EINVAL;
  if (num_cache_blocks > INT32_MAX) return MIP_EINVAL;

  prefill::PrefillArgs a{};
  a.out = static_cast<char*>(out);
  a.out_st = out_stride_tok;
  a.out_sh = out_stride_head;
  a.q = static_cast<const char*>(q);
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.k = static_cast<const char*>(k_cache);
  a.v = static_cast<const char*>(v_cache);
  a.ncb = num_cache_blocks;
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  a.cu_q = cu_q;
  a.ctx_start = ctx_start;
  a.hkv = num_kv_heads;
  a.group = group;
  a.bs = block_size;
  a.log2_bs = ilog2_exact(block_size);
  a.max_blocks = max_blocks_per_seq;
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MIP_BF16) return prefill::launch_dt<MIP_BF16>(a, head_dim, num_seqs, max_q_len, s);
  return prefill::launch_dt<MIP_F16>(a, head_dim, num_seqs, max_q_len, s);
}
