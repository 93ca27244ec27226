// Stream-K paged decode attention for gfx950: persistent wavefronts, LDS ring fed by direct
// global->LDS loads, MFMA tiles.
//
// Reference semantics: as paged_decode.hip (engine/kv_cache.py:615-620 gather + mask,
// engine/model.py:126-147 GQA decode attention).
//
// Work split (16-bit K/V, head_dim 64/128, up to 16 query heads per kv head):
//   * The grid is the device's resident capacity, so it is fixed and graph-capturable.
//     Every workgroup copies the clamped context lengths into LDS and scans the per-sequence
//     tile counts (16 keys per tile). Segment (sequence b, kv head) owns tiles
//     [Hkv*P[b] + kvh*n_b, + n_b) of one global tile sequence of T tiles.
//   * Wavefront gw streams tiles [gw*T/W, (gw+1)*T/W): equal shares regardless of how
//     context lengths are distributed, crossing segment boundaries without a pause.
//   * A segment a wavefront covers completely is normalised and written directly. A split
//     segment leaves one record (m, l, unnormalised acc of 16 heads) per piece: slot 0 for
//     the piece holding the wavefront's first tile, slot 1 for its last. The merge kernel
//     combines the pieces.
//
// Memory pipeline (per wavefront, NS stages of K tile | V tile | q block in LDS):
//   * global_load_lds_dwordx4 moves 64 x 16 bytes per instruction straight into LDS, so the
//     loads in flight cost no registers. Stage i+NS-1 is issued before stage i is consumed.
//   * The loop reads the ring only through inline-asm ds_read, after an explicit
//     s_waitcnt vmcnt((NS-1) * loads-per-stage): the compiler cannot tell which ring stage a
//     direct load fills and would otherwise drain every load before each LDS read. Block
//     tables and context lengths are read with scalar loads, and cross-lane sums use
//     v_permlane{16,32}_swap, so nothing else in the loop touches LDS.
//   * K and q rows are stored with their 16-byte chunks XOR-swizzled by row, so the 16 rows
//     read by one ds_read_b128 hit distinct banks. V rows are swizzled by an even XOR (whole
//     32-byte segments) and read with gfx950's transposing ds_read_b64_tr_b16 (4 keys of one
//     dim per lane, one read per 16 dims), so its rows too start in distinct banks.
//
// Tile arithmetic (lane l: row/head l%16, lane group l/16):
//   S^T[16 keys x 16 heads] = K . Q^T        v_mfma_f32_16x16x32_{bf16,f16}, D/32 steps
//   O^T[D x 16 heads]      += V^T . P^T      v_mfma_f32_16x16x32_{bf16,f16}, D/16 M-tiles,
//   P^T is the S^T output layout (kept in registers), split into hi + lo 16-bit parts so the
//   PV product keeps ~fp32 precision: the 32-deep k index runs over the lane group's 4 keys
//   twice, V^T against hi and again against lo. Online softmax in base 2 with a per-head running max
//   that is only raised when a key exceeds it by more than kRescaleLog2.
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <vector>

#include "paged_decode_common.h"

namespace mip {
namespace decode {
namespace {

#ifndef MIP_STREAM_WAVES
#define MIP_STREAM_WAVES 4
#endif
#ifndef MIP_STREAM_STAGES_D64
#define MIP_STREAM_STAGES_D64 3
#endif
#ifndef MIP_STREAM_STAGES_D128
#define MIP_STREAM_STAGES_D128 3
#endif
#ifndef MIP_STREAM_PRIO
#define MIP_STREAM_PRIO 1
#endif
#ifndef MIP_STREAM_MAX_PIECES
#define MIP_STREAM_MAX_PIECES 64
#endif
constexpr int kSW = MIP_STREAM_WAVES;   // wavefronts per workgroup
constexpr int kStreamMaxBatch = 4096;   // context lengths + tile prefix fit in LDS

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;
typedef __attribute__((address_space(3))) char lchar_t;

template <int D, int QR>
struct Ring {
  static constexpr int RB = D * 2;              // bytes per key / value / query row
  static constexpr int CPR = RB / 16;           // 16-byte chunks per row
  static constexpr int RPD = 1024 / RB;         // rows per direct load (64 lanes x 16 bytes)
  static constexpr int KI = 16 * RB / 1024;     // direct loads per 16-row K (or V) tile
  static constexpr int QI = QR * RB / 1024;     // direct loads per q block of QR heads
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = 16 * RB;
  static constexpr int Q_OFF = 32 * RB;
  static constexpr int STAGE = (32 + QR) * RB;
  static constexpr int DMA = 2 * KI + QI;       // direct loads per stage (static)
  static constexpr int KC = D / 32;
  static constexpr int MT = D / 16;
  static_assert(QI >= 1, "q block must fill at least one direct load");
  // V row r keeps its 16-byte chunk c at c ^ vsw(r). The XOR is even, so each 32-byte segment a
  // transposing read takes stays whole, and the 8 rows one 32-lane half of such a read touches
  // start their segments in distinct banks (the layout of the prefill kernel's V tile).
  static __device__ __forceinline__ int vsw(int r) { return CPR >= 16 ? 2 * (r & 7) : 2 * ((r + (r >> 2)) & 3); }
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  // gfx9 s_waitcnt: vmcnt [3:0] and [15:14], expcnt [6:4] (7 = no wait), lgkmcnt [11:8] (15 = no wait).
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void dma16(const char* g, lchar_t* l) {
  __builtin_amdgcn_global_load_lds((gvoid_t*)g, (lvoid_t*)l, 16, 0, 0);
}
// K/V tile rows are read once per call: direct loads with the nontemporal cache policy (the
// instruction's nt bit, cache-policy operand 2), which streams a 160 MB read of randomly placed
// 2 KiB tiles about 10 % faster on gfx950 than the default policy.
#ifndef MIP_KV_CPOL
#define MIP_KV_CPOL 2
#endif
__device__ __forceinline__ void dma16_kv(const char* g, lchar_t* l) {
  __builtin_amdgcn_global_load_lds((gvoid_t*)g, (lvoid_t*)l, 16, 0, MIP_KV_CPOL);
}

template <int OFF>
__device__ __forceinline__ u32x4_t lds_b128(uint32_t addr) {
  u32x4_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
// Transposing read (ds_read_b64_tr_b16): within each 16-lane group, lane j supplies the
// address of 4 consecutive 16-bit elements A[j][0..3], and lane i receives A[i / 4][i % 4],
// A[4 + i / 4][i % 4], A[8 + i / 4][i % 4], A[12 + i / 4][i % 4] (layout measured on gfx950).
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
template <int OFF>
__device__ __forceinline__ u32x2_t lds_tr16(uint32_t addr) {
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
// Wait for the asm LDS reads, then pass each destination through an empty asm so every use
// of it is ordered after the wait.
__device__ __forceinline__ void lgkm_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void after_wait(u32x4_t& r) { asm volatile("" : "+v"(r)); }
__device__ __forceinline__ void after_wait(uint32_t& r) { asm volatile("" : "+v"(r)); }
__device__ __forceinline__ void after_wait(u32x2_t& r) { asm volatile("" : "+v"(r)); }

// Sum / max over the four lanes l, l^16, l^32, l^48 with VALU lane swaps.
__device__ __forceinline__ float sum4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float max4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

template <int V>
using ic = std::integral_constant<int, V>;

// Call f(ic<I>{}) for I = B .. E-1 (compile-time loop, for immediates such as LDS offsets).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(ic<B>{});
    static_for<B + 1, E>(f);
  }
}

// Call f(ic<I>{}) for I = B .. E-1 in order until one returns false; returns whether all did.
template <int B, int E, typename F>
__device__ __forceinline__ bool static_all(F&& f) {
  if constexpr (B < E) {
    if (!f(ic<B>{})) return false;
    return static_all<B + 1, E>(f);
  }
  return true;
}

template <int DT, int D, int QR, int NS, bool FUSED>
__global__ __launch_bounds__(kSW * kWave) void paged_decode_stream(const int32_t*, int32_t, int32_t, StreamArgs sa) {
  using R = Ring<D, QR>;
  using Ops = MfmaOps<DT>;
  using S = typename Elem<DT>::S;
  constexpr int KC = R::KC, MT = R::MT, RB = R::RB, CPR = R::CPR, RPD = R::RPD;
  constexpr int RING = NS * R::STAGE;
  const DecodeArgs& a = sa.a;
  const int B = sa.batch, G = sa.group;
  extern __shared__ __attribute__((aligned(16))) char dsm[];
  int* s_len = reinterpret_cast<int*>(dsm);  // [B] clamped context lengths
  int* s_pre = s_len + B;                     // [B + 1] exclusive tile prefix over sequences
  int* s_wtot = s_pre + B + 1;                // [kSW] per-wavefront scan totals

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int i16 = lane & 15, grp = lane >> 4;
  const int cap = a.max_blocks * a.bs;

  const AppendRows& ap = sa.app;

  auto seq_len = [&](int b) __attribute__((always_inline)) {
    int L = load_uniform_i32(a.lens + b);
    L = L < cap ? L : cap;
    return L > 0 ? L : 0;
  };
  const int gw = blockIdx.x * kSW + w;
  int lo = 0, hi = 0, cb = 0, ckvh = 0, ct = 0, cL = 0;
  // ---- work split: context lengths -> tile prefix (block-wide exclusive scan).
  for (int i = tid; i < B; i += kSW * kWave) {
    int L = a.lens[i];
    L = L < cap ? L : cap;
    s_len[i] = L > 0 ? L : 0;
  }
  __syncthreads();
  {
    const int chunk = (B + kSW * kWave - 1) / (kSW * kWave);
    const int beg = tid * chunk < B ? tid * chunk : B;
    const int end = beg + chunk < B ? beg + chunk : B;
    int sum = 0;
    for (int i = beg; i < end; ++i) sum += (s_len[i] + 15) >> 4;
    const int incl = wave_inclusive_scan(sum, lane);
    if (lane == kWave - 1) s_wtot[w] = incl;
    __syncthreads();
    int off = 0;
    for (int j = 0; j < w; ++j) off += s_wtot[j];
    int run = off + incl - sum;
    for (int i = beg; i < end; ++i) {
      s_pre[i] = run;
      run += (s_len[i] + 15) >> 4;
    }
    if (tid == kSW * kWave - 1) s_pre[B] = off + incl;
  }
  __syncthreads();
  const int total = a.hkv * s_pre[B];
  if (blockIdx.x == 0) {
    for (int i = tid; i <= B; i += kSW * kWave) sa.ws_prefix[i] = s_pre[i];
  }
  const int tw = stream_active_waves(sa.tw, total, sa.min_tiles, static_cast<int64_t>(sa.batch) * a.hkv, sa.max_pieces);
  const bool active = total > 0 && gw < tw;
  if (active) {
    lo = static_cast<int>(static_cast<int64_t>(gw) * total / tw);
    hi = static_cast<int>(static_cast<int64_t>(gw + 1) * total / tw);
    int lb = 0, ub = B - 1;  // largest b with Hkv * P[b] <= lo; its segment is not empty
    while (lb < ub) {
      const int mid = (lb + ub + 1) >> 1;
      if (a.hkv * __builtin_amdgcn_readfirstlane(s_pre[mid]) <= lo) lb = mid; else ub = mid - 1;
    }
    cb = lb;
    const int n = __builtin_amdgcn_readfirstlane((s_len[cb] + 15) >> 4);
    const int rem = lo - a.hkv * __builtin_amdgcn_readfirstlane(s_pre[cb]);
    ckvh = rem / n;
    ct = rem - ckvh * n;
  }
  __syncthreads();  // the rings below reuse the scan area
  if (!active || lo >= hi) return;
  cL = seq_len(cb);
  int cn = (cL + 15) >> 4;
  int pb = cb, pkvh = ckvh, pt = ct, pL = cL, pn = cn;  // producer cursor (next tile to load)
  // Fused append: the new token's slot of the producer's sequence, fetched when the producer
  // enters the sequence so it has arrived by the sequence's last tile.
  int64_t p_slot = FUSED ? load_uniform_i64(ap.slots + pb) : -1;
  auto advance = [&](int& b_, int& kvh_, int& t_, int& L_, int& n_) __attribute__((always_inline)) {
    if (++t_ < n_) return;
    t_ = 0;
    if (++kvh_ < a.hkv) return;
    kvh_ = 0;
    do {
      ++b_;
      L_ = b_ < B ? seq_len(b_) : 16;
      n_ = (L_ + 15) >> 4;
    } while (n_ == 0);
  };

  // ---- per-lane LDS addresses (ring base of this wavefront; stage offsets are immediates).
  lchar_t* lds = (lchar_t*)(dsm);  // address-space cast: generic -> LDS
  lchar_t* ring_ptr = lds + w * RING;
  const uint32_t ring = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring_ptr));
  uint32_t k_addr[KC], q_addr[KC];
  const int qrow = i16 & (QR - 1);
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    const int c = 4 * kc + grp;
    k_addr[kc] = ring + R::K_OFF + i16 * RB + ((c ^ (i16 & (CPR - 1))) * 16);
    q_addr[kc] = ring + R::Q_OFF + qrow * RB + ((c ^ (qrow & (CPR - 1))) * 16);
  }
  // V^T operand by transposing reads: lane i16 = 4k + r points at dims 4r .. 4r + 3 (+16 mt) of
  // key 4 grp + k and receives dim 16 mt + i16 of keys 4 grp + 0..3. Segment mt of the lane's
  // row sits at chunk (2 mt) ^ vsw(row).
  uint32_t v_addr[MT];
  {
    const int vrow = 4 * grp + (i16 >> 2), vs = R::vsw(vrow);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      v_addr[mt] = ring + R::V_OFF + vrow * RB + (((2 * mt) ^ vs) * 16) + (i16 & 3) * 8;
  }
  const int dma_r = lane / CPR, dma_pc = lane % CPR;

  uint32_t vmask[NS];  // per stage: bit r = key row r of the tile is a key of its segment

  auto produce = [&](auto stage_c, auto scalar_table) __attribute__((always_inline)) {
    constexpr int s = decltype(stage_c)::value;
    lchar_t* st = ring_ptr + s * R::STAGE;
    const int tb = 16 * pt;
    const int32_t* table = a.bt + static_cast<int64_t>(pb) * sa.bt_stride;
    if constexpr (decltype(scalar_table)::value) {
      // block_size >= 16: the tile lies in one block.
      const int blk = load_uniform_i32(table + (tb >> a.log2_bs));
      const bool bok = blk >= 0 && blk < sa.ncb;
      const int rem = pL - tb;
      const int nvalid = bok ? (rem < 16 ? rem : 16) : 0;
      vmask[s] = nvalid >= 16 ? 0xffffu : ((1u << nvalid) - 1u);
      const int64_t row0 = static_cast<int64_t>((bok ? blk : 0) * a.hkv + pkvh) * a.bs + (tb & (a.bs - 1));
      // The segment's last tile holds the newest key (position pL - 1); with a fused append
      // whose slot is that key's slot, its row comes from the new-row source.
      int nr = -1;
      if (FUSED && pt == pn - 1 && bok) {
        const int64_t want = static_cast<int64_t>(blk) * a.bs + ((pL - 1) & (a.bs - 1));
        if (p_slot == want) nr = pL - 1 - tb;
      }
      const char* nk = ap.k + static_cast<int64_t>(pb) * ap.k_st + static_cast<int64_t>(pkvh) * ap.k_sh;
      const char* nv = ap.v + static_cast<int64_t>(pb) * ap.v_st + static_cast<int64_t>(pkvh) * ap.v_sh;
#pragma unroll
      for (int j = 0; j < R::KI; ++j) {
        const int r = j * RPD + dma_r;
        const int64_t row = row0 + (r < nvalid ? r : 0);
        const int lc = dma_pc ^ (r & (CPR - 1)), vc = dma_pc ^ R::vsw(r);
        const bool fresh = r == nr;
        dma16_kv(fresh ? nk + lc * 16 : a.k + row * RB + lc * 16, st + R::K_OFF + j * 1024);
        dma16_kv(fresh ? nv + vc * 16 : a.v + row * RB + vc * 16, st + R::V_OFF + j * 1024);
      }
    } else {
      // Small blocks: every row looks its block up; rows that are not keys re-read the
      // tile's first key (block 0 if even that id is out of range, which the mask drops).
      const int tk0 = tb;
      const int b0 = table[tk0 >> a.log2_bs];
      const bool ok0 = b0 >= 0 && b0 < sa.ncb;
      const int64_t row_first = static_cast<int64_t>((ok0 ? b0 : 0) * a.hkv + pkvh) * a.bs + (tk0 & (a.bs - 1));
      {
        const int tok = tb + i16;
        const int bl = table[(tok < pL ? tok : tk0) >> a.log2_bs];
        const bool ok = tok < pL && bl >= 0 && bl < sa.ncb;
        vmask[s] = static_cast<uint32_t>(__ballot(ok)) & 0xffffu;
      }
      const int64_t new_slot = (FUSED && pt == pn - 1) ? p_slot : -1;
      const char* nk = ap.k + static_cast<int64_t>(pb) * ap.k_st + static_cast<int64_t>(pkvh) * ap.k_sh;
      const char* nv = ap.v + static_cast<int64_t>(pb) * ap.v_st + static_cast<int64_t>(pkvh) * ap.v_sh;
#pragma unroll
      for (int j = 0; j < R::KI; ++j) {
        const int r = j * RPD + dma_r;
        const int tok = tb + r;
        const int bl = table[(tok < pL ? tok : tk0) >> a.log2_bs];
        const bool ok = tok < pL && bl >= 0 && bl < sa.ncb;
        const int64_t row = ok ? static_cast<int64_t>(bl * a.hkv + pkvh) * a.bs + (tok & (a.bs - 1)) : row_first;
        const int lc = dma_pc ^ (r & (CPR - 1)), vc = dma_pc ^ R::vsw(r);
        const bool fresh = ok && tok == pL - 1 && static_cast<int64_t>(bl) * a.bs + (tok & (a.bs - 1)) == new_slot;
        dma16_kv(fresh ? nk + lc * 16 : a.k + row * RB + lc * 16, st + R::K_OFF + j * 1024);
        dma16_kv(fresh ? nv + vc * 16 : a.v + row * RB + vc * 16, st + R::V_OFF + j * 1024);
      }
    }
#pragma unroll
    for (int j = 0; j < R::QI; ++j) {
      const int hr = j * RPD + dma_r;
      const int hh = hr < G ? hr : 0;
      const int lc = dma_pc ^ (hr & (CPR - 1));
      dma16(a.q + (static_cast<int64_t>(pb) * sa.q_sb + static_cast<int64_t>(pkvh * G + hh) * sa.q_sh) * 2 + lc * 16,
            st + R::Q_OFF + j * 1024);
    }
  };

  f32x4_t acc[MT];
  u32x4_t qreg[KC];
  float m = -INFINITY, l = 0.0f;
  bool full_start = false;  // the current segment started at its tile 0 in this wavefront
  bool first_seg = true;    // the current segment holds this wavefront's first tile
  const bool live = i16 < G;
  S* out_base = reinterpret_cast<S*>(a.out);

  auto consume = [&](auto stage_c, int i) __attribute__((always_inline)) {
    constexpr int s = decltype(stage_c)::value;
    constexpr int SO = s * R::STAGE;
    wait_vmcnt<(NS - 1) * R::DMA>();
    if (ct == 0 || i == lo) {
      m = -INFINITY;
      l = 0.0f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      full_start = ct == 0;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) qreg[kc] = lds_b128<SO>(q_addr[kc]);
      lgkm_wait();
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) after_wait(qreg[kc]);
    }
    const uint32_t vm = vmask[s];
    u32x4_t kreg[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) kreg[kc] = lds_b128<SO>(k_addr[kc]);
    u32x2_t ve[MT];  // V^T operand: keys 4*grp + 0..3 at dim 16*mt + i16, packed in pairs
    if (vm) {
      static_for<0, MT>([&](auto mtc) {
        constexpr int mt = decltype(mtc)::value;
        ve[mt] = lds_tr16<SO>(v_addr[mt]);
      });
    }
    lgkm_wait();
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) after_wait(kreg[kc]);
    uint32_t vt[MT][2];
    if (vm) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        after_wait(ve[mt]);
        vt[mt][0] = ve[mt][0];
        vt[mt][1] = ve[mt][1];
      }
    }

    f32x4_t st = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      st = Ops::qk(__builtin_bit_cast(uint4, kreg[kc]), __builtin_bit_cast(uint4, qreg[kc]), st);
    float sv[4];
    bool need = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = live && ((vm >> (4 * grp + j)) & 1u);
      sv[j] = ok ? st[j] * a.scale_log2 : -INFINITY;
      need |= sv[j] > m + kRescaleLog2;
    }
    if (__any(need)) {
      const float mx = max4(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
      const float mn = fmaxf(m, mx);
      const float alpha = (m == -INFINITY) ? 0.0f : fast_exp2(m - mn);
      l *= alpha;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] *= alpha;
      m = mn;
    }
    if (vm) {
      // P as hi + lo 16-bit parts: p = hi + lo to ~2^-16 relative (bf16) or better (fp16).
      uint32_t ph[2], pl[2];
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        const float p0 = sv[j] == -INFINITY ? 0.0f : fast_exp2(sv[j] - m);
        const float p1 = sv[j + 1] == -INFINITY ? 0.0f : fast_exp2(sv[j + 1] - m);
        l += p0 + p1;
        ph[j / 2] = Ops::pack2(p0, p1);
        pl[j / 2] = Ops::pack2(p0 - Ops::lo(ph[j / 2]), p1 - Ops::hi(ph[j / 2]));
      }
      // One 16x16x32 product per 16 dims: its k index runs over this lane group's 4 keys
      // twice, V^T repeated against P's rounded part, then against its remainder.
      const uint4 pb = make_uint4(ph[0], ph[1], pl[0], pl[1]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = Ops::qk(make_uint4(vt[mt][0], vt[mt][1], vt[mt][0], vt[mt][1]), pb, acc[mt]);
    }

    if (ct == cn - 1 || i == hi - 1) {
      const float lt = sum4(l);
      if (full_start && ct == cn - 1) {
        if (live) {
          const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
          S* orow = out_base + static_cast<int64_t>(cb) * sa.out_sb + static_cast<int64_t>(ckvh * G + i16) * sa.out_sh;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const uint32_t w0 = Ops::pack2(acc[mt][0] * inv, acc[mt][1] * inv);
            const uint32_t w1 = Ops::pack2(acc[mt][2] * inv, acc[mt][3] * inv);
            *reinterpret_cast<uint2*>(orow + 16 * mt + 4 * grp) = make_uint2(w0, w1);
          }
        }
      } else {
        float* rec = sa.ws_rec + (static_cast<int64_t>(gw) * 2 + (first_seg ? 0 : 1)) * sa.rec_stride;
        if (live) {
          if (grp == 0) {
            rec[i16] = m;
            rec[16 + i16] = lt;
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            *reinterpret_cast<f32x4_t*>(rec + 32 + i16 * D + 16 * mt + 4 * grp) = acc[mt];
        }
      }
      first_seg = false;
    }
  };

  // The producer cursor moves to tile x only while x < hi; past the end it stays on the
  // last tile, which is loaded again so every stage issues the same number of loads.
  auto adv_p = [&](int x) __attribute__((always_inline)) {
    if (x < hi) {
      const int ob = pb;
      advance(pb, pkvh, pt, pL, pn);
      if (FUSED && pb != ob && pb < B) p_slot = load_uniform_i64(ap.slots + pb);
    }
  };
  auto run = [&](auto scalar_table) __attribute__((always_inline)) {
    // Prologue: tiles lo .. lo+NS-2 into stages 0 .. NS-2.
    static_for<0, NS - 1>([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      if constexpr (k > 0) adv_p(lo + k);
      produce(ic<k>{}, scalar_table);
    });
    int i = lo;
#if MIP_STREAM_PRIO
    // Issue priority falls as the wavefront's own range progresses (3 in its first quarter
    // ... 0 in its last). The arbiter otherwise favours older wavefronts, so the ones
    // dispatched last on a CU fall behind and finish long after the rest.
    const int span = hi - lo;
    const int q1 = lo + (span + 3) / 4, q2 = lo + (2 * span + 3) / 4, q3 = lo + (3 * span + 3) / 4;
    int next_q = q1, quarter = 0;
    __builtin_amdgcn_s_setprio(3);
    auto reprioritise = [&]() __attribute__((always_inline)) {
      if (i < next_q) return;
      ++quarter;
      if (quarter == 1) {
        __builtin_amdgcn_s_setprio(2);
        next_q = q2;
      } else if (quarter == 2) {
        __builtin_amdgcn_s_setprio(1);
        next_q = q3;
      } else {
        __builtin_amdgcn_s_setprio(0);
        next_q = hi;
      }
    };
#endif
    // Step on stage k: load tile i+NS-1 into the stage freed last step, then compute tile i.
    auto step = [&](auto kc) __attribute__((always_inline)) -> bool {
      constexpr int k = decltype(kc)::value;
      adv_p(i + NS - 1);
      produce(ic<(k + NS - 1) % NS>{}, scalar_table);
      consume(ic<k>{}, i);
      if (++i >= hi) return false;
      advance(cb, ckvh, ct, cL, cn);
#if MIP_STREAM_PRIO
      reprioritise();
#endif
      return true;
    };
    while (static_all<0, NS>(step)) {
    }
  };
  if (a.bs >= 16) {
    run(std::true_type{});
  } else {
    run(std::false_type{});
  }
  wait_vmcnt<0>();  // no direct load may land in LDS after this wavefront ends
}

// The stream kernel driven by a work plan (block size >= 16): the same split, ring, tile
// arithmetic and records as paged_decode_stream, but every tile's pool row, sequence, kv
// head, valid-key count and segment edges come from the plan's tile descriptors, so the loop
// does no block-table lookups and no cursor arithmetic. A wavefront holds up to 64 of its
// descriptors in registers (one per lane, loaded once) and takes each with a lane read.
template <int DT, int D, int QR, int NS, bool FUSED>
__global__ __launch_bounds__(kSW * kWave) void paged_decode_stream_tiles(const int32_t* __restrict__ plan,
                                                                        int32_t plan_tile_off, int32_t plan_wave_cap,
                                                                        StreamArgs sa) {
  using R = Ring<D, QR>;
  using Ops = MfmaOps<DT>;
  using S = typename Elem<DT>::S;
  constexpr int KC = R::KC, MT = R::MT, RB = R::RB, CPR = R::CPR, RPD = R::RPD;
  constexpr int RING = NS * R::STAGE;
  const DecodeArgs& a = sa.a;
  const int G = sa.group;
  extern __shared__ __attribute__((aligned(16))) char dsm[];

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int i16 = lane & 15, grp = lane >> 4;
  const AppendRows& ap = sa.app;
  const int gw = blockIdx.x * kSW + w;
  // All plan words this wavefront needs are read before any of them is tested, so their
  // latencies overlap. (The wavefront record of a wavefront past W is inside the plan too.)
  // This wavefront's descriptor slots start at a fixed place, so its first 64 descriptors
  // are read together with its range instead of after it.
  // The header's word pairs, the wavefront record and one descriptor per lane go out as one
  // group of loads (load_now_u64: the plan is 8-byte aligned, the record and descriptors sit
  // at even word offsets), so the start-up waits one round trip for all of them.
  const uint64_t* tdesc = reinterpret_cast<const uint64_t*>(plan + plan_tile_off) +
                          static_cast<int64_t>(gw) * plan_wave_cap;
  const uint64_t* plan64 = reinterpret_cast<const uint64_t*>(plan);
  const uint64_t h01 = load_now_u64(plan64 + 0);  // T, W
  const uint64_t h23 = load_now_u64(plan64 + 1);  // batch, kv heads
  const uint64_t h45 = load_now_u64(plan64 + 2);  // descriptor offset, segment-record offset
  const uint64_t h67 = load_now_u64(plan64 + 3);  // descriptor slots per wavefront, 0
  const uint64_t wr = load_now_u64(plan64 + (kPlanHeader + kPlanWave * gw) / 2);
  const uint64_t d64 = load_now_u64(tdesc + lane);
  static_assert(kPlanHeader % 2 == 0 && kPlanWave == 2 && kPlanTileOffWord == 4 && kPlanWaveCapWord == 6,
                "plan header words are read in 8-byte pairs");
  const int pw = uniform_hi(h01), pb = uniform_lo(h23), ph = uniform_hi(h23);
  const int pt = uniform_lo(h45), pc = uniform_lo(h67);
  const int lo = uniform_lo(wr), hi = uniform_hi(wr);
  uint2 dv = make_uint2(static_cast<uint32_t>(d64), static_cast<uint32_t>(d64 >> 32));
  // One field from each 64-byte line of the argument block the first tiles use (q, the pool,
  // the scale, batch and kv heads, the pool's row count and q strides): their loads go out
  // now, beside the plan reads, instead of each line costing one more round trip before the
  // first K/V loads and the first tile's arithmetic.
  asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.scale_log2), "s"(sa.batch), "s"(sa.nrows));
  // A plan made for another batch, kv-head count or layout would index past this call's tensors.
  if ((pb != sa.batch) | (ph != a.hkv) | (pt != plan_tile_off) | (pc != plan_wave_cap) | (gw >= pw) |
      (lo >= hi))
    return;

  // ---- descriptors of tiles cbase .. cbase + 63 in registers (lane j holds tile cbase + j).
  int cbase = lo;
  if (lane >= hi - lo) dv = make_uint2(kTileNoRow, 0u);

  // ---- per-lane LDS addresses (as paged_decode_stream).
  lchar_t* lds = (lchar_t*)(dsm);
  lchar_t* ring_ptr = lds + w * RING;
  const uint32_t ring = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring_ptr));
  uint32_t k_addr[KC], q_addr[KC];
  const int qrow = i16 & (QR - 1);
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    const int c = 4 * kc + grp;
    k_addr[kc] = ring + R::K_OFF + i16 * RB + ((c ^ (i16 & (CPR - 1))) * 16);
    q_addr[kc] = ring + R::Q_OFF + qrow * RB + ((c ^ (qrow & (CPR - 1))) * 16);
  }
  // V^T operand by transposing reads: lane i16 = 4k + r points at dims 4r .. 4r + 3 (+16 mt) of
  // key 4 grp + k and receives dim 16 mt + i16 of keys 4 grp + 0..3. Segment mt of the lane's
  // row sits at chunk (2 mt) ^ vsw(row).
  uint32_t v_addr[MT];
  {
    const int vrow = 4 * grp + (i16 >> 2), vs = R::vsw(vrow);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      v_addr[mt] = ring + R::V_OFF + vrow * RB + (((2 * mt) ^ vs) * 16) + (i16 & 3) * 8;
  }
  const int dma_r = lane / CPR, dma_pc = lane % CPR;
  // Lane offsets inside a tile's rows (row r < valid keys; other rows re-read row 0).
  uint32_t k_lane[R::KI], v_lane[R::KI];
  int r_lane[R::KI];
#pragma unroll
  for (int j = 0; j < R::KI; ++j) {
    const int r = j * RPD + dma_r;
    r_lane[j] = r;
    k_lane[j] = static_cast<uint32_t>(r * RB + ((dma_pc ^ (r & (CPR - 1))) * 16));
    v_lane[j] = static_cast<uint32_t>(r * RB + ((dma_pc ^ R::vsw(r)) * 16));
  }
  uint32_t q_lane[R::QI];
#pragma unroll
  for (int j = 0; j < R::QI; ++j) {
    const int hr = j * RPD + dma_r;
    const int hh = hr < G ? hr : 0;
    q_lane[j] = static_cast<uint32_t>(hh * sa.q_sh * 2 + ((dma_pc ^ (hr & (CPR - 1))) * 16));
  }

  uint32_t vmask[NS];  // per stage: bit r = key row r of the tile is a key of its segment
  uint32_t smeta[NS];  // per stage: the tile's meta word (valid count corrected)

  // Stage tile x: its K and V rows (2 * KI loads), and the q block of its sequence when the
  // consumer starts a segment there (QI more). Tiles past the range issue nothing; the
  // consumer's waits cover both (see consume).
  auto produce = [&](auto stage_c, int x) __attribute__((always_inline)) {
    constexpr int s = decltype(stage_c)::value;
    lchar_t* st = ring_ptr + s * R::STAGE;
    if (x >= hi) return;
    if (x - cbase >= kWave) {  // next 64 descriptors (long ranges only; drains the loads in flight)
      cbase = x;
      dv = x + lane < hi ? __builtin_bit_cast(uint2, tdesc[x - lo + lane]) : make_uint2(kTileNoRow, 0u);
    }
    const uint32_t row0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(dv.x), x - cbase));
    uint32_t meta = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(dv.y), x - cbase));
    const bool ok = row0 < sa.nrows;
    const int nvalid = ok ? static_cast<int>((meta >> 24) & 31u) : 0;
    meta = (meta & ~(31u << 24)) | (static_cast<uint32_t>(nvalid) << 24);
    smeta[s] = meta;
    vmask[s] = nvalid >= 16 ? 0xffffu : ((1u << nvalid) - 1u);
    const uint64_t tile_off = static_cast<uint64_t>(ok ? row0 : 0u) * RB;
    const char* kb = a.k + tile_off;
    const char* vb = a.v + tile_off;
    const int b = static_cast<int>(meta & 0xffffu), kvh = static_cast<int>((meta >> 16) & 0xffu);
    // Fused append: the segment's last tile holds the newest key (position L - 1); when the new
    // token's slot is that key's slot, its row comes from the new-row source.
    int nr = -1;
    if (FUSED && ((meta >> 30) & 1u) && nvalid > 0) {
      const int64_t slot = load_uniform_i64(ap.slots + b);
      if (slot >= 0 && (slot >> a.log2_bs) < sa.ncb) {  // then every row index below fits 31 bits
        const int s32 = static_cast<int>(slot);
        const int srow = ((s32 >> a.log2_bs) * a.hkv + kvh) * a.bs + (s32 & (a.bs - 1));
        if (static_cast<uint32_t>(srow) == row0 + static_cast<uint32_t>(nvalid - 1)) nr = nvalid - 1;
      }
    }
    if (FUSED && nr >= 0) {
      const char* nk = ap.k + static_cast<int64_t>(b) * ap.k_st + static_cast<int64_t>(kvh) * ap.k_sh;
      const char* nv = ap.v + static_cast<int64_t>(b) * ap.v_st + static_cast<int64_t>(kvh) * ap.v_sh;
#pragma unroll
      for (int j = 0; j < R::KI; ++j) {
        const int r = r_lane[j];
        const bool fresh = r == nr;
        const uint32_t ko = r < nvalid ? k_lane[j] : k_lane[j] - static_cast<uint32_t>(r * RB);
        const uint32_t vo = r < nvalid ? v_lane[j] : v_lane[j] - static_cast<uint32_t>(r * RB);
        dma16_kv(fresh ? nk + (k_lane[j] - r * RB) : kb + ko, st + R::K_OFF + j * 1024);
        dma16_kv(fresh ? nv + (v_lane[j] - r * RB) : vb + vo, st + R::V_OFF + j * 1024);
      }
    } else {
#pragma unroll
      for (int j = 0; j < R::KI; ++j) {
        const int r = r_lane[j];
        const uint32_t ko = r < nvalid ? k_lane[j] : k_lane[j] - static_cast<uint32_t>(r * RB);
        const uint32_t vo = r < nvalid ? v_lane[j] : v_lane[j] - static_cast<uint32_t>(r * RB);
        dma16_kv(kb + ko, st + R::K_OFF + j * 1024);
        dma16_kv(vb + vo, st + R::V_OFF + j * 1024);
      }
    }
    if (((meta >> 29) & 1u) || x == lo) {
      const char* qb = a.q + (static_cast<int64_t>(b) * sa.q_sb + static_cast<int64_t>(kvh * G) * sa.q_sh) * 2;
#pragma unroll
      for (int j = 0; j < R::QI; ++j) dma16(qb + q_lane[j], st + R::Q_OFF + j * 1024);
    }
  };

  f32x4_t acc[MT];
  u32x4_t qreg[KC];
  float m = -INFINITY, l = 0.0f;
  bool full_start = false;  // the current segment started at its tile 0 in this wavefront
  bool first_seg = true;    // the current segment holds this wavefront's first tile
  const bool live = i16 < G;
  S* out_base = reinterpret_cast<S*>(a.out);

  auto consume = [&](auto stage_c, int i) __attribute__((always_inline)) {
    constexpr int s = decltype(stage_c)::value;
    constexpr int SO = s * R::STAGE;
    // Loads complete in issue order. Every later stage issued at least 2 * KI loads, so at most
    // (NS - 1) * 2 * KI outstanding means this stage's loads have landed. Near the end of the
    // range fewer stages follow: wait for everything.
    if (i + NS - 1 < hi) {
      wait_vmcnt<(NS - 1) * 2 * R::KI>();
    } else {
      wait_vmcnt<0>();
    }
    const uint32_t meta = smeta[s];
    const bool seg_first = (meta >> 29) & 1u, seg_last = (meta >> 30) & 1u;
    if (seg_first || i == lo) {
      m = -INFINITY;
      l = 0.0f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      full_start = seg_first;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) qreg[kc] = lds_b128<SO>(q_addr[kc]);
      lgkm_wait();
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) after_wait(qreg[kc]);
    }
    const uint32_t vm = vmask[s];
    u32x4_t kreg[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) kreg[kc] = lds_b128<SO>(k_addr[kc]);
    u32x2_t ve[MT];  // V^T operand: keys 4*grp + 0..3 at dim 16*mt + i16, packed in pairs
    if (vm) {
      static_for<0, MT>([&](auto mtc) {
        constexpr int mt = decltype(mtc)::value;
        ve[mt] = lds_tr16<SO>(v_addr[mt]);
      });
    }
    lgkm_wait();
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) after_wait(kreg[kc]);
    uint32_t vt[MT][2];
    if (vm) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        after_wait(ve[mt]);
        vt[mt][0] = ve[mt][0];
        vt[mt][1] = ve[mt][1];
      }
    }

    f32x4_t st = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      st = Ops::qk(__builtin_bit_cast(uint4, kreg[kc]), __builtin_bit_cast(uint4, qreg[kc]), st);
    float sv[4];
    bool need = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = live && ((vm >> (4 * grp + j)) & 1u);
      sv[j] = ok ? st[j] * a.scale_log2 : -INFINITY;
      need |= sv[j] > m + kRescaleLog2;
    }
    if (__any(need)) {
      const float mx = max4(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
      const float mn = fmaxf(m, mx);
      const float alpha = (m == -INFINITY) ? 0.0f : fast_exp2(m - mn);
      l *= alpha;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] *= alpha;
      m = mn;
    }
    if (vm) {
      uint32_t ph[2], pl[2];
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        const float p0 = sv[j] == -INFINITY ? 0.0f : fast_exp2(sv[j] - m);
        const float p1 = sv[j + 1] == -INFINITY ? 0.0f : fast_exp2(sv[j + 1] - m);
        l += p0 + p1;
        ph[j / 2] = Ops::pack2(p0, p1);
        pl[j / 2] = Ops::pack2(p0 - Ops::lo(ph[j / 2]), p1 - Ops::hi(ph[j / 2]));
      }
      // One 16x16x32 product per 16 dims: its k index runs over this lane group's 4 keys
      // twice, V^T repeated against P's rounded part, then against its remainder.
      const uint4 pb = make_uint4(ph[0], ph[1], pl[0], pl[1]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = Ops::qk(make_uint4(vt[mt][0], vt[mt][1], vt[mt][0], vt[mt][1]), pb, acc[mt]);
    }

    if (seg_last || i == hi - 1) {
      const float lt = sum4(l);
      const int b = static_cast<int>(meta & 0xffffu), kvh = static_cast<int>((meta >> 16) & 0xffu);
      if (full_start && seg_last) {
        if (live) {
          const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
          S* orow = out_base + static_cast<int64_t>(b) * sa.out_sb + static_cast<int64_t>(kvh * G + i16) * sa.out_sh;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const uint32_t w0 = Ops::pack2(acc[mt][0] * inv, acc[mt][1] * inv);
            const uint32_t w1 = Ops::pack2(acc[mt][2] * inv, acc[mt][3] * inv);
            *reinterpret_cast<uint2*>(orow + 16 * mt + 4 * grp) = make_uint2(w0, w1);
          }
        }
      } else {
        float* rec = sa.ws_rec + (static_cast<int64_t>(gw) * 2 + (first_seg ? 0 : 1)) * sa.rec_stride;
        if (live) {
          if (grp == 0) {
            rec[i16] = m;
            rec[16 + i16] = lt;
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            *reinterpret_cast<f32x4_t*>(rec + 32 + i16 * D + 16 * mt + 4 * grp) = acc[mt];
        }
      }
      first_seg = false;
    }
  };

  // Prologue: tiles lo .. lo+NS-2 into stages 0 .. NS-2.
  static_for<0, NS - 1>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    produce(ic<k>{}, lo + k);
  });
  int i = lo;
#if MIP_STREAM_PRIO
  // Tile indices where the priority drops (the quarters of the range), computed once.
  const int span = hi - lo;
  const int q1 = lo + (span + 3) / 4, q2 = lo + (2 * span + 3) / 4, q3 = lo + (3 * span + 3) / 4;
  int next_q = q1, quarter = 0;
  __builtin_amdgcn_s_setprio(3);
  auto reprioritise = [&]() __attribute__((always_inline)) {
    if (i < next_q) return;
    ++quarter;
    if (quarter == 1) {
      __builtin_amdgcn_s_setprio(2);
      next_q = q2;
    } else if (quarter == 2) {
      __builtin_amdgcn_s_setprio(1);
      next_q = q3;
    } else {
      __builtin_amdgcn_s_setprio(0);
      next_q = hi;
    }
  };
#endif
  auto step = [&](auto kc) __attribute__((always_inline)) -> bool {
    constexpr int k = decltype(kc)::value;
    produce(ic<(k + NS - 1) % NS>{}, i + NS - 1);
    consume(ic<k>{}, i);
    if (++i >= hi) return false;
#if MIP_STREAM_PRIO
    reprioritise();
#endif
    return true;
  };
  while (static_all<0, NS>(step)) {
  }
  wait_vmcnt<0>();  // no direct load may land in LDS after this wavefront ends
}

// Pieces per merge chunk (one memory round trip), streams of the merge for calls with few
// segments, and the runs a long segment of such a call is cut into.
constexpr int kMergeChunk = 16;
constexpr int kWideMergeStreams = 2;
constexpr int kStreamParts = 16;

// Combine the pieces of every segment the stream kernel split. Grid (kv heads, batch, runs),
// NSTR * 256 threads: NSTR streams of 256 threads take alternate chunks of 16 pieces (each
// stream with its own online maximum), and stream 0 then combines the streams' states in
// stream order. NSTR = 1 serves batches of many segments (each segment has few pieces);
// NSTR = 2 serves a few long sequences, whose segments have up to a few hundred pieces (two
// streams, not more: each thread keeps a chunk's 16 partial sums and (m, l) pairs per quad in
// registers, and at 1024 threads a thread has 128 registers). With runs > 1 (at most 16
// segments), a segment of more than NSTR chunks is cut into runs of consecutive pieces, one
// workgroup each, whose states paged_decode_stream_fold combines.
template <int DT, int D, bool FUSED, bool PLANNED, int NSTR, int NJ>
__global__ __launch_bounds__(256 * NSTR) void paged_decode_stream_merge(const int32_t* __restrict__ plan,
                                                                       int32_t plan_seg_off, int32_t hkv,
                                                                       StreamArgs sa) {
  using S = typename Elem<DT>::S;
  const int64_t REC = sa.rec_stride;
  const DecodeArgs& a = sa.a;
  const int kvh = blockIdx.x, b = blockIdx.y, G = sa.group;
  // Run z of Z of a parted segment (only the two-stream merge is launched with Z > 1; with one
  // stream the run logic folds away at compile time).
  const int z = NSTR > 1 ? static_cast<int>(blockIdx.z) : 0, Z = NSTR > 1 ? static_cast<int>(gridDim.z) : 1;
  S* out_base = reinterpret_cast<S*>(a.out);
  const int cap = a.max_blocks * a.bs;
  // Fused append: copy sequence b's new K and V rows of this kv head into the pool. The
  // stream kernel, which ran before this one, took the newest key straight from the source,
  // so nothing reads these pool rows in this call. The rows are loaded here and stored once
  // the plan is known to fit the call.
  const AppendRows& ap = sa.app;
  constexpr int CPR = D * 2 / 16;  // 16-byte chunks per row
  const bool app_lane = FUSED && z == 0 && threadIdx.x < 2 * CPR;
  // The plan's header and this segment's descriptor are read first, from the preloaded plan
  // pointer and by vector loads issued as one group (load_now_u64), so the records are read
  // one round trip after the start: the kernel arguments arrive in parallel. The new token's
  // slot and rows are needed only by the store at the end; the row source does not depend on
  // the slot.
  int pb = 0, ph = 0, ps = 0, sd0 = 0, sd1 = 0, sd2 = 0, sd3 = 0;
  if constexpr (PLANNED) {
    // The plan is 8-byte aligned and the segment records start at an even word.
    static_assert(kPlanSegOffWord == 5 && kPlanSeg == 4, "plan words are read in 8-byte pairs");
    const uint64_t* p64 = reinterpret_cast<const uint64_t*>(plan);
    const uint64_t* sd = reinterpret_cast<const uint64_t*>(plan + plan_seg_off) + (static_cast<int64_t>(b) * hkv + kvh) * 2;
    const uint64_t h23 = load_now_u64(p64 + 1), h45 = load_now_u64(p64 + 2);
    const uint64_t s01 = load_now_u64(sd), s23 = load_now_u64(sd + 1);
    pb = uniform_lo(h23);
    ph = uniform_hi(h23);
    ps = uniform_hi(h45);
    sd0 = uniform_lo(s01);
    sd1 = uniform_hi(s01);
    sd2 = uniform_lo(s23);
    sd3 = uniform_hi(s23);
  }
  // The slot is loaded by the append lanes only, as a vector load: a uniform load would be
  // moved to a scalar register (and waited for) at once, and a scalar load would make the
  // next wait for the kernel arguments wait for it as well. Only the store at the end reads it.
  uint64_t slot_raw = ~0ull;
  uint4 app_row = make_uint4(0u, 0u, 0u, 0u);
  if (app_lane) {
    slot_raw = load_now_u64(reinterpret_cast<const uint64_t*>(ap.slots) + b);
    const int side = threadIdx.x / CPR, c = threadIdx.x % CPR;
    const char* src = side ? ap.v + static_cast<int64_t>(b) * ap.v_st + static_cast<int64_t>(kvh) * ap.v_sh
                           : ap.k + static_cast<int64_t>(b) * ap.k_st + static_cast<int64_t>(kvh) * ap.k_sh;
    app_row = *reinterpret_cast<const uint4*>(src + c * 16);
  }
  // The pool geometry the store at the end needs sits in another line of the kernel arguments:
  // read it now, with the rest, rather than one argument load before the kernel can end.
  if constexpr (FUSED) asm volatile("" ::"s"(a.ncb), "s"(a.bs), "s"(a.log2_bs), "s"(a.hkv));
  int L, gw_lo, gw_hi;
  bool lo_split;
  if constexpr (PLANNED) {
    gw_lo = sd0;
    gw_hi = sd0 + sd1 - 1;
    lo_split = sd2 != 0;
    L = sd3;
    // A plan of another shape: the main kernel computed nothing. The call fails visibly:
    // NaN in every output row of this segment, and the pool is left as it was (no append).
    // (Bitwise ors: one test of all the words, after all of them have arrived.)
    if ((pb != sa.batch) | (ph != hkv) | (ps != plan_seg_off) | (gw_lo < 0) | (gw_hi >= sa.tw)) {
      if (z == 0)
        for (int i = threadIdx.x; i < G * D; i += blockDim.x)
          out_base[static_cast<int64_t>(b) * a.out_sb + static_cast<int64_t>(kvh * G + i / D) * a.out_sh + i % D] =
              from_f32<DT>(__builtin_nanf(""));
      return;
    }
  } else {
    L = a.lens[b];
    L = L < cap ? L : cap;
  }
  // The new rows are stored on each way out of the kernel (the workgroup z = 0 of a segment
  // takes one of them), after the record loads are issued: a store of the rows before those
  // loads would make them wait for the rows' load as well.
  auto store_app = [&]() __attribute__((always_inline)) {
    const int64_t slot = static_cast<int64_t>(slot_raw);
    if (app_lane && slot >= 0 && slot < a.ncb * a.bs) {
      const int side = threadIdx.x / CPR, c = threadIdx.x % CPR;
      char* dst = (side ? ap.v_cache : ap.k_cache) +
                  (((slot >> a.log2_bs) * a.hkv + kvh) * a.bs + (slot & (a.bs - 1))) * (D * 2) + c * 16;
      *reinterpret_cast<uint4*>(dst) = app_row;
    }
  };
  if (L <= 0) {
    if (z == 0)
      for (int i = threadIdx.x; i < G * D; i += blockDim.x)
        out_base[static_cast<int64_t>(b) * a.out_sb + static_cast<int64_t>(kvh * G + i / D) * a.out_sh + i % D] =
            from_f32<DT>(0.0f);
    store_app();
    return;
  }
  if constexpr (!PLANNED) {
    const int total = a.hkv * sa.ws_prefix[sa.batch];
    const int tw = stream_active_waves(sa.tw, total, sa.min_tiles, static_cast<int64_t>(sa.batch) * a.hkv, sa.max_pieces);
    const int n = (L + 15) >> 4;
    const int64_t s0 = static_cast<int64_t>(a.hkv) * sa.ws_prefix[b] + static_cast<int64_t>(kvh) * n;
    const int64_t e1 = s0 + n - 1;
    gw_lo = static_cast<int>(((s0 + 1) * tw - 1) / total);
    gw_hi = static_cast<int>(((e1 + 1) * tw - 1) / total);
    lo_split = static_cast<int64_t>(gw_lo) * total / tw < s0;
  }
  if (gw_lo >= gw_hi) {  // one wavefront held the whole segment and wrote it
    store_app();
    return;
  }
  const int R = gw_hi - gw_lo + 1;
  // A segment of more than one round of chunks, with Z > 1, is cut into Z runs of consecutive
  // pieces [p0, p0 + np), one per workgroup z; each leaves its state in a second-level record
  // that paged_decode_stream_fold combines. Otherwise workgroup 0 merges the whole segment.
  const bool parted = Z > 1 && R > NSTR * kMergeChunk;
  int p0 = 0, np = R;
  if (parted) {
    const int P = (R + Z - 1) / Z;
    p0 = z * P;
    if (p0 >= R) return;
    np = R - p0 < P ? R - p0 : P;
  } else if (z > 0) {
    return;
  }
  // Record r of this segment: the first piece sits in the "last segment" slot of wavefront
  // gw_lo when that wavefront started inside an earlier segment, every other piece in the
  // "first segment" slot of its wavefront.
  auto rec_of = [&](int r) -> const float* {
    return sa.ws_rec + (static_cast<int64_t>(gw_lo + r) * 2 + (r == 0 && lo_split ? 1 : 0)) * REC;
  };
  // Passes over chunks of 16 records with an online maximum per row. Every thread owns NJ
  // quads of four output columns of one row (NJ = 2 only where a segment has more than 256
  // quads, 9 to 16 heads at head_dim 128: the registers of a second quad would halve the
  // merge's occupancy everywhere else); the quads' partial sums of a chunk are
  // loaded together with the row's (m, l) pairs, so a chunk costs one memory round trip.
  // Stream str takes chunks str, str + NSTR, ... (a round count uniform over the workgroup,
  // so every thread reaches the barrier of the stream fold below).
  constexpr int kRC = kMergeChunk;
  constexpr int Q = D / 4;  // column quads per row
  const int str = NSTR > 1 ? static_cast<int>(threadIdx.x) / 256 : 0;
  const int t = NSTR > 1 ? static_cast<int>(threadIdx.x) % 256 : static_cast<int>(threadIdx.x);
  const int nq = G * Q;  // quads per (kv head, sequence): at most 512
  float4 acc[NJ];
  float mrun[NJ], lrun[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    mrun[j] = -INFINITY;
    lrun[j] = 0.0f;
  }
  const int rounds = ((np + kRC - 1) / kRC + NSTR - 1) / NSTR;
  // One round as a function, called for the first round outside the loop over the others, so
  // that the common single-round call has no loop-carried state at all.
  auto round = [&](int rd) __attribute__((always_inline)) {
    const int c0 = p0 + (rd * NSTR + str) * kRC;  // first piece of this stream's chunk
    const int nr = c0 >= p0 + np ? 0 : (p0 + np - c0 < kRC ? p0 + np - c0 : kRC);  // 0: no chunk this round
    // Each thread loads its own row's (m, l) pair of every record of the chunk beside the
    // record's partial sums, so the chunk is folded in registers right after its one round
    // trip (no exchange through LDS, no barrier). Records are read once: nontemporal loads.
    float4 v[NJ][kRC];
    float mk[NJ][kRC], lk[NJ][kRC];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int qd = t + 256 * j;
      if (qd < nq) {
        const int g = qd / Q, col = (qd % Q) * 4;
#pragma unroll
        for (int k = 0; k < kRC; ++k)
          if (k < nr) {
            const float* rec = rec_of(c0 + k);
            const f32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(rec + 32 + g * D + col));
            v[j][k] = make_float4(x[0], x[1], x[2], x[3]);
            mk[j][k] = __builtin_nontemporal_load(rec + g);
            lk[j][k] = __builtin_nontemporal_load(rec + 16 + g);
          }
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int qd = t + 256 * j;
      if (nr > 0 && qd < nq) {
        float cm = mrun[j];
#pragma unroll
        for (int k = 0; k < kRC; ++k)
          if (k < nr) cm = fmaxf(cm, mk[j][k]);
        const float alpha = mrun[j] == -INFINITY ? 0.0f : fast_exp2(mrun[j] - cm);
        float4 s = make_float4(acc[j].x * alpha, acc[j].y * alpha, acc[j].z * alpha, acc[j].w * alpha);
        float ls = lrun[j] * alpha;
#pragma unroll
        for (int k = 0; k < kRC; ++k)
          if (k < nr) {
            const float wk = mk[j][k] == -INFINITY ? 0.0f : fast_exp2(mk[j][k] - cm);
            s.x = fmaf(wk, v[j][k].x, s.x);
            s.y = fmaf(wk, v[j][k].y, s.y);
            s.z = fmaf(wk, v[j][k].z, s.z);
            s.w = fmaf(wk, v[j][k].w, s.w);
            ls = fmaf(wk, lk[j][k], ls);
          }
        acc[j] = s;
        lrun[j] = ls;
        mrun[j] = cm;
      }
    }
    // Every load of this round has been folded; saying so lets the next round issue its
    // loads back to back (without it the compiler waits before each one for the same
    // registers' load of the previous round).
    wait_vmcnt<0>();
  };
  round(0);
  for (int rd = 1; rd < rounds; ++rd) round(rd);
  if constexpr (NSTR > 1) {
    // Streams 1.. hand their state to stream 0, which folds them in stream order with weights
    // exp2(m_s - M), M the largest m_s (an empty stream, m = -inf, weighs 0).
    __shared__ float4 s_acc[NSTR - 1][NJ][256];
    __shared__ float2 s_ml[NSTR - 1][NJ][256];
    if (str > 0) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        s_acc[str - 1][j][t] = acc[j];
        s_ml[str - 1][j][t] = make_float2(mrun[j], lrun[j]);
      }
    }
    __syncthreads();
    if (str > 0) return;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float mm = mrun[j];
#pragma unroll
      for (int u = 0; u < NSTR - 1; ++u) mm = fmaxf(mm, s_ml[u][j][t].x);
      const float w0 = mrun[j] == -INFINITY ? 0.0f : fast_exp2(mrun[j] - mm);
      float4 s = make_float4(acc[j].x * w0, acc[j].y * w0, acc[j].z * w0, acc[j].w * w0);
      float ls = lrun[j] * w0;
#pragma unroll
      for (int u = 0; u < NSTR - 1; ++u) {
        const float2 ml = s_ml[u][j][t];
        const float4 a4 = s_acc[u][j][t];
        const float wu = ml.x == -INFINITY ? 0.0f : fast_exp2(ml.x - mm);
        s.x = fmaf(wu, a4.x, s.x);
        s.y = fmaf(wu, a4.y, s.y);
        s.z = fmaf(wu, a4.z, s.z);
        s.w = fmaf(wu, a4.w, s.w);
        ls = fmaf(wu, ml.y, ls);
      }
      acc[j] = s;
      lrun[j] = ls;
      mrun[j] = mm;  // the folded state is relative to mm (a run record stores it)
    }
  }
  if (parted) {
    // Second-level record of run z: m[16] | l[16] | acc[G][D], as the stream kernel's records.
    float* rec = sa.ws_part + ((static_cast<int64_t>(b) * a.hkv + kvh) * Z + z) * REC;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int qd = t + 256 * j;
      if (qd < nq) {
        const int g = qd / Q, col = (qd % Q) * 4;
        *reinterpret_cast<float4*>(rec + 32 + g * D + col) = acc[j];
        if (col == 0) {
          rec[g] = mrun[j];
          rec[16 + g] = lrun[j];
        }
      }
    }
    store_app();
    return;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int qd = t + 256 * j;
    if (qd < nq) {
      const int g = qd / Q, col = (qd % Q) * 4;
      const float inv = lrun[j] > 0.0f ? 1.0f / lrun[j] : 0.0f;
      S* o = out_base + static_cast<int64_t>(b) * a.out_sb + static_cast<int64_t>(kvh * G + g) * a.out_sh + col;
      o[0] = from_f32<DT>(acc[j].x * inv);
      o[1] = from_f32<DT>(acc[j].y * inv);
      o[2] = from_f32<DT>(acc[j].z * inv);
      o[3] = from_f32<DT>(acc[j].w * inv);
    }
  }
  store_app();
}

// Second level of the merge for calls with few segments: combines the kStreamParts run
// states the merge left for every parted segment, in run order with weights exp2(m_z - M),
// M the largest m_z. Grid (kv heads, batch); segments the merge combined whole are skipped.
template <int DT, int D, bool PLANNED>
__global__ __launch_bounds__(256) void paged_decode_stream_fold(const int32_t*, int32_t, int32_t, StreamArgs sa) {
  using S = typename Elem<DT>::S;
  const int64_t REC = sa.rec_stride;
  const DecodeArgs& a = sa.a;
  const int kvh = blockIdx.x, b = blockIdx.y, G = sa.group, Z = sa.parts;
  int L, gw_lo, gw_hi;
  if constexpr (PLANNED) {
    const int32_t* sd = sa.plan + sa.plan_seg_off + (static_cast<int64_t>(b) * a.hkv + kvh) * kPlanSeg;
    const int pb = load_uniform_i32(sa.plan + 2), ph = load_uniform_i32(sa.plan + 3);
    const int ps = load_uniform_i32(sa.plan + kPlanSegOffWord);
    gw_lo = load_uniform_i32(sd + 0);
    gw_hi = gw_lo + load_uniform_i32(sd + 1) - 1;
    L = load_uniform_i32(sd + 3);
    if (pb != sa.batch || ph != a.hkv || ps != sa.plan_seg_off || gw_lo < 0 || gw_hi >= sa.tw) return;
  } else {
    const int cap = a.max_blocks * a.bs;
    L = a.lens[b];
    L = L < cap ? L : cap;
    if (L <= 0) return;
    const int total = a.hkv * sa.ws_prefix[sa.batch];
    const int tw = stream_active_waves(sa.tw, total, sa.min_tiles, static_cast<int64_t>(sa.batch) * a.hkv, sa.max_pieces);
    const int n = (L + 15) >> 4;
    const int64_t s0 = static_cast<int64_t>(a.hkv) * sa.ws_prefix[b] + static_cast<int64_t>(kvh) * n;
    gw_lo = static_cast<int>(((s0 + 1) * tw - 1) / total);
    gw_hi = static_cast<int>(((s0 + n) * tw - 1) / total);
  }
  const int R = gw_hi - gw_lo + 1;
  if (L <= 0 || Z <= 1 || R <= kWideMergeStreams * kMergeChunk) return;  // merged whole
  const int P = (R + Z - 1) / Z, nz = (R + P - 1) / P;
  const float* base = sa.ws_part + (static_cast<int64_t>(b) * a.hkv + kvh) * Z * REC;
  constexpr int Q = D / 4;
  const int nq = G * Q;
  for (int qd = threadIdx.x; qd < nq; qd += blockDim.x) {
    const int g = qd / Q, col = (qd % Q) * 4;
    float mz[kStreamParts], lz[kStreamParts];
    float4 az[kStreamParts];
#pragma unroll
    for (int k = 0; k < kStreamParts; ++k)
      if (k < nz) {
        mz[k] = base[k * REC + g];
        lz[k] = base[k * REC + 16 + g];
        az[k] = *reinterpret_cast<const float4*>(base + k * REC + 32 + g * D + col);
      }
    float mm = -INFINITY;
#pragma unroll
    for (int k = 0; k < kStreamParts; ++k)
      if (k < nz) mm = fmaxf(mm, mz[k]);
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    float ls = 0.0f;
#pragma unroll
    for (int k = 0; k < kStreamParts; ++k)
      if (k < nz) {
        const float w = mz[k] == -INFINITY ? 0.0f : fast_exp2(mz[k] - mm);
        s.x = fmaf(w, az[k].x, s.x);
        s.y = fmaf(w, az[k].y, s.y);
        s.z = fmaf(w, az[k].z, s.z);
        s.w = fmaf(w, az[k].w, s.w);
        ls = fmaf(w, lz[k], ls);
      }
    const float inv = ls > 0.0f ? 1.0f / ls : 0.0f;
    S* o = reinterpret_cast<S*>(a.out) + static_cast<int64_t>(b) * a.out_sb + static_cast<int64_t>(kvh * G + g) * a.out_sh +
           col;
    o[0] = from_f32<DT>(s.x * inv);
    o[1] = from_f32<DT>(s.y * inv);
    o[2] = from_f32<DT>(s.z * inv);
    o[3] = from_f32<DT>(s.w * inv);
  }
}

// ---- the per-step work plan (mip_paged_decode_plan): computed once per decode step from the
// context lengths and block tables, shared by every layer's call. Every workgroup scans the
// lengths into the tile prefix (cheap: at most 4096 sequences), then the grid writes, in
// grid-stride loops, the wavefront ranges, the segment records for the merge kernel and one
// descriptor per tile. Layout: kPlanHeader / kPlanWave / kPlanSeg / tile descriptors.
constexpr int kPlanThreads = 256;
#ifndef MIP_PLAN_TILES_PER_THREAD
#define MIP_PLAN_TILES_PER_THREAD 2
#endif
constexpr int kPlanTilesPerThread = MIP_PLAN_TILES_PER_THREAD;

struct PlanArgs {
  const int32_t* lens;
  const int32_t* bt;
  int64_t bt_stride;
  int32_t* plan;
  int batch, hkv, bs, log2_bs, cap, tw, min_tiles, max_pieces;
  int seg_off, tile_off;  // word offsets of the segment records and tile descriptors
  int wave_cap;           // descriptor slots per wavefront
};

__global__ __launch_bounds__(kPlanThreads) void paged_decode_plan_kernel(PlanArgs p) {
  extern __shared__ __attribute__((aligned(16))) char psm[];
  const int B = p.batch;
  int* s_len = reinterpret_cast<int*>(psm);  // [B] clamped context lengths
  int* s_pre = s_len + B;                     // [B + 1] exclusive tile prefix
  int* s_wtot = s_pre + B + 1;                // [kPlanThreads / kWave]
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  for (int i = tid; i < B; i += kPlanThreads) {
    int L = p.lens[i];
    L = L < p.cap ? L : p.cap;
    s_len[i] = L > 0 ? L : 0;
  }
  __syncthreads();
  {
    const int chunk = (B + kPlanThreads - 1) / kPlanThreads;
    const int beg = tid * chunk < B ? tid * chunk : B;
    const int end = beg + chunk < B ? beg + chunk : B;
    int sum = 0;
    for (int i = beg; i < end; ++i) sum += (s_len[i] + 15) >> 4;
    const int incl = wave_inclusive_scan(sum, lane);
    if (lane == kWave - 1) s_wtot[w] = incl;
    __syncthreads();
    int off = 0;
    for (int j = 0; j < w; ++j) off += s_wtot[j];
    int run = off + incl - sum;
    for (int i = beg; i < end; ++i) {
      s_pre[i] = run;
      run += (s_len[i] + 15) >> 4;
    }
    if (tid == kPlanThreads - 1) s_pre[B] = off + incl;
  }
  __syncthreads();
  const int64_t T = static_cast<int64_t>(p.hkv) * s_pre[B];
  const int W = T > 0 ? stream_active_waves(p.tw, static_cast<int>(T), p.min_tiles,
                                            static_cast<int64_t>(B) * p.hkv, p.max_pieces)
                     : 0;
  const int gtid = blockIdx.x * kPlanThreads + tid, gstride = gridDim.x * kPlanThreads;
  if (gtid == 0) {
    p.plan[0] = static_cast<int32_t>(T);
    p.plan[1] = W;
    p.plan[2] = B;
    p.plan[3] = p.hkv;
    p.plan[kPlanTileOffWord] = p.tile_off;
    p.plan[kPlanSegOffWord] = p.seg_off;
    p.plan[kPlanWaveCapWord] = p.wave_cap;
    p.plan[7] = 0;
  }
  // Wavefront ranges: the same split as the in-kernel path.
  for (int g = gtid; g < W; g += gstride) {
    int32_t* r = p.plan + kPlanHeader + static_cast<int64_t>(g) * kPlanWave;
    r[0] = static_cast<int>(static_cast<int64_t>(g) * T / W);
    r[1] = static_cast<int>(static_cast<int64_t>(g + 1) * T / W);
  }
  // Segment records for the merge kernel.
  for (int sidx = gtid; sidx < B * p.hkv; sidx += gstride) {
    const int b = sidx / p.hkv, kvh = sidx - b * p.hkv;
    const int L = s_len[b], n = (L + 15) >> 4;
    int g_lo = 0, R = 0, lo_split = 0;
    if (n > 0) {
      const int64_t s0 = static_cast<int64_t>(p.hkv) * s_pre[b] + static_cast<int64_t>(kvh) * n;
      const int64_t e1 = s0 + n - 1;
      g_lo = static_cast<int>(((s0 + 1) * W - 1) / T);
      const int g_hi = static_cast<int>(((e1 + 1) * W - 1) / T);
      R = g_hi - g_lo + 1;
      lo_split = static_cast<int64_t>(g_lo) * T / W < s0 ? 1 : 0;
    }
    int32_t* r = p.plan + p.seg_off + static_cast<int64_t>(sidx) * kPlanSeg;
    r[0] = g_lo;
    r[1] = R;
    r[2] = lo_split;
    r[3] = L;
  }
  // Tile descriptors: tile x of the global sequence (sequence-major, then kv head, then key
  // tile), in slot x - lo of its wavefront g (the largest g with g * T / W <= x).
  uint2* td = reinterpret_cast<uint2*>(p.plan + p.tile_off);
  for (int64_t x = gtid; x < T; x += gstride) {
    const int64_t g = ((x + 1) * W - 1) / T;
    const int64_t slot = g * p.wave_cap + (x - g * T / W);
    int lb = 0, ub = B - 1;  // largest b with Hkv * P[b] <= x; its segment is not empty
    while (lb < ub) {
      const int mid = (lb + ub + 1) >> 1;
      if (static_cast<int64_t>(p.hkv) * s_pre[mid] <= x) lb = mid; else ub = mid - 1;
    }
    const int b = lb, L = s_len[b], n = (L + 15) >> 4;
    const int rem = static_cast<int>(x - static_cast<int64_t>(p.hkv) * s_pre[b]);
    const int kvh = rem / n, t = rem - kvh * n;
    const int tb = 16 * t;
    const int blk = p.bt[static_cast<int64_t>(b) * p.bt_stride + (tb >> p.log2_bs)];
    const int64_t row = (static_cast<int64_t>(blk) * p.hkv + kvh) * p.bs + (tb & (p.bs - 1));
    const uint32_t row0 = (blk < 0 || row >= static_cast<int64_t>(kTileNoRow)) ? kTileNoRow : static_cast<uint32_t>(row);
    const int nvalid = L - tb < 16 ? L - tb : 16;
    const uint32_t meta = static_cast<uint32_t>(b) | (static_cast<uint32_t>(kvh) << 16) |
                          (static_cast<uint32_t>(nvalid) << 24) | (t == 0 ? 1u << 29 : 0u) |
                          (t == n - 1 ? 1u << 30 : 0u);
    td[slot] = make_uint2(row0, meta);
  }
}

// Every stream kernel takes the plan pointer and two scalars ahead of the argument block (the
// main kernel: the plan's descriptor offset and slots per wavefront; the merge: the plan's
// segment-record offset and the kv-head count). The build preloads these leading arguments
// into scalar registers (gfx950 kernel-argument preloading), so a planned kernel issues its
// first plan reads without first waiting for a load of its arguments. Kernels that do not use
// them ignore them.
using StreamFn = void (*)(const int32_t*, int32_t, int32_t, StreamArgs);

struct StreamPick {
  StreamFn main[2][2] = {};   // [fused: with the step's K/V append][planned: from a work plan]
  StreamFn merge[2][2][2] = {};  // [fused][planned][2 streams and runs: a few long segments]
  StreamFn fold[2] = {};         // [planned]
  int ring_bytes = 0;  // per wavefront
};

template <int DT, int D, int QR>
StreamPick pick_one() {
  constexpr int NS = D == 64 ? MIP_STREAM_STAGES_D64 : MIP_STREAM_STAGES_D128;
  constexpr int NJ = QR * D / 4 > 256 ? 2 : 1;  // merge quads per thread: at most QR heads of D / 4 quads
  StreamPick p;
  p.main[0][0] = paged_decode_stream<DT, D, QR, NS, false>;
  p.main[0][1] = paged_decode_stream_tiles<DT, D, QR, NS, false>;
  p.main[1][0] = paged_decode_stream<DT, D, QR, NS, true>;
  p.main[1][1] = paged_decode_stream_tiles<DT, D, QR, NS, true>;
  p.merge[0][0][0] = paged_decode_stream_merge<DT, D, false, false, 1, NJ>;
  p.merge[0][1][0] = paged_decode_stream_merge<DT, D, false, true, 1, NJ>;
  p.merge[1][0][0] = paged_decode_stream_merge<DT, D, true, false, 1, NJ>;
  p.merge[1][1][0] = paged_decode_stream_merge<DT, D, true, true, 1, NJ>;
  p.merge[0][0][1] = paged_decode_stream_merge<DT, D, false, false, kWideMergeStreams, NJ>;
  p.merge[0][1][1] = paged_decode_stream_merge<DT, D, false, true, kWideMergeStreams, NJ>;
  p.merge[1][0][1] = paged_decode_stream_merge<DT, D, true, false, kWideMergeStreams, NJ>;
  p.merge[1][1][1] = paged_decode_stream_merge<DT, D, true, true, kWideMergeStreams, NJ>;
  p.fold[0] = paged_decode_stream_fold<DT, D, false>;
  p.fold[1] = paged_decode_stream_fold<DT, D, true>;
  p.ring_bytes = NS * Ring<D, QR>::STAGE;
  return p;
}

StreamPick pick(int dtype, int d, int group) {
  const bool q8 = group <= 8;
  if (dtype == MIP_BF16) {
    if (d == 64) return q8 ? pick_one<MIP_BF16, 64, 8>() : pick_one<MIP_BF16, 64, 16>();
    if (d == 128) return q8 ? pick_one<MIP_BF16, 128, 8>() : pick_one<MIP_BF16, 128, 16>();
  } else if (dtype == MIP_F16) {
    if (d == 64) return q8 ? pick_one<MIP_F16, 64, 8>() : pick_one<MIP_F16, 64, 16>();
    if (d == 128) return q8 ? pick_one<MIP_F16, 128, 8>() : pick_one<MIP_F16, 128, 16>();
  }
  return {};
}


// Calls with at most kWideMergeSegments segments (batch x kv heads) merge with 2 streams per
// workgroup: a few long sequences, whose segments are split into tens of pieces each (B=1 at
// 32k keys: 29.2 -> 26.4 us per call, B=4 at 8k: 18.2 -> 15.1 us, B=16 at 16k: 37.1 -> 34.2
// us). Calls with at most kPartsSegments segments also cut a segment of more than one round of
// chunks into kStreamParts runs, one workgroup each, folded by a second kernel, and allow 256
// pieces per segment (B=1 at 32k: 26.4 -> 18.2 us; B=2 at 32k, 28q/4kv d128: 39.8 -> 37.6
// us); with 16 to 64 segments the fold's launch costs more than it saves (B=16 at 16k: 34.0
// -> 39.5 us). Batches of more segments have a handful of pieces per segment.
constexpr int64_t kWideMergeSegments = 64;
constexpr int64_t kPartsSegments = 16;
int stream_wide_merge(int64_t segments) { return segments <= kWideMergeSegments ? 1 : 0; }
int stream_merge_parts(int64_t segments) { return segments <= kPartsSegments ? kStreamParts : 1; }

// Most pieces per segment on average (see stream_active_waves). With the one- or two-stream
// merge, 64 measured best for one to four long sequences (one-stream merge, B=1 at 32k keys:
// 74 -> 32 us per call; 128: 31 us, 256: 42 us, 32: 46 us; two-stream merge: 26.4 us, 128:
// 23.3 us but B=4 at 8k 18.6 against 15.1 us) and leaves batches of hundreds of sequences
// untouched; with merge runs, 256 (B=1 at 32k: 18.2 us, 64: 29.2 us, 1024: 18.5 us).
int stream_max_pieces(int64_t segments) {
  const int v = stream_max_pieces_env();
  if (v > 0) return v;
  return stream_merge_parts(segments) > 1 ? 256 : MIP_STREAM_MAX_PIECES;
}

int env_positive(const char* name) {
  const char* env = std::getenv(name);
  const int v = env ? std::atoi(env) : 0;
  return v > 0 ? v : 0;
}

// Occupancy of the stream kernel per (device, dtype, head_dim, q rows): one query per
// process and shape, since it is the same for every call.
struct GridKey {
  int dev, dtype, d, qr;
  bool operator==(const GridKey& o) const { return dev == o.dev && dtype == o.dtype && d == o.d && qr == o.qr; }
};
struct GridEntry {
  GridKey key;
  int grid;  // workgroups of the persistent grid (0: the query failed)
};

}  // namespace

int stream_min_tiles() {
  static const int v = [] {
    const int e = env_positive("MIP_STREAM_MIN_TILES");
    return e > 0 ? e : 4;
  }();
  return v;
}

int stream_max_pieces_env() {
  static const int v = env_positive("MIP_STREAM_MAX_PIECES");
  return v;
}

int64_t stream_part_floats(const StreamConfig& cfg, int batch, int num_kv_heads) {
  const int64_t segments = static_cast<int64_t>(batch) * num_kv_heads;
  const int parts = stream_merge_parts(segments);
  return parts > 1 ? segments * parts * cfg.rec_floats : 0;
}

StreamConfig stream_config(int dtype, int d, int group, int batch) {
  StreamConfig c{};
  if (batch < 1 || batch > kStreamMaxBatch || group < 1 || group > 16) return c;
  const StreamPick p = pick(dtype, d, group);
  if (!p.main[0][0]) return c;
  // The LDS rings (at least 60 KiB per workgroup) always exceed the scan area of
  // kStreamMaxBatch sequences (33 KiB), so the size, and with it the occupancy, does not
  // depend on the batch.
  const int scan_bytes = (2 * kStreamMaxBatch + 1 + kSW) * 4;
  const int ring_bytes = kSW * p.ring_bytes;
  static_assert((2 * kStreamMaxBatch + 1 + kSW) * 4 <= kSW * 3 * (32 + 8) * 128, "scan area within the rings");
  c.lds_bytes = scan_bytes > ring_bytes ? scan_bytes : ring_bytes;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return c;
  const GridKey key{dev, dtype, d, group <= 8 ? 8 : 16};
  static std::mutex mu;
  static std::vector<GridEntry> known;
  int grid = -1;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const GridEntry& e : known)
      if (e.key == key) grid = e.grid;
  }
  if (grid < 0) {
    int cus = 0, per_cu = 0;
    grid = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0 &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(p.main[0][0]),
                                                     kSW * kWave, c.lds_bytes) == hipSuccess)
      grid = cus * (per_cu > 0 ? per_cu : 1);
    if (grid > 0) {  // a failed query is not remembered: the next call asks again
      std::lock_guard<std::mutex> lock(mu);
      known.push_back(GridEntry{key, grid});
    }
  }
  if (grid <= 0) return c;
  c.grid = grid;
  c.tw = c.grid * kSW;
  c.rec_floats = 32 + static_cast<int64_t>(group) * d;
  c.ok = true;
  return c;
}

int stream_launch(const StreamConfig& cfg, const StreamArgs& sa_in, int dtype, int d, int group, int num_kv_heads,
                  int batch, hipStream_t stream) {
  const StreamPick p = pick(dtype, d, group);
  StreamArgs sa = sa_in;
  sa.tw = cfg.tw;
  sa.min_tiles = stream_min_tiles();
  sa.max_pieces = stream_max_pieces(static_cast<int64_t>(batch) * num_kv_heads);
  sa.rec_stride = static_cast<int>(cfg.rec_floats);
  const int fused = sa.app.slots != nullptr, planned = sa.plan != nullptr;
  hipLaunchKernelGGL(p.main[fused][planned], dim3(cfg.grid), dim3(kSW * kWave), cfg.lds_bytes, stream, sa.plan,
                     sa.plan_tile_off, sa.plan_wave_cap, sa);
  const int64_t segments = static_cast<int64_t>(batch) * num_kv_heads;
  const int wide = stream_wide_merge(segments);
  sa.parts = stream_merge_parts(segments);
  hipLaunchKernelGGL(p.merge[fused][planned][wide], dim3(num_kv_heads, batch, sa.parts),
                     dim3(wide ? 256 * kWideMergeStreams : 256), 0, stream, sa.plan, sa.plan_seg_off, num_kv_heads,
                     sa);
  if (sa.parts > 1)
    hipLaunchKernelGGL(p.fold[planned], dim3(num_kv_heads, batch), dim3(256), 0, stream, sa.plan, sa.plan_seg_off, 0,
                       sa);
  return static_cast<int>(hipGetLastError());
}

namespace {
struct PlanLayout {
  int64_t seg_off, tile_off, wave_cap, words;
};
PlanLayout plan_layout(const StreamConfig& cfg, int batch, int num_kv_heads, int block_size, int max_blocks) {
  PlanLayout l{};
  const int64_t tiles_per_seq = (static_cast<int64_t>(max_blocks) * block_size + 15) / 16;
  const int64_t max_tiles = static_cast<int64_t>(batch) * num_kv_heads * tiles_per_seq;
  // A wavefront's range holds at most ceil(T / W) tiles: ceil(max_tiles / tw) when all tw
  // wavefronts are active, at most min_tiles when W = ceil(T / min_tiles), and at most
  // ceil(max_tiles / (segments * max_pieces)) when the piece cap sets W.
  const int64_t min_tiles = stream_min_tiles();
  const int64_t per_wave = (max_tiles + cfg.tw - 1) / cfg.tw;
  const int64_t segments = static_cast<int64_t>(batch) * num_kv_heads;
  const int64_t seg_cap = segments * stream_max_pieces(segments);
  const int64_t per_piece = (max_tiles + seg_cap - 1) / seg_cap;
  l.wave_cap = per_wave > min_tiles ? per_wave : min_tiles;
  if (per_piece > l.wave_cap) l.wave_cap = per_piece;
  l.seg_off = kPlanHeader + static_cast<int64_t>(cfg.tw) * kPlanWave;
  l.tile_off = l.seg_off + static_cast<int64_t>(batch) * num_kv_heads * kPlanSeg;
  l.tile_off += l.tile_off & 1;  // descriptors are 8-byte pairs
  l.words = l.tile_off + 2 * (static_cast<int64_t>(cfg.tw) * l.wave_cap + kWave);
  return l;
}
}  // namespace

int64_t stream_plan_bytes(const StreamConfig& cfg, int batch, int num_kv_heads, int block_size, int max_blocks) {
  // Tile descriptors hold one pool row per tile, so a tile must lie in one block; the
  // descriptor's meta word holds the sequence and kv head in 16 and 8 bits.
  if (block_size < 16 || batch > 65535 || num_kv_heads > 255) return 0;
  const PlanLayout l = plan_layout(cfg, batch, num_kv_heads, block_size, max_blocks);
  if (l.words >= (int64_t{1} << 31) || l.wave_cap >= (int64_t{1} << 30) / cfg.tw) return 0;
  return l.words * 4;
}

void stream_plan_offsets(const StreamConfig& cfg, int batch, int num_kv_heads, int block_size, int max_blocks,
                         int32_t* seg_off, int32_t* tile_off, int32_t* wave_cap) {
  const PlanLayout l = plan_layout(cfg, batch, num_kv_heads, block_size, max_blocks);
  *seg_off = static_cast<int32_t>(l.seg_off);
  *tile_off = static_cast<int32_t>(l.tile_off);
  *wave_cap = static_cast<int32_t>(l.wave_cap);
}

int stream_plan_launch(const StreamConfig& cfg, const int32_t* lens, const int32_t* block_tables, int64_t bt_stride,
                       int batch, int num_kv_heads, int block_size, int max_blocks, int32_t* plan,
                       hipStream_t stream) {
  const PlanLayout l = plan_layout(cfg, batch, num_kv_heads, block_size, max_blocks);
  PlanArgs p{};
  p.lens = lens;
  p.bt = block_tables;
  p.bt_stride = bt_stride;
  p.plan = plan;
  p.batch = batch;
  p.hkv = num_kv_heads;
  p.bs = block_size;
  p.log2_bs = ilog2_exact(block_size);
  p.cap = max_blocks * block_size;
  p.tw = cfg.tw;
  p.min_tiles = stream_min_tiles();
  p.max_pieces = stream_max_pieces(static_cast<int64_t>(batch) * num_kv_heads);
  p.seg_off = static_cast<int>(l.seg_off);
  p.tile_off = static_cast<int>(l.tile_off);
  p.wave_cap = static_cast<int>(l.wave_cap);
  // Enough workgroups for about kPlanTilesPerThread descriptors per thread at the largest
  // tile count.
  const int64_t max_tiles = (l.words - l.tile_off) / 2;
  int64_t grid = (max_tiles + kPlanTilesPerThread * kPlanThreads - 1) / (kPlanTilesPerThread * kPlanThreads);
  grid = grid < 1 ? 1 : (grid > 1024 ? 1024 : grid);
  const size_t lds = static_cast<size_t>(2 * batch + 1 + kPlanThreads / kWave) * 4;
  hipLaunchKernelGGL(paged_decode_plan_kernel, dim3(static_cast<unsigned>(grid)), dim3(kPlanThreads), lds, stream, p);
  return static_cast<int>(hipGetLastError());
}

}  // namespace decode
}  // namespace mip
