// MFMA product core for gfx950:  C[b](i,j) = sum_k P[b](i,k) * Q[b](j,k)
//
// Operands are row-major with K contiguous ("NT", every element type: X·Xᵀ,
// S·S for symmetric S, B·X via a stored Xᵀ, ...), where each lane's MFMA
// fragment is a contiguous 16-byte run in LDS; bf16 operands may instead be
// stored [K][·] ("QN" for Q, "PT" for P) and read through transposing LDS
// loads (see below).
//
// Operand contract (checked by the host launchers):
//   * K is a multiple of one ring of K tiles (Tile::NS * BK) and the pad
//     columns of both operands are zero (workspace buffers are padded to
//     kPadK);
//   * rows beyond M (P) or N (Q) are never read (masked to zero);
//   * operand base pointers and leading dimensions are 16-byte aligned.
//
// Grid: blockIdx.x enumerates output tiles, blockIdx.y the batch. In UPPER
// mode only tiles with tile_row <= tile_col are launched; the value computed
// for (i, j), i <= j, is stored at (i, j) and at (j, i), so the result is an
// exactly symmetric matrix at half the MFMA work.
//
// Pipeline: a ring of LDS stages (four, or eight for the small fp32 tiles)
// filled by direct global-to-LDS loads, NS - 1 K tiles ahead of the MFMAs;
// one barrier per K tile, or two in the ping-pong schedule of the 256² bf16
// tiles (details below).
#pragma once

#include <atomic>
#include <type_traits>
#include <utility>

#include "pto_common.h"
#include "upper_order.h"

namespace pto {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef double f64x4_t __attribute__((ext_vector_type(4)));

// Per element type: which MFMA, its fragment shapes and output lane map.
//   MN  : output block is MN x MN
//   KPL : consecutive k values one lane feeds per instruction
//   G   : lane groups along k (64 / MN)
template <typename T>
struct Mfma;

// bf16 uses the 16x16x32 shape: for the same wave tile it gives four times
// as many independent accumulators as 32x32x16 at the same operand reads
// and registers, and measured faster in this core. Lane l feeds row (or
// column) l % 16 with k = 8*(l/16) .. +7 (both operands use the same k
// assignment, so the sum is exact whatever order the hardware uses).
template <>
struct Mfma<bf16> {  // v_mfma_f32_16x16x32_bf16
  typedef float acc_t;
  typedef f32x4_t cvec_t;
  static constexpr int MN = 16, KPL = 8, G = 4, NACC = 4;
  __device__ static __forceinline__ cvec_t mma(const uint4& a, const uint4& b, int, cvec_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane, int r) { return (lane >> 4) * 4 + r; }
  __device__ static __forceinline__ int col(int lane, int) { return lane & 15; }
};

// fp32 uses the 16x16x4 shape: lane l feeds row (or column) l % 16 with
// k = 4*(l/16) + ii of its 16-byte run in instruction ii, both operands
// alike. Measured 1.5-2% faster than 32x32x2 on the fp32 NS5, kron and
// apply products at the same tiles (a microbenchmark sustains 154 against
// 148 TFLOP/s).
template <>
struct Mfma<float> {  // v_mfma_f32_16x16x4_f32
  typedef float acc_t;
  typedef f32x4_t cvec_t;
  static constexpr int MN = 16, KPL = 1, G = 4, NACC = 4;
  __device__ static __forceinline__ cvec_t mma(const uint4& a, const uint4& b, int ii, cvec_t c) {
    float av = __uint_as_float(ii == 0 ? a.x : ii == 1 ? a.y : ii == 2 ? a.z : a.w);
    float bv = __uint_as_float(ii == 0 ? b.x : ii == 1 ? b.y : ii == 2 ? b.z : b.w);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane, int r) { return (lane >> 4) * 4 + r; }
  __device__ static __forceinline__ int col(int lane, int) { return lane & 15; }
};

template <>
struct Mfma<double> {  // v_mfma_f64_16x16x4_f64
  typedef double acc_t;
  typedef f64x4_t cvec_t;
  static constexpr int MN = 16, KPL = 1, G = 4, NACC = 4;
  __device__ static __forceinline__ cvec_t mma(const uint4& a, const uint4& b, int ii, cvec_t c) {
    unsigned long long ab = ii == 0 ? ((unsigned long long)a.y << 32 | a.x) : ((unsigned long long)a.w << 32 | a.z);
    unsigned long long bb = ii == 0 ? ((unsigned long long)b.y << 32 | b.x) : ((unsigned long long)b.w << 32 | b.z);
    return __builtin_amdgcn_mfma_f64_16x16x4f64(__longlong_as_double((long long)ab),
                                                __longlong_as_double((long long)bb), c, 0, 0, 0);
  }
  // Output lane map measured on gfx950: lane l, element r holds
  // D[l/16 + 4r][l%16] (unlike the f32 16x16 family's 4(l/16) + r).
  __device__ static __forceinline__ int row(int lane, int r) { return (lane >> 4) + 4 * r; }
  __device__ static __forceinline__ int col(int lane, int) { return lane & 15; }
};

// Tile configuration: BM x BN output tile, BK deep (64 bytes), WM x WN
// waves, NS LDS stages (4 or 8), PP: ping-pong schedule (main loop), KG:
// K groups (KG = 2: two WM x WN wave groups take alternate K tiles, each
// accumulating the whole tile, summed at the end).
template <int BM_, int BN_, int BK_, int WM_, int WN_, int NS_ = 4, bool PP_ = false, int KG_ = 1>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, NS = NS_, KG = KG_;
  static constexpr bool PP = PP_;
  static constexpr int NT = 64 * WM * WN * KG;
  static_assert(NS == 4 || NS == 8, "ring of 4 or 8 stages");
  static_assert(!PP || (NS == 4 && WM == 2 && WN == 4 && KG == 1), "ping-pong: two groups of four waves, four stages");
  static_assert(KG == 1 || (KG == 2 && NS == 4 && !PP), "K groups: two, four stages");
};

struct GemmArgs {
  const void* P;
  int64_t ldp, sP;  // row pitch and batch stride, in elements
  const void* Q;
  int64_t ldq, sQ;
  int M, N, K;
  int tiles_m, tiles_n;
  const int* guard;  // if non-null and guard[b * guard_stride] != 0, matrix b is skipped
  int guard_stride;  // ints between the guard words of consecutive matrices (0: one word)
  int cus;           // compute units of the device (set by the launcher)
};

// Workgroups are dispatched to the 8 XCDs round-robin by linear id, each
// XCD has its own L2, and all XCDs share the memory-side Infinity Cache.
// With one tile per CU in flight, workgroups w = k·C .. k·C + C - 1 (C the
// CU count) run together as round k; they take logical tiles k·C .. k·C +
// C - 1, XCD x the contiguous block k·C + x·C/8 .. + C/8 - 1. The tiles
// co-resident on an XCD are then neighbours in the (batch, tile) order and
// share operand panels in its L2, and the eight XCDs work on the same
// matrix at once, so each one's panel misses are mostly served by the
// Infinity Cache rather than HBM (a contiguous 1/8 of all tiles per XCD put
// eight matrices in flight, 512 MB of NS5 operands against a 256 MB cache:
// batched NS5 +2%). A last partial round, and launches of fewer than C
// tiles, give each XCD one contiguous range of what is left.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_range(int w, int total) {
  const int q = total / kXcds, r = total % kXcds;
  const int xcd = w % kXcds, slot = w / kXcds;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
}
__device__ __forceinline__ int xcd_remap(int w, int total, int cus) {
  if (cus <= 0 || cus % kXcds != 0) return xcd_range(w, total);
  const int full = total / cus * cus, per = cus / kXcds;
  if (w < full) return w / cus * cus + (w % kXcds) * per + (w / kXcds) % per;
  return full + xcd_range(w - full, total - full);
}

// Map the linear tile id to (tile_row, tile_col).
// UPPER, BLOCKED: the upper tiles in blocks of 4 tile rows x 8 tile columns
// (blocks row-major, tiles row-major inside a block), so the ~32 tiles an XCD
// runs at once read fewer operand panels than whole upper-triangle rows
// (14-18 against 16-22 at 22 x 22 tiles); measured on the bf16 K-FAC Gram
// (16384x4096, one round of 253 tiles of 192²): -1 to -3.5% over three A/B
// calls. The small fp32 root tiles run slower with it (n = 1024 +6%) and
// keep plain rows. One-round launches of one matrix with at most 22 x 22
// tiles use the searched orders of upper_order.h instead (10-11 panels per
// XCD at 22 x 22).
template <bool UPPER, bool BLOCKED = false>
__device__ __forceinline__ void decode_tile(int t, int tiles_m, int tiles_n, int& ti, int& tj) {
  if (UPPER && BLOCKED) {
    constexpr int BR = 4, BC = 8;
    const int nbr = (tiles_n + BR - 1) / BR, nbc = (tiles_n + BC - 1) / BC;
    int rem = t;
    ti = 0;
    tj = 0;
    for (int R = 0; R < nbr; ++R) {
      const int r0 = R * BR, r1 = min(r0 + BR, tiles_n);
      for (int C = r0 / BC; C < nbc; ++C) {
        const int c0 = C * BC, c1 = min(c0 + BC, tiles_n);
        int cnt = 0;
        for (int i = r0; i < r1; ++i) cnt += max(0, c1 - max(c0, i));
        if (rem < cnt) {
          for (int i = r0; i < r1; ++i) {
            const int n = max(0, c1 - max(c0, i));
            if (rem < n) {
              ti = i;
              tj = max(c0, i) + rem;
              return;
            }
            rem -= n;
          }
        }
        rem -= cnt;
      }
    }
  } else if (UPPER) {
    int r = 0, rem = t;
    while (rem >= tiles_n - r) {
      rem -= tiles_n - r;
      ++r;
    }
    ti = r;
    tj = r + rem;
  } else {
    // Column-group ordering: walk 8 tile rows at a time so consecutive
    // workgroups share the Q panel and a small set of P panels.
    const int GRP = 8;
    int group = t / (GRP * tiles_n);
    int first = group * GRP;
    int rows = min(tiles_m - first, GRP);
    int in = t - group * GRP * tiles_n;
    ti = first + in % rows;
    tj = in / rows;
  }
}

// ------------------------------------------------------------- main loop
// K tiles are 64 bytes deep (bf16 BK=32, fp32 16, fp64 8). Operand tiles
// go from global memory straight into LDS (global_load_lds_dwordx4: each
// wave instruction fills 1 KiB = 16 rows of 64 bytes) through a ring of NS
// stages, so NS - 1 tiles are in flight while one is consumed, with no
// staging registers and no ds_write instructions. The stages are separate
// __shared__ arrays and the loop is unrolled by NS, so every LDS access
// names its stage statically and the compiler's wait insertion can tell the
// in-flight stages apart; prefetches are unconditional (past the end they
// re-read the last tile into a stage that is never consumed) so the
// outstanding-load count is the same on every path.
//
// A tile's load is issued NS - 2 steps before its LDS reads, so a step
// cannot be shorter than the load latency / (NS - 2). The big tiles' steps
// (512+ MFMA cycles per wave) cover it with four stages; the small fp32
// tiles (128-512 cycles per step) use eight (measured a few percent faster
// on one-matrix roots, where their launches are latency-bound).
//
// LDS rows are unpadded; 16-byte chunk c of row r lives at physical chunk
// c ^ f(r), f(r) = ((r >> 2) & 3) ^ (r & 2), which makes the fragment
// reads (16 consecutive rows, one chunk) conflict-free in both 8- and
// 16-lane windows. The DMA side needs no care: it writes 1 KiB runs.
constexpr int kStages = 4;  // the default ring
constexpr int kRowBytes = 64;

__device__ __forceinline__ int swz(int r) { return ((r >> 2) & 3) ^ (r & 2); }

// "QN" operand layout (bf16 only): Q is stored [K][N], N contiguous, the
// natural layout of X in X' = B·X, so no transposed copy of X is needed.
// A stage then holds BK rows of BN elements (BN*2 bytes) for Q, and the
// MFMA B fragments come from transposing LDS reads (ds_read_b64_tr_b16).
// Within each 16-lane group, lane s addresses 4 elements at row k0 + s/4,
// column n0 + 4*(s%4); lane s then receives column n0 + s of rows
// k0..k0+3. With the 16x16x32 MFMA, 16-lane group g holds k = 8g..8g+7,
// so one read covers rows {4t..4t+3} + 8g and two 16-byte chunks per
// group. A half-wave reads 8 rows ({0..3, 8..11} + 16h, or those plus 4
// for the second half of a fragment), one 32-byte segment each, and is
// conflict-free when the 8 segments fall in distinct 32-byte slots of
// the 256-byte bank row. 16-byte chunk c of Q row r lives at physical
// chunk c ^ swzq<RB>(r) (an even XOR, so a segment's two chunks stay
// adjacent):
//  - rows of a multiple of 256 bytes start at slot 0, and
//    2·((r & 3) | ((r >> 1) & 4)) spreads the 8 rows over 8 slots;
//  - rows of 384 bytes (the 192-wide tile) alternate between slots 0 and 4
//    with r's parity, so the XOR only has to separate the four rows of each
//    parity: 2·(((r >> 1) & 1) | ((r >> 2) & 2)), which flips chunk bits 1-2
//    only and so keeps every chunk inside its 128-byte group (below 24).
// Both depend on row bits 0, 1 and 3 only, so the second half of a
// fragment (4 rows on) keeps the swizzle.
template <int RB>
__device__ __forceinline__ int swzq(int r) {
  // (the kernel asserts RB % 256 is 0 or 128 wherever the layout is used)
  if constexpr (RB % 256 == 0) return 2 * ((r & 3) | ((r >> 1) & 4));
  return 2 * (((r >> 1) & 1) | ((r >> 2) & 2));
}
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

// s_waitcnt with only the vector-memory counter constrained (gfx9 layout:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
#define PTO_VMCNT(n) ((((n) & 0xF) | ((((n) >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8)))
// ... and with only lgkmcnt(0) required.
#define PTO_LGKM0 ((0xF) | (3 << 14) | (0x7 << 4))

// All waves' earlier LDS reads are done and their waited-for DMA writes
// visible. A bare s_barrier (no release fence, which would force every
// in-flight load to complete) bracketed by compiler-only fences.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_waitcnt(PTO_LGKM0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gbl_void_t;

// LDS plan: NS stages of (BM + BN) rows x 64 bytes; after the loop each
// stage array also hosts the epilogue staging of WPA waves (RPP rows x
// (WTN + 1) accumulator-type values per wave, odd pitch). With K groups a
// wave stores WTE = WTM / KG rows of its sub-tile (the partner group stores
// the rest).
template <typename T, class Cfg, typename S>
struct LdsPlan {
  static constexpr int NW = Cfg::WM * Cfg::WN * Cfg::KG, NS = Cfg::NS;
  static constexpr int WTM = Cfg::BM / Cfg::WM, WTN = Cfg::BN / Cfg::WN, WTE = WTM / Cfg::KG;
  static constexpr int STAGE = (Cfg::BM + Cfg::BN) * kRowBytes;
  static constexpr int WPA = (NW + NS - 1) / NS;  // waves per array in the epilogue
  static constexpr int SP = WTN + 1;
  static constexpr int kLdsMax = 160 * 1024;
  // rows per epilogue pass: the largest multiple of 16, at most 64, that
  // divides the rows a wave stores and lets the four arrays fit
  static constexpr int pick_rpp() {
    for (int r = (WTE < 64 ? WTE : 64) / 16 * 16; r > 16; r -= 16) {
      const int epi = WPA * r * SP * (int)sizeof(S);
      if (WTE % r == 0 && NS * (STAGE > epi ? STAGE : epi) <= kLdsMax) return r;
    }
    return 16;
  }
  static constexpr int RPP = pick_rpp();
  static constexpr int EPI = WPA * RPP * SP * (int)sizeof(S);
  static constexpr int ARR = ((STAGE > EPI ? STAGE : EPI) + 15) / 16 * 16;
};

// An epilogue functor may carry a skip hook, `bool skip(int b, bool first)
// const`, evaluated by every wave of every workgroup before any other work:
// true skips matrix b (the workgroup exits). It must return the same value
// in every wave of a workgroup; `first` marks one workgroup per matrix (the
// first tile of b), which may record the decision for later launches.
template <class E, class = void>
struct HasSkip : std::false_type {};
template <class E>
struct HasSkip<E, std::void_t<decltype(std::declval<const E&>().skip(0, false))>> : std::true_type {};

// PT: P is stored [K][M] (M contiguous) and read like a QN operand. For a
// symmetric P (B' in X' = B'·X, A in A·A) that is P itself: its rows are
// its columns, so the product reads it with conflict-free transposing LDS
// reads and 512-byte DMA rows instead of 16-byte row chunks.
template <typename T, class Cfg, bool UPPER, class Epi, bool QN = false, bool PT = false, bool COMP = false>
__global__ void __launch_bounds__(Cfg::NT) gemm_nt_kernel(GemmArgs g, Epi epi) {
  typedef Mfma<T> MF;
  typedef typename MF::cvec_t cvec_t;
  typedef typename Epi::S S;
  typedef LdsPlan<T, Cfg, S> Plan;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, NW = Plan::NW;
  constexpr int BK = kRowBytes / (int)sizeof(T);   // elements per K tile
  constexpr int VEC = 16 / (int)sizeof(T);         // elements per 16-byte chunk
  constexpr int WTM = Plan::WTM, WTN = Plan::WTN;
  constexpr int FM = WTM / MF::MN, FN = WTN / MF::MN;
  constexpr int KSPAN = BK / MF::G;                // k values per lane group per tile
  constexpr int NRG = KSPAN / VEC;                 // 16-byte fragment reads per tile
  constexpr int IPR = VEC / MF::KPL;               // MFMAs per 16-byte read
  constexpr int IPW = (BM + BN) / 16 / NW;         // DMA instructions per wave per tile
  constexpr int QRB = QN ? BN * (int)sizeof(T) : kRowBytes;  // bytes per Q row in LDS
  constexpr int CPR = QRB / 16;                    // 16-byte chunks per Q row
  constexpr int PRB = PT ? BM * (int)sizeof(T) : kRowBytes;  // bytes per P row in LDS
  constexpr int CPRP = PRB / 16;                   // 16-byte chunks per P row
  static_assert((BM + BN) % (16 * NW) == 0 && IPW >= 1, "DMA split");
  static_assert(!PT || (QN && CPRP >= 16 && (PRB % 256 == 0 || PRB % 256 == 128)),
                "PT layout: with QN, P rows of 256·k or 256·k + 128 bytes");
  static_assert(WTM % MF::MN == 0 && WTN % MF::MN == 0 && WTM % 16 == 0, "wave tile");
  static_assert(KSPAN % VEC == 0 && NRG >= 1, "fragment runs");
  constexpr int NS = Cfg::NS;
  static_assert((NS - 2) * IPW <= 63, "vmcnt range");
  static_assert(Plan::RPP % MF::MN == 0 && Plan::WTE % Plan::RPP == 0, "epilogue passes");
  constexpr int KG = Cfg::KG, NWG = Cfg::WM * Cfg::WN;  // K groups, waves per group
  static_assert(KG == 1 || (FM % 2 == 0 && Plan::WTE % MF::MN == 0), "K groups: halves of whole fragments");
  static_assert(Cfg::NS * Plan::ARR <= Plan::kLdsMax, "LDS budget");
  static_assert(!QN || (sizeof(T) == 2 && (!UPPER || PT) && CPR >= 16 && (QRB % 256 == 0 || QRB % 256 == 128) &&
                        (BM * kRowBytes) % 1024 == 0 && NRG == 1),
                "QN layout: bf16, Q rows of 256·k or 256·k + 128 bytes; symmetric products only with PT");

  // stages 4..7 exist (at full size) only in eight-stage rings
  constexpr int ARR_HI = NS > 4 ? Plan::ARR : 16;
  __shared__ __attribute__((aligned(16))) char st0[Plan::ARR];
  __shared__ __attribute__((aligned(16))) char st1[Plan::ARR];
  __shared__ __attribute__((aligned(16))) char st2[Plan::ARR];
  __shared__ __attribute__((aligned(16))) char st3[Plan::ARR];
  __shared__ __attribute__((aligned(16))) char st4[ARR_HI];
  __shared__ __attribute__((aligned(16))) char st5[ARR_HI];
  __shared__ __attribute__((aligned(16))) char st6[ARR_HI];
  __shared__ __attribute__((aligned(16))) char st7[ARR_HI];

  const int tid = threadIdx.x;
  // wave index in a scalar register: DMA destinations and per-wave offsets
  // are then scalar arithmetic
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = KG == 1 ? 0 : wave / NWG, wl = wave - kg * NWG;  // K group, wave in the group
  const int wm = wl / Cfg::WN, wn = wl % Cfg::WN;
  const int ntile = gridDim.x;  // tiles per matrix
  const int logical = xcd_remap(blockIdx.y * ntile + blockIdx.x, ntile * gridDim.y, g.cus);
  const int b = logical / ntile;
  if (g.guard != nullptr && g.guard[(int64_t)b * g.guard_stride] != 0) return;
  if constexpr (HasSkip<Epi>::value) {
    if (epi.skip(b, logical == b * ntile)) return;
  }
  int ti, tj;
  if (UPPER && gridDim.y == 1 && g.tiles_n <= kUpperOrderMaxT && ntile == g.tiles_n * (g.tiles_n + 1) / 2 &&
      ntile <= g.cus) {
    // one round of one matrix: each XCD's contiguous range of logical ids
    // is a set of upper tiles chosen to read few operand panels
    const int e = kUpperOrder[kUpperOrderOff[g.tiles_n - 1] + logical];
    ti = e >> 5;
    tj = e & 31;
  } else {
    decode_tile<UPPER, sizeof(T) == 2>(logical - b * ntile, g.tiles_m, g.tiles_n, ti, tj);
  }
  const int row0 = ti * BM, col0 = tj * BN;
  // On a diagonal tile of a symmetric product a wave whose sub-tile lies
  // entirely below the diagonal stores nothing (both epilogue passes use
  // positions i <= j only). In the two-group schedules it still issues its
  // share of the DMA and every barrier, but skips its fragment reads and
  // MFMAs, which saves their energy (the board runs at its power limit).
  const bool idle = UPPER && (Cfg::PP || KG == 2) && ti == tj && wm * WTM >= (wn + 1) * WTN;

  // Per-thread DMA sources: instruction q of this wave fills the 1 KiB of
  // the stage at R0*64 bytes, R0 = 16*(wave*IPW + q) (P rows first, then
  // Q); lane L supplies bytes 16L..16L+15 of it. In the K-contiguous
  // layout that is row R0 + L/4, physical chunk L%4, i.e. logical chunk
  // (L%4) ^ swz(row); rows past M (N) re-read the last valid row. In the
  // QN layout a Q lane's byte offset o in the Q region gives row
  // rq = o / QRB, physical chunk (o % QRB) / 16, logical chunk that ^
  // swzq(rq) (a row may straddle two instructions); columns past the row
  // pitch re-read its last chunk. A PT lane does the same in the P region
  // (rows of PRB bytes, columns from row0).
  const char* src[IPW];
  unsigned step[IPW];  // bytes between consecutive K tiles (the launcher bounds it)
  int dst_off[IPW];
#pragma unroll
  for (int q = 0; q < IPW; ++q) {
    const int R0 = 16 * (wave * IPW + q), r = R0 + (lane >> 2);
    const int chunk = (lane & 3) ^ swz(r);
    const T* s;
    if (PT && R0 < BM) {
      const int o = R0 * kRowBytes + 16 * lane;
      const int rp = o / PRB;
      const int c = ((o % PRB) >> 4) ^ swzq<PRB>(rp);
      const int64_t col = min((int64_t)row0 + c * VEC, g.ldp - VEC);
      s = static_cast<const T*>(g.P) + (int64_t)b * g.sP + (int64_t)rp * g.ldp + col;
      step[q] = (unsigned)(kRowBytes * g.ldp);
    } else if (R0 < BM) {
      const int gr = min(row0 + r, max(g.M - 1, 0));
      s = static_cast<const T*>(g.P) + (int64_t)b * g.sP + (int64_t)gr * g.ldp + chunk * VEC;
      step[q] = kRowBytes;
    } else if (!QN) {
      const int gr = min(col0 + (r - BM), max(g.N - 1, 0));
      s = static_cast<const T*>(g.Q) + (int64_t)b * g.sQ + (int64_t)gr * g.ldq + chunk * VEC;
      step[q] = kRowBytes;
    } else {
      const int o = (R0 - BM) * kRowBytes + 16 * lane;
      const int rq = o / QRB;
      const int c = ((o % QRB) >> 4) ^ swzq<QRB>(rq);
      const int64_t col = min((int64_t)col0 + c * VEC, g.ldq - VEC);
      s = static_cast<const T*>(g.Q) + (int64_t)b * g.sQ + (int64_t)rq * g.ldq + col;
      step[q] = (unsigned)(kRowBytes * g.ldq);
    }
    src[q] = reinterpret_cast<const char*>(s);
    dst_off[q] = R0 * kRowBytes;
  }
  auto issue = [&](int kt, char* stage) {
#pragma unroll
    for (int q = 0; q < IPW; ++q)
      __builtin_amdgcn_global_load_lds((gbl_void_t*)(src[q] + (uint64_t)(unsigned)kt * step[q]),
                                       (lds_void_t*)(stage + dst_off[q]), 16, 0, 0);
  };

  cvec_t acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int r = 0; r < MF::NACC; ++r) acc[fm][fn][r] = 0;

  const int lr = lane % MF::MN, lg = lane / MF::MN;
  const int sw = swz(lr);  // rows of every fragment are lr mod 16
  // QN: byte offset of this lane's transposing read for fragment fn, MFMA
  // step 0, first half (k = KSPAN*lg + 0..3); step rg (8 rows) and the
  // second half (4 rows) add rows that keep the row's swizzle, which
  // depends on row bits 0, 1 and 3 only.
  int qoff[FN];
  if constexpr (QN) {
    static_assert(KSPAN % 8 == 0, "QN row steps must keep the swizzle");
    const int li = lane & 15, qr = KSPAN * lg + (li >> 2);
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int col = wn * WTN + fn * MF::MN + (lane & (MF::MN - 1) & ~15) + 4 * (li & 3);
      qoff[fn] = qr * QRB + (((col >> 3) ^ swzq<QRB>(qr)) << 4) + ((col & 7) << 1);
    }
  }
  int poff[FM];  // PT: the same for fragment fm of P (columns = rows of the output)
  if constexpr (PT) {
    const int li = lane & 15, qr = KSPAN * lg + (li >> 2);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int col = wm * WTM + fm * MF::MN + (lane & (MF::MN - 1) & ~15) + 4 * (li & 3);
      poff[fm] = qr * PRB + (((col >> 3) ^ swzq<PRB>(qr)) << 4) + ((col & 7) << 1);
    }
  }
  // One K tile's MFMA operands for this wave.
  struct Frag {
    uint4 a[NRG][FM], b[NRG][FN];
  };
  constexpr int kTileMfma = NRG * IPR * FM * FN;              // MFMAs per K tile
  constexpr int kFragReads = NRG * ((PT ? 2 : 1) * FM + (QN ? 2 : 1) * FN);  // LDS reads per K tile
  static_assert(kTileMfma % IPW == 0 && kFragReads % IPW == 0, "schedule groups");
  // Order within a step: LDS reads for the next tile all first, or spread
  // between the MFMA groups (measured faster for the QN layout, slower for
  // the symmetric K-contiguous products).
  constexpr bool kSpreadReads = QN;
  auto load_frags = [&](const char* stage, Frag& f) {
    const char* Pw = stage + (wm * WTM + lr) * kRowBytes;
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      const int off = ((lg * NRG + rg) ^ sw) * 16;
      if constexpr (PT) {
        const char* Ps = stage + 8 * rg * PRB;
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(Ps + poff[fm]));
          v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(Ps + poff[fm] + 4 * PRB));
          uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          f.a[rg][fm] = make_uint4(l2.x, l2.y, h2.x, h2.y);
        }
      } else {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          f.a[rg][fm] = *reinterpret_cast<const uint4*>(Pw + fm * MF::MN * kRowBytes + off);
      }
      if constexpr (QN) {
        // lanes of k-group lg, step rg: k = KSPAN*lg + 8*rg + 0..7
        const char* Qs = stage + BM * kRowBytes + 8 * rg * QRB;
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(Qs + qoff[fn]));
          v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(Qs + qoff[fn] + 4 * QRB));
          uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          f.b[rg][fn] = make_uint4(l2.x, l2.y, h2.x, h2.y);
        }
      } else {
        const char* Qw = stage + (BM + wn * WTN + lr) * kRowBytes;
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          f.b[rg][fn] = *reinterpret_cast<const uint4*>(Qw + fn * MF::MN * kRowBytes + off);
      }
    }
  };
  // COMP (fp32 only): blocked accumulation. gfx950's fp32 MFMA rounds
  // after every k (its results match a sequential FMA chain bit for bit,
  // as hipBLASLt's do), so one accumulator over all of K carries ~sqrt(K)
  // roundings. With COMP each K tile's 16 products form a fresh chain of
  // four MFMAs and the tile sums are added into the accumulator, which
  // cuts the relative error of a 1024-deep product from 5.7e-7 to 1.6e-7
  // (4096-deep: 1.1e-6 to 3.0e-7), below a cache-blocked CPU sgemm's. The
  // coupled Newton root, whose fp32 iterate amplifies product rounding in
  // ill-conditioned directions, uses it; the extra adds cost 7-25% on
  // other fp32 products, which keep the plain chain.
  constexpr bool kComp = COMP && std::is_same<T, float>::value;
  auto mma = [&](const Frag& f) {
    if constexpr (kComp) {
      // one row of FN chains at a time, interleaved, so consecutive MFMAs
      // are independent
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        cvec_t t[FN];
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
          for (int ii = 0; ii < IPR; ++ii)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
              t[fn] = MF::mma(f.a[rg][fm], f.b[rg][fn], ii, (rg | ii) ? t[fn] : cvec_t{0, 0, 0, 0});
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
          for (int r = 0; r < MF::NACC; ++r) acc[fm][fn][r] += t[fn][r];
        }
      }
    } else {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
        for (int ii = 0; ii < IPR; ++ii)
#pragma unroll
          for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = MF::mma(f.a[rg][fm], f.b[rg][fn], ii, acc[fm][fn]);
    }
  };

  // Skewed pipeline: during step s the wave issues the LDS reads of tile
  // s+1 into one register set, then the MFMAs of tile s from the other set
  // (read during step s-1), with the DMA of tile s+NS-1 spread between
  // them; LDS latency hides behind a whole tile of MFMAs and the memory
  // unit's queue never holds up MFMA issue. One barrier per step covers
  // both hazards: every wave has waited for its reads (lgkmcnt(0)) before
  // arriving, so the stage of tile s-1 may be refilled, and every wave's
  // part of tile s+1 has landed (vmcnt: only tiles s+2 .. s+NS-2 may be
  // outstanding). The launchers require K to be a multiple of NS tiles, so
  // every step of the unrolled group is a real one and the MFMAs need no
  // branch.
  const int KT = g.K / BK;
  if constexpr (KG == 2) {
    // K groups: waves 0..NWG-1 (group 0) take the even K tiles, the others
    // the odd ones, each group accumulating the whole tile in its own
    // registers (summed after the loop). Intervals j = 0 .. KT, each ended
    // by lgkmcnt(0), vmcnt(2·IPW) and a barrier: in interval j the group of
    // tile j reads it (R) into its one register set while the other group
    // issues the MFMAs of tile j-1 (M), and every wave issues its share of
    // the DMA of tile j+3 into the stage of tile j-1 (read in interval j-1).
    // vmcnt(2·IPW) leaves only tiles j+2, j+3 in flight, so tile j+1 has
    // landed when interval j+1 reads it. Per group this is R, M, R, M, ...
    // over its own tiles, group 1 starting one interval late and group 0
    // ending one late, so both run KT + 1 intervals.
    if (KT > 0) {
      Frag f;
      issue(0, st0);
      issue(min(1, KT - 1), st1);
      issue(min(2, KT - 1), st2);
      __builtin_amdgcn_s_waitcnt(PTO_VMCNT(2 * IPW));
      stage_barrier();
#define PTO_KG_END()                                          \
  __builtin_amdgcn_s_waitcnt(PTO_VMCNT(2 * IPW));             \
  __builtin_amdgcn_sched_barrier(0);                          \
  stage_barrier();                                            \
  __builtin_amdgcn_sched_barrier(0);
#define PTO_KG_R(J, RD, DMA)                                  \
  if (!idle) load_frags(RD, f);                               \
  issue(min((J) + 3, KT - 1), DMA);                           \
  PTO_KG_END()
#define PTO_KG_M(J, DMA)                                      \
  if (!idle) mma(f);                                          \
  issue(min((J) + 3, KT - 1), DMA);                           \
  PTO_KG_END()
      if (kg == 0) {
        // tiles 4v and 4v+2: intervals 4v .. 4v+3
        for (int v = 0; v < KT; v += kStages) {
          PTO_KG_R(v, st0, st3)
          PTO_KG_M(v + 1, st0)
          PTO_KG_R(v + 2, st2, st1)
          PTO_KG_M(v + 3, st2)
        }
        issue(KT - 1, st3);  // interval KT (tile KT-1 is group 1's)
        PTO_KG_END()
      } else {
        issue(min(3, KT - 1), st3);  // interval 0 (tile 0 is group 0's)
        PTO_KG_END()
        // tiles 4v+1 and 4v+3: intervals 4v+1 .. 4v+4
        for (int v = 0; v < KT; v += kStages) {
          PTO_KG_R(v + 1, st1, st0)
          PTO_KG_M(v + 2, st1)
          PTO_KG_R(v + 3, st3, st2)
          PTO_KG_M(v + 4, st3)
        }
      }
#undef PTO_KG_R
#undef PTO_KG_M
#undef PTO_KG_END
      __builtin_amdgcn_s_waitcnt(PTO_VMCNT(0));
      stage_barrier();
    }
  } else if constexpr (Cfg::PP) {
    // Ping-pong: waves 0-3 (group 0) and 4-7 (group 1), one of each per
    // SIMD, run the same sequence of phases, group 1 one phase behind:
    //   R(t): LDS reads of tile t into the one register set, DMA of tile
    //         t+3 into the stage of tile t-1;   M(t): the MFMAs of tile t;
    // with a barrier after every phase. While one group issues its MFMAs
    // the other reads, so the SIMD's MFMA pipe is not left idle by both of
    // its waves waiting on the same barrier. Every phase ends with
    // lgkmcnt(0) and vmcnt(2·IPW) (only tiles t+2, t+3 may be in flight),
    // which orders: tile t+1 landed before group 0 reads it (group 1's part
    // is waited at the end of its R(t), one phase earlier); a stage's old
    // tile read by both groups before either refills it (three phases
    // apart). Both groups execute 2·KT + 3 barriers.
    if (KT > 0) {
      const int grp = wm;
      Frag f;
      issue(0, st0);
      issue(min(1, KT - 1), st1);
      issue(min(2, KT - 1), st2);
      __builtin_amdgcn_s_waitcnt(PTO_VMCNT(2 * IPW));
      stage_barrier();
      if (grp) {
        __builtin_amdgcn_sched_barrier(0);
        stage_barrier();
        __builtin_amdgcn_sched_barrier(0);
      }
      for (int kt = 0; kt < KT; kt += kStages) {
#define PTO_PP(J, RD, DMA)                                    \
  if (!idle) load_frags(RD, f);                               \
  issue(min(kt + (J) + 3, KT - 1), DMA);                      \
  __builtin_amdgcn_s_waitcnt(PTO_VMCNT(2 * IPW));             \
  __builtin_amdgcn_sched_barrier(0);                          \
  stage_barrier();                                            \
  __builtin_amdgcn_sched_barrier(0);                          \
  if (!idle) mma(f);                                          \
  __builtin_amdgcn_s_waitcnt(PTO_VMCNT(2 * IPW));             \
  __builtin_amdgcn_sched_barrier(0);                          \
  stage_barrier();                                            \
  __builtin_amdgcn_sched_barrier(0);
        PTO_PP(0, st0, st3)
        PTO_PP(1, st1, st0)
        PTO_PP(2, st2, st1)
        PTO_PP(3, st3, st2)
#undef PTO_PP
      }
      if (!grp) stage_barrier();
      __builtin_amdgcn_s_waitcnt(PTO_VMCNT(0));
      stage_barrier();
    }
  } else if (KT > 0) {
    Frag f0, f1;
    issue(0, st0);
    issue(min(1, KT - 1), st1);
    issue(min(2, KT - 1), st2);
    if constexpr (NS == 8) {
      issue(min(3, KT - 1), st3);
      issue(min(4, KT - 1), st4);
      issue(min(5, KT - 1), st5);
      issue(min(6, KT - 1), st6);
    }
    __builtin_amdgcn_s_waitcnt(PTO_VMCNT((NS - 2) * IPW));
    stage_barrier();
    load_frags(st0, f0);
    for (int kt = 0; kt < KT; kt += NS) {
      // J: step in the unrolled group; RD: stage of tile kt+J+1; DMA:
      // stage of tile kt+J+NS-1
#define PTO_STEP(J, CUR, NXT, RD, DMA)                                \
  __builtin_amdgcn_s_waitcnt(PTO_VMCNT((NS - 3) * IPW));              \
  stage_barrier();                                                    \
  load_frags(RD, NXT);                                                \
  issue(min(kt + (J) + NS - 1, KT - 1), DMA);                         \
  mma(CUR);                                                           \
  if constexpr (!kSpreadReads)                                        \
    __builtin_amdgcn_sched_group_barrier(0x100, kFragReads, 0);       \
  for (int q = 0; q < IPW; ++q) {                                     \
    if constexpr (kSpreadReads)                                       \
      __builtin_amdgcn_sched_group_barrier(0x100, kFragReads / IPW, 0); \
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                \
    __builtin_amdgcn_sched_group_barrier(0x008, kTileMfma / IPW, 0);  \
  }
      if constexpr (NS == 4) {
        PTO_STEP(0, f0, f1, st1, st3)
        PTO_STEP(1, f1, f0, st2, st0)
        PTO_STEP(2, f0, f1, st3, st1)
        PTO_STEP(3, f1, f0, st0, st2)
      } else {
        PTO_STEP(0, f0, f1, st1, st7)
        PTO_STEP(1, f1, f0, st2, st0)
        PTO_STEP(2, f0, f1, st3, st1)
        PTO_STEP(3, f1, f0, st4, st2)
        PTO_STEP(4, f0, f1, st5, st3)
        PTO_STEP(5, f1, f0, st6, st4)
        PTO_STEP(6, f0, f1, st7, st5)
        PTO_STEP(7, f1, f0, st0, st6)
      }
#undef PTO_STEP
    }
    __builtin_amdgcn_s_waitcnt(PTO_VMCNT(0));  // stray prefetches land before reuse
    stage_barrier();
  }

  // Epilogue, per wave and staged through LDS so every global access of the
  // functor is a run of up to 8 consecutive elements of one output row.
  // Each wave owns a private slice (RPP rows of its WTM x WTN sub-tile at a
  // time), so no cross-wave synchronisation is needed:
  //   1. the functor's global reads for all of this lane's direct runs are
  //      issued (epi.load), then the wave writes RPP rows of raw
  //      accumulators to its slice while they are in flight;
  //   2. direct pass: runs along output rows (i, j..j+7) -> epi.put, which
  //      hands back the value the transposed pass should see;
  //   3. transposed pass (mirror of a symmetric tile, or the functor's
  //      transposed copy): reads for all runs (epi.load_t), then runs along
  //      (j, i..i+7) -> epi.put_t.
  // Reading before writing keeps one memory latency per pass instead of
  // one per run: a functor may read and write the same array (X' = a·X + v
  // in place), so the compiler cannot hoist a run's read above the
  // previous run's store by itself. Each run reads and writes only its own
  // elements, and the direct and transposed runs of one tile cover
  // disjoint positions, so the early reads see the values from before the
  // launch.
  // In symmetric (UPPER) products the value for (i, j), i <= j, is stored
  // at (i, j) by its own direct pass and at (j, i) by its transposed pass,
  // so the stored matrix is exactly symmetric. On diagonal tiles the 8x8
  // blocks on the diagonal are written whole by the direct pass, each
  // position below the diagonal taking the staged value of its mirror
  // (j, i), so every run stays a full 16-byte access (partial runs there
  // made the diagonal tiles' epilogue 1.5-2x longer than the others' and
  // the last to finish); the transposed pass covers the rest below the
  // diagonal.
  constexpr int RPP = Plan::RPP, SP = Plan::SP, WTE = Plan::WTE;
  const int wa = wave / Plan::WPA;  // < NS
  char* arr = wa == 0 ? st0 : wa == 1 ? st1 : wa == 2 ? st2 : wa == 3 ? st3 : wa == 4 ? st4 : wa == 5 ? st5 : wa == 6 ? st6 : st7;
  S* stg = reinterpret_cast<S*>(arr) + (wave % Plan::WPA) * RPP * SP;
  const bool diag = UPPER && ti == tj;
  const bool need_t = UPPER || epi.has_t();
  const int wr0 = row0 + wm * WTM, wc0 = col0 + wn * WTN;  // sub-tile origin
  const int nrem = g.N - wc0;
  // direct runs: 8 lanes cover 64 consecutive columns of one row
  constexpr int RUNS = WTN / 8;  // 8-element runs per row
  // lanes per output row: the largest divisor of RUNS that is at most 8
  constexpr int LGD = RUNS % 8 == 0 ? 8 : RUNS % 6 == 0 ? 6 : RUNS % 4 == 0 ? 4 : RUNS % 2 == 0 ? 2 : 1;
  constexpr int RPB = 64 / LGD;
  constexpr int CBLK = RUNS / LGD;
  static_assert(RUNS % LGD == 0 && LGD * 8 <= 64, "wave tile width: whole 8-element runs");
  constexpr int ITEMS = ((RPP + RPB - 1) / RPB) * CBLK;  // direct runs per lane
  // when LGD does not divide 64 (wave tiles 48 wide) the last 64 % LGD lanes
  // would repeat the next block's first runs: they sit out
  const bool lane_ok = LGD * RPB == 64 || lane < LGD * RPB;
  // transposed runs: 8 lanes share a column c and cover 64 consecutive rows
  constexpr int CBT = WTN / 8;
  constexpr int ITEMS_T = ((RPP / 8 + 7) / 8) * CBT;
  if constexpr (KG == 2) {
    // Sum the two groups' partial tiles: each wave keeps WTE rows of its
    // sub-tile (group 0 the first half, group 1 the second) and hands the
    // other half to its partner (same wm, wn, other group) through LDS,
    // 16 bytes per lane per fragment, lane-minor (each instruction writes
    // one contiguous KiB). Every wave adds the other group's values to its
    // own, so both halves hold (even tiles) + (odd tiles).
    constexpr int HF = FM / 2, PER = HF * FN;
    static_assert(sizeof(cvec_t) == 16 && NW <= 2 * NS && 2 * PER * 1024 <= Plan::ARR,
                  "K-group exchange: 4-byte accumulators, two waves per stage array");
    // wave w's block: half of stage array w / 2
#define PTO_SLOT(w) \
  (((w) / 2 == 0 ? st0 : (w) / 2 == 1 ? st1 : (w) / 2 == 2 ? st2 : st3) + ((w) & 1) * (PER * 1024))
#define PTO_EXCHANGE(SEND, KEEP)                                                  \
  {                                                                               \
    char* mine = PTO_SLOT(wave);                                                  \
    _Pragma("unroll") for (int e = 0; e < PER; ++e)                               \
        *reinterpret_cast<cvec_t*>(mine + (e * 64 + lane) * 16) =                 \
            acc[(SEND) + e / FN][e % FN];                                         \
    stage_barrier();                                                              \
    const char* theirs = PTO_SLOT(kg ? wave - NWG : wave + NWG);                  \
    _Pragma("unroll") for (int e = 0; e < PER; ++e) {                             \
      const cvec_t o = *reinterpret_cast<const cvec_t*>(theirs + (e * 64 + lane) * 16); \
      _Pragma("unroll") for (int r = 0; r < MF::NACC; ++r)                        \
          acc[(KEEP) + e / FN][e % FN][r] += o[r];                                \
    }                                                                             \
    stage_barrier(); /* the arrays host the epilogue staging next */             \
  }
    if (kg == 0)
      PTO_EXCHANGE(HF, 0)
    else
      PTO_EXCHANGE(0, HF)
#undef PTO_EXCHANGE
#undef PTO_SLOT
  }
  // The epilogue for the fragment rows EFM .. EFM + WTE/16 - 1 of this
  // wave's sub-tile (all of them, or with K groups its half), written
  // out with a constant EFM so that acc stays in registers.
#define PTO_STORE_ROWS(EFM)                                                                          \
_Pragma("unroll")                                                                                    \
  for (int hp = 0; hp < WTE / RPP; ++hp) {                                                           \
    const int pr0 = wr0 + (EFM) * MF::MN + hp * RPP;  /* first output row of this pass */            \
    if (pr0 >= g.M || nrem <= 0) break;                                                              \
    const int rows = min(RPP, g.M - pr0);                                                            \
    typename Epi::Pre pre[ITEMS];                                                                    \
_Pragma("unroll")                                                                                    \
    for (int it = 0; it < ITEMS; ++it) {                                                             \
      const int r = (it / CBLK) * RPB + lane / LGD;                                                  \
      const int c = ((it % CBLK) * LGD + lane % LGD) * 8;                                            \
      const int i = pr0 + r, j0 = wc0 + c;                                                           \
      const int n = min(8, nrem - c);                                                                \
      /* diagonal tiles: skip runs below the diagonal; a run inside an 8x8 block on it is full */     \
      const int kbeg = diag && i - j0 >= 8 ? 8 : 0;                                                  \
      if (lane_ok && r < rows && c < nrem && kbeg < n) epi.load(b, i, j0, kbeg, n, pre[it]);         \
    }                                                                                                \
_Pragma("unroll")                                                                                    \
    for (int fm = (EFM) + hp * (RPP / MF::MN); fm < (EFM) + (hp + 1) * (RPP / MF::MN); ++fm)         \
_Pragma("unroll")                                                                                    \
      for (int fn = 0; fn < FN; ++fn)                                                                \
_Pragma("unroll")                                                                                    \
        for (int r = 0; r < MF::NACC; ++r) {                                                         \
          const int li = (fm - (EFM)) * MF::MN - hp * RPP + MF::row(lane, r);                        \
          const int lj = fn * MF::MN + MF::col(lane, r);                                             \
          stg[li * SP + lj] = static_cast<S>(acc[fm][fn][r]);                                        \
        }                                                                                            \
    __builtin_amdgcn_s_waitcnt(PTO_LGKM0);                                                           \
    __builtin_amdgcn_wave_barrier();                                                                 \
_Pragma("unroll")                                                                                    \
    for (int it = 0; it < ITEMS; ++it) {                                                             \
      const int r = (it / CBLK) * RPB + lane / LGD;                                                  \
      const int c = ((it % CBLK) * LGD + lane % LGD) * 8;                                            \
      const int i = pr0 + r, j0 = wc0 + c;                                                           \
      const int n = min(8, nrem - c);                                                                \
      const int kbeg = diag && i - j0 >= 8 ? 8 : 0;                                                  \
      if (!(lane_ok && r < rows && c < nrem && kbeg < n)) continue;                                  \
      /* dk in 1..7: the run crosses the diagonal; its positions k < dk lie below it and take the  \
         mirrored value, staged at row j0 + k, column i of the same slab (the 16-aligned slab holds \
         the whole 8-row group; those diagonal-block entries are never written back) */            \
      S v[8], vo[8];                                                                                 \
_Pragma("unroll")                                                                                    \
      for (int k = 0; k < 8; ++k) v[k] = stg[r * SP + c + k];                                        \
      if (diag && i - j0 > 0) {                                                                      \
        const int dk = i - j0;                                                                       \
_Pragma("unroll")                                                                                    \
        for (int k = 0; k < 7; ++k)                                                                  \
          if (k < dk) v[k] = stg[(c + k - (pr0 - wc0)) * SP + r + (pr0 - wc0)];                      \
      }                                                                                              \
      epi.put(b, i, j0, v, kbeg, n, pre[it], vo);                                                    \
      if (need_t && !Epi::kVoIsV && !(diag && i - j0 >= 0)) {                                        \
_Pragma("unroll")                                                                                    \
        for (int k = 0; k < 8; ++k) stg[r * SP + c + k] = vo[k];                                     \
      }                                                                                              \
    }                                                                                                \
    if (need_t) {                                                                                    \
      if constexpr (!Epi::kVoIsV) {  /* the write-back above must land first */                      \
        __builtin_amdgcn_s_waitcnt(PTO_LGKM0);                                                       \
        __builtin_amdgcn_wave_barrier();                                                             \
      }                                                                                              \
  /* output row j = wc0 + c, columns i = pr0 + r..r+7 */                                             \
      typename Epi::PreT pret[ITEMS_T];                                                              \
_Pragma("unroll")                                                                                    \
      for (int it = 0; it < ITEMS_T; ++it) {                                                         \
        const int c = (it % CBT) * 8 + lane / 8;                                                     \
        const int r = ((it / CBT) * 8 + lane % 8) * 8;                                               \
        const int j = wc0 + c, i0 = pr0 + r;                                                         \
        int n = min(8, rows - r);                                                                    \
        if (diag && j - i0 < 8) n = 0;  /* below the diagonal, outside its 8x8 blocks */             \
        if (c < nrem && r < rows && n > 0) epi.load_t(b, j, i0, n, pret[it]);                        \
      }                                                                                              \
_Pragma("unroll")                                                                                    \
      for (int it = 0; it < ITEMS_T; ++it) {                                                         \
        const int c = (it % CBT) * 8 + lane / 8;                                                     \
        const int r = ((it / CBT) * 8 + lane % 8) * 8;                                               \
        const int j = wc0 + c, i0 = pr0 + r;                                                         \
        int n = min(8, rows - r);                                                                    \
        if (diag && j - i0 < 8) n = 0;                                                               \
        if (!(c < nrem && r < rows && n > 0)) continue;                                              \
        S v[8];                                                                                      \
_Pragma("unroll")                                                                                    \
        for (int k = 0; k < 8; ++k) v[k] = k < n ? stg[(r + k) * SP + c] : S(0);                     \
        epi.put_t(b, j, i0, v, n, pret[it]);                                                         \
      }                                                                                              \
    }                                                                                                \
    __builtin_amdgcn_s_waitcnt(PTO_LGKM0);                                                           \
    __builtin_amdgcn_wave_barrier();                                                                 \
  }
  if constexpr (KG == 1) {
    PTO_STORE_ROWS(0)
  } else {
    if (kg == 0) {
      PTO_STORE_ROWS(0)
    } else {
      PTO_STORE_ROWS(FM / 2)
    }
  }
#undef PTO_STORE_ROWS
  epi.finish(b);
}

// ------------------------------------------------------------- host launch

// Tile choices per element type: full products and symmetric (upper-tile)
// products, each with a "big" tile and a "small" one. Symmetric products
// need square tiles. kBigRate is the big tile's throughput per CU relative
// to the small tile's (area per unit time, measured on MI355X over square
// and rectangular products from 512 to 11008): the big tile reuses each
// staged operand byte for more MFMA work. bf16 symmetric products also
// have a 192 x 192 "mid" tile (kMidRate, same units): a 4096² symmetric
// product has 136 upper tiles of 256² for 256 CUs but 253 of 192², one
// full round.
template <typename T>
struct TileSet;
template <>
struct TileSet<bf16> {
  // the 256² tiles run the ping-pong schedule (measured +1% on batched NS5,
  // and no spills in the update and square kernels)
  typedef Tile<256, 256, 32, 2, 4, 4, true> big;
  typedef Tile<128, 128, 32, 2, 2> small;
  typedef Tile<256, 256, 32, 2, 4, 4, true> sym_big;
  typedef Tile<128, 128, 32, 2, 2> sym_small;
  // the 192² tile: two K groups of four 96×96 waves (LDS bytes per MFMA
  // as the 256² tile's; K-FAC Gram and one-matrix NS5 products −1–5%)
  typedef Tile<192, 192, 32, 2, 2, 4, false, 2> sym_mid;
  typedef sym_small sym_tiny;  // unused
  static constexpr bool kHasMid = true, kHasTiny = false, kMidAll = false;
  static constexpr double kBigRate = 1.5;
  static constexpr double kMidRate = 1.35;
  static constexpr double kTinyRate = 0.0;
};
// fp32 symmetric products also have a 32 x 32 "tiny" tile (4 waves of
// 16 x 16): an n = 1024 product is 136 upper tiles of 64² (120 of 256 CUs
// idle) but 528 of 32², about two co-resident workgroups per CU.
template <>
struct TileSet<float> {
  typedef Tile<128, 128, 16, 2, 2> big;
  typedef Tile<64, 64, 16, 2, 2, 8> small;
  typedef big sym_big;
  typedef small sym_small;
  typedef Tile<192, 192, 16, 2, 4> sym_mid;
  typedef Tile<32, 32, 16, 2, 2, 8> sym_tiny;
  static constexpr bool kHasMid = true, kHasTiny = true, kMidAll = false;
  static constexpr double kBigRate = 1.22;
  static constexpr double kMidRate = 1.3;
  static constexpr double kTinyRate = 0.85;
};
// fp64 products choose among 128² (8 waves of 64×32), 64² and 32² tiles,
// symmetric or not: the 128² tile ran the 96 × 2048² per-matrix fp64 roots
// of a Shampoo refresh 10% faster than 64² (1241–1252 → 1116–1122 ms, same
// roots; an 8-stage ring or 4×2 waves measured the same); the 64² and 32²
// tiles keep smaller products on the CUs (a 1024² product on one round of
// 64² tiles, a symmetric 2048² one on nine of 32²).
template <>
struct TileSet<double> {
  typedef Tile<128, 128, 8, 2, 4> big;
  typedef Tile<32, 32, 8, 2, 2> small;
  typedef big sym_big;
  typedef small sym_small;
  typedef Tile<64, 64, 8, 2, 2> sym_mid;  // the mid tile of every fp64 product
  typedef small sym_tiny;                 // unused
  static constexpr bool kHasMid = true, kHasTiny = false, kMidAll = true;
  static constexpr double kBigRate = 1.39;
  static constexpr double kMidRate = 1.25;
  static constexpr double kTinyRate = 0.0;
};

// K granularity of a type's products: every tile's ring of K tiles (at
// most kPadK elements, the pitch every operand buffer is padded to).
template <typename T>
constexpr int ring_k() {
  typedef TileSet<T> S;
  int r = 0;
  for (int v : {S::big::NS * S::big::BK, S::small::NS * S::small::BK, S::sym_big::NS * S::sym_big::BK,
                S::sym_small::NS * S::sym_small::BK, S::sym_mid::NS * S::sym_mid::BK,
                S::sym_tiny::NS * S::sym_tiny::BK})
    r = v > r ? v : r;
  return r;
}
static_assert(kPadK % ring_k<bf16>() == 0 && kPadK % ring_k<float>() == 0 && kPadK % ring_k<double>() == 0,
              "padded K covers every ring");

// Compute units of the current device (256 on a full MI355X), cached per
// device ordinal.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <typename T, class Cfg, bool UPPER, class Epi, bool QN = false, bool PT = false, bool COMP = false>
int launch_gemm_cfg(GemmArgs g, const Epi& epi, int batch, hipStream_t stream, const char* name) {
  g.tiles_m = (g.M + Cfg::BM - 1) / Cfg::BM;
  g.tiles_n = (g.N + Cfg::BN - 1) / Cfg::BN;
  g.cus = device_cus();
  int64_t tiles = UPPER ? (int64_t)g.tiles_m * (g.tiles_m + 1) / 2 : (int64_t)g.tiles_m * g.tiles_n;
  if (tiles == 0 || batch == 0) return 0;
  // the kernel numbers workgroups across the batch in 32-bit arithmetic
  PTO_REQUIRE(batch < 65536 && tiles * batch < (1ll << 31), std::string(name) + ": grid too large");
  ProfScope ps(name, stream);
  hipLaunchKernelGGL((gemm_nt_kernel<T, Cfg, UPPER, Epi, QN, PT, COMP>), dim3((unsigned)tiles, (unsigned)batch),
                     dim3(Cfg::NT), 0, stream, g, epi);
  PTO_LAUNCHED(name);
  return 0;
}

template <typename T, bool UPPER>
struct PickTiles {
  typedef typename TileSet<T>::big Big;
  typedef typename TileSet<T>::small Small;
};
template <typename T>
struct PickTiles<T, true> {
  typedef typename TileSet<T>::sym_big Big;
  typedef typename TileSet<T>::sym_small Small;
};

// Tiles are spread over the CUs, so the product ends when the busiest CU has
// run ceil(tiles / CUs) of them. Pick the tile size whose busiest CU covers
// the least area after weighting each size by its measured rate (small 1.0,
// big kBigRate, the mid tile kMidRate: symmetric products only, unless the
// type's kMidAll). At the same number of tiles per CU the big tile wins; a
// big tiling that leaves half the CUs idle (e.g. 64 big tiles against 256
// small ones) loses. Returns 0 = small, 1 = big, 2 = mid, 3 = tiny.
template <typename T, bool UPPER>
int pick_tile(int64_t M, int64_t N, int64_t batch) {
  typedef typename PickTiles<T, UPPER>::Big Big;
  typedef typename PickTiles<T, UPPER>::Small Small;
  typedef typename TileSet<T>::sym_mid Mid;
  const int64_t cus = device_cus();
  auto load = [&](int bm, int bn, double rate) {
    const int64_t tm = (M + bm - 1) / bm, tn = (N + bn - 1) / bn;
    const int64_t tiles = (UPPER ? tm * (tm + 1) / 2 : tm * tn) * batch;
    return double((tiles + cus - 1) / cus) * (bm * bn) / rate;
  };
  double best = load(Small::BM, Small::BN, 1.0);
  int pick = 0;
  const double big = load(Big::BM, Big::BN, TileSet<T>::kBigRate);
  if (big < best) {
    best = big;
    pick = 1;
  }
  if ((UPPER || TileSet<T>::kMidAll) && TileSet<T>::kHasMid && load(Mid::BM, Mid::BN, TileSet<T>::kMidRate) < best) {
    best = load(Mid::BM, Mid::BN, TileSet<T>::kMidRate);
    pick = 2;
  }
  if (UPPER && TileSet<T>::kHasTiny) {
    typedef typename TileSet<T>::sym_tiny Tiny;
    if (load(Tiny::BM, Tiny::BN, TileSet<T>::kTinyRate) < best) pick = 3;
  }
  return pick;
}

// Validate the operand contract and pick a tile size. COMP: blocked fp32
// accumulation (see the main loop).
template <typename T, bool UPPER, class Epi, bool COMP = false>
int launch_gemm(const GemmArgs& g, const Epi& epi, int batch, hipStream_t stream, const char* name) {
  typedef typename PickTiles<T, UPPER>::Big Big;
  typedef typename PickTiles<T, UPPER>::Small Small;
  static_assert(!UPPER || (Big::BM == Big::BN && Small::BM == Small::BN), "symmetric products need square tiles");
  PTO_REQUIRE(g.M >= 0 && g.N >= 0 && g.K >= 0, std::string(name) + ": negative extent");
  PTO_REQUIRE(!UPPER || g.M == g.N, std::string(name) + ": symmetric product needs M == N");
  PTO_REQUIRE(g.K % ring_k<T>() == 0, std::string(name) + ": K not padded");
  PTO_REQUIRE(g.ldp % (16 / sizeof(T)) == 0 && g.ldq % (16 / sizeof(T)) == 0 &&
                  (reinterpret_cast<uintptr_t>(g.P) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(g.Q) & 15) == 0,
              std::string(name) + ": operands not 16-byte aligned");
  const int pick = pick_tile<T, UPPER>(g.M, g.N, batch);
  if constexpr ((UPPER || TileSet<T>::kMidAll) && TileSet<T>::kHasMid) {
    typedef typename TileSet<T>::sym_mid Mid;
    static_assert(Mid::BM == Mid::BN && Mid::BK == Big::BK, "mid tile: square, same K tile");
    if (pick == 2) return launch_gemm_cfg<T, Mid, UPPER, Epi, false, false, COMP>(g, epi, batch, stream, name);
  }
  if constexpr (UPPER && TileSet<T>::kHasTiny) {
    typedef typename TileSet<T>::sym_tiny Tiny;
    static_assert(Tiny::BM == Tiny::BN && Tiny::BK == Big::BK, "tiny tile: square, same K tile");
    if (pick == 3) return launch_gemm_cfg<T, Tiny, UPPER, Epi, false, false, COMP>(g, epi, batch, stream, name);
  }
  if (pick == 1) return launch_gemm_cfg<T, Big, UPPER, Epi, false, false, COMP>(g, epi, batch, stream, name);
  return launch_gemm_cfg<T, Small, UPPER, Epi, false, false, COMP>(g, epi, batch, stream, name);
}

// C[b](i,j) = sum_k P[b](i,k) * Q[b](k,j) with Q stored [K][N] (row pitch
// ldq, N contiguous), bf16 only. Q must hold K rows of ldq elements, and
// its rows past the true contraction length must be zero (as the pad
// columns of P are). With PT, P is stored [K][M] as well (row pitch ldp,
// ldp >= M, K rows, the rows past the true K zero) — for a symmetric P
// that is P itself. UPPER (with PT): a symmetric product on upper tiles,
// mirrored, as in launch_gemm.
// pick: the tile (pick_tile's codes), or -1 to let pick_tile choose.
template <class Epi, bool PT = false, bool UPPER = false>
int launch_gemm_qn(const GemmArgs& g, const Epi& epi, int batch, hipStream_t stream, const char* name,
                   int pick = -1) {
  static_assert(PT || !UPPER, "symmetric QN products need PT");
  typedef typename PickTiles<bf16, UPPER>::Big Big;
  typedef typename PickTiles<bf16, UPPER>::Small Small;
  PTO_REQUIRE(g.M >= 0 && g.N >= 0 && g.K >= 0, std::string(name) + ": negative extent");
  PTO_REQUIRE(!UPPER || g.M == g.N, std::string(name) + ": symmetric product needs M == N");
  PTO_REQUIRE(g.K % ring_k<bf16>() == 0, std::string(name) + ": K not padded");
  PTO_REQUIRE(g.ldq < (int64_t(1) << 26) && g.ldp < (int64_t(1) << 26),
              std::string(name) + ": row pitch too large");  // 64-byte K steps in 32 bits
  PTO_REQUIRE(g.ldp % 8 == 0 && g.ldq % 8 == 0 && g.ldq >= g.N && g.ldq >= 8 && (!PT || (g.ldp >= g.M && g.ldp >= 8)) &&
                  (reinterpret_cast<uintptr_t>(g.P) & 15) == 0 && (reinterpret_cast<uintptr_t>(g.Q) & 15) == 0,
              std::string(name) + ": operands not 16-byte aligned");
  PTO_REQUIRE(pick >= -1 && pick <= 2 && (UPPER || pick != 2), std::string(name) + ": tile choice");
  if (pick < 0) pick = pick_tile<bf16, UPPER>(g.M, g.N, batch);
  if constexpr (UPPER) {
    // the 192² tile: 384-byte transposing rows (swzq's second form)
    typedef typename TileSet<bf16>::sym_mid Mid;
    static_assert(Mid::BM == Mid::BN && Mid::BK == Big::BK, "mid tile: square, same K tile");
    if (pick == 2) return launch_gemm_cfg<bf16, Mid, UPPER, Epi, true, PT>(g, epi, batch, stream, name);
  }
  if (pick == 1) return launch_gemm_cfg<bf16, Big, UPPER, Epi, true, PT>(g, epi, batch, stream, name);
  return launch_gemm_cfg<bf16, Small, UPPER, Epi, true, PT>(g, epi, batch, stream, name);
}

// ------------------------------------------------------------- epilogues
// Functor interface (S = staging/accumulation type):
//   Pre, PreT                            what a direct / transposed run
//       reads from global memory before it writes (empty if nothing);
//   load(b, i, j0, kbeg, n, Pre&)        issue those reads for a direct run;
//   put(b, i, j0, v[8], kbeg, n, pre, vo[8])  output row i, columns j0+k
//       for k in [kbeg, n); vo receives what the transposed pass should see;
//   load_t(b, j, i0, n, PreT&)           reads for a transposed run;
//   put_t(b, j, i0, v[8], n, pre_t)      output row j, columns i0+k, k < n
//       (the mirror of a symmetric product, or a transposed copy);
//   has_t()                              whether put_t is needed outside
//       symmetric products;
//   kVoIsV                               vo is always v (the staged values
//       then serve the transposed pass as they are);
//   finish(b)                            once per thread at the end.
// j0 and i0 are multiples of 8; `vec` (set by the host when the row pitch,
// batch stride and base allow) enables 16-byte accesses for full runs.

struct NoPre {};

template <typename T>
__device__ __forceinline__ bool full_run(bool vec, int kbeg, int n) {
  return vec && kbeg == 0 && n == 8;
}

// out[k] = p[k] for k in [kbeg, n)
template <typename T, typename S>
__device__ __forceinline__ void ld8(const T* p, S* out, int kbeg, int n, bool vec) {
  if (full_run<T>(vec, kbeg, n)) {
    if constexpr (sizeof(T) == 2) {
      uint4 u = *reinterpret_cast<const uint4*>(p);
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int k = 0; k < 8; ++k) out[k] = static_cast<S>(to_f(e[k]));
    } else if constexpr (sizeof(T) == 4) {
      float4 a = reinterpret_cast<const float4*>(p)[0], c = reinterpret_cast<const float4*>(p)[1];
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
      out[4] = c.x; out[5] = c.y; out[6] = c.z; out[7] = c.w;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        double2 d = reinterpret_cast<const double2*>(p)[q];
        out[2 * q] = static_cast<S>(d.x);
        out[2 * q + 1] = static_cast<S>(d.y);
      }
    }
  } else {
    for (int k = kbeg; k < n; ++k) out[k] = static_cast<S>(to_f(p[k]));
  }
}

// p[k] = in[k] for k in [kbeg, n), converted to T
template <typename T, typename S>
__device__ __forceinline__ void st8(T* p, const S* in, int kbeg, int n, bool vec) {
  if (full_run<T>(vec, kbeg, n)) {
    if constexpr (sizeof(T) == 2) {
      uint4 u;
      T* e = reinterpret_cast<T*>(&u);
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = convert<T>(in[k]);
      *reinterpret_cast<uint4*>(p) = u;
    } else if constexpr (sizeof(T) == 4) {
      reinterpret_cast<float4*>(p)[0] = make_float4(convert<float>(in[0]), convert<float>(in[1]),
                                                    convert<float>(in[2]), convert<float>(in[3]));
      reinterpret_cast<float4*>(p)[1] = make_float4(convert<float>(in[4]), convert<float>(in[5]),
                                                    convert<float>(in[6]), convert<float>(in[7]));
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        reinterpret_cast<double2*>(p)[q] = make_double2(static_cast<double>(in[2 * q]),
                                                        static_cast<double>(in[2 * q + 1]));
    }
  } else {
    for (int k = kbeg; k < n; ++k) p[k] = convert<T>(in[k]);
  }
}

// Eight elements of T held in their storage format between the read and
// the use, so a pending run costs 4 (bf16), 8 (fp32) or 16 (fp64) VGPRs.
template <typename T>
struct Raw8 {
  uint4 w[sizeof(T) / 2];
};

// Early read of a full run (16-byte loads straight into r). Partial runs
// (matrix edges, diagonal tiles) are read at use time by ld8_use instead:
// filling single elements of r here would make the compiler split the
// full-run registers, and so wait for the loads, right after issuing them.
template <typename T>
__device__ __forceinline__ void ld8_pre(const T* p, Raw8<T>& r, int kbeg, int n, bool vec) {
  if (full_run<T>(vec, kbeg, n)) {
#pragma unroll
    for (int q = 0; q < (int)(sizeof(T) / 2); ++q) r.w[q] = reinterpret_cast<const uint4*>(p)[q];
  }
}

// out[k] = p[k] for k in [kbeg, n), from r if ld8_pre read the run. The
// unpacking works on whole 32-bit words (a bf16 is the high half of the
// float with the same value) so the registers stay whole until here.
template <typename T, typename S>
__device__ __forceinline__ void ld8_use(const T* p, const Raw8<T>& r, S* out, int kbeg, int n, bool vec) {
  if (full_run<T>(vec, kbeg, n)) {
    if constexpr (sizeof(T) == 2) {
      const unsigned w[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        out[2 * q] = static_cast<S>(__uint_as_float(w[q] << 16));
        out[2 * q + 1] = static_cast<S>(__uint_as_float(w[q] & 0xffff0000u));
      }
    } else if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        out[4 * q] = static_cast<S>(__uint_as_float(r.w[q].x));
        out[4 * q + 1] = static_cast<S>(__uint_as_float(r.w[q].y));
        out[4 * q + 2] = static_cast<S>(__uint_as_float(r.w[q].z));
        out[4 * q + 3] = static_cast<S>(__uint_as_float(r.w[q].w));
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        out[2 * q] = static_cast<S>(__hiloint2double((int)r.w[q].y, (int)r.w[q].x));
        out[2 * q + 1] = static_cast<S>(__hiloint2double((int)r.w[q].w, (int)r.w[q].z));
      }
    }
  } else {
    for (int k = kbeg; k < n; ++k) out[k] = static_cast<S>(to_f(p[k]));
  }
}

// Host-side check that a [.., ld] buffer allows 16-byte runs of 8 elements.
template <typename T>
inline bool vec_ok(const void* p, int64_t ld, int64_t sb) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && ld % 8 == 0 && sb % 8 == 0;
}

// dst = v
template <typename TO, typename A>
struct EpiStore {
  typedef A S;
  TO* dst;
  int64_t ld, sd;
  bool vec;
  typedef NoPre Pre;
  typedef NoPre PreT;
  static constexpr bool kVoIsV = true;
  __device__ __forceinline__ bool has_t() const { return false; }
  __device__ __forceinline__ void load(int, int, int, int, int, Pre&) const {}
  __device__ __forceinline__ void load_t(int, int, int, int, PreT&) const {}
  __device__ __forceinline__ void put(int b, int i, int j0, const S* v, int kbeg, int n, const Pre&, S* vo) const {
    st8<TO, S>(dst + (int64_t)b * sd + (int64_t)i * ld + j0, v, kbeg, n, vec);
#pragma unroll
    for (int k = 0; k < 8; ++k) vo[k] = v[k];
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const S* v, int n, const PreT&) const {
    st8<TO, S>(dst + (int64_t)b * sd + (int64_t)j * ld + i0, v, 0, n, vec);
  }
  __device__ __forceinline__ void finish(int) const {}
};

// dst = beta * dst + alpha * v   (beta == 0 overwrites without reading dst)
template <typename TO, typename A>
struct EpiBlend {
  typedef A S;
  TO* dst;
  int64_t ld, sd;
  A beta, alpha;
  bool vec;
  typedef Raw8<TO> Pre;
  typedef Raw8<TO> PreT;
  static constexpr bool kVoIsV = true;
  __device__ __forceinline__ bool has_t() const { return false; }
  __device__ __forceinline__ void load(int b, int i, int j0, int kbeg, int n, Pre& p) const {
    if (beta != A(0)) ld8_pre<TO>(dst + (int64_t)b * sd + (int64_t)i * ld + j0, p, kbeg, n, vec);
  }
  __device__ __forceinline__ void load_t(int b, int j, int i0, int n, PreT& p) const {
    if (beta != A(0)) ld8_pre<TO>(dst + (int64_t)b * sd + (int64_t)j * ld + i0, p, 0, n, vec);
  }
  __device__ __forceinline__ void blend(TO* p, const S* v, int kbeg, int n, const Raw8<TO>& raw) const {
    S r[8];
    if (beta != A(0)) {
      S old[8];
      ld8_use<TO, S>(p, raw, old, kbeg, n, vec);
      // one fixed rounding (an explicit fma), the same in every kernel
      // instantiation that blends (single and batched factor updates)
#pragma unroll
      for (int k = 0; k < 8; ++k) r[k] = fma(beta, old[k], alpha * v[k]);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) r[k] = alpha * v[k];
    }
    st8<TO, S>(p, r, kbeg, n, vec);
  }
  __device__ __forceinline__ void put(int b, int i, int j0, const S* v, int kbeg, int n, const Pre& pre,
                                      S* vo) const {
    blend(dst + (int64_t)b * sd + (int64_t)i * ld + j0, v, kbeg, n, pre);
#pragma unroll
    for (int k = 0; k < 8; ++k) vo[k] = v[k];
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const S* v, int n, const PreT& pre) const {
    blend(dst + (int64_t)b * sd + (int64_t)j * ld + i0, v, 0, n, pre);
  }
  __device__ __forceinline__ void finish(int) const {}
};

// EpiBlend over up to kBlendTab separately allocated outputs of one shape:
// matrix b of the launch blends into dst[b] (row pitch ld). The table
// travels in the kernel arguments, so it needs no device copy.
constexpr int kBlendTab = 64;
template <typename TO, typename A>
struct EpiBlendTab {
  typedef A S;
  TO* dst[kBlendTab];
  int64_t ld;
  A beta, alpha;
  bool vec;
  typedef Raw8<TO> Pre;
  typedef Raw8<TO> PreT;
  static constexpr bool kVoIsV = true;
  __device__ __forceinline__ EpiBlend<TO, A> one(int b) const { return EpiBlend<TO, A>{dst[b], ld, 0, beta, alpha, vec}; }
  __device__ __forceinline__ bool has_t() const { return false; }
  __device__ __forceinline__ void load(int b, int i, int j0, int kbeg, int n, Pre& p) const {
    one(b).load(0, i, j0, kbeg, n, p);
  }
  __device__ __forceinline__ void load_t(int b, int j, int i0, int n, PreT& p) const { one(b).load_t(0, j, i0, n, p); }
  __device__ __forceinline__ void put(int b, int i, int j0, const S* v, int kbeg, int n, const Pre& pre,
                                      S* vo) const {
    one(b).put(0, i, j0, v, kbeg, n, pre, vo);
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const S* v, int n, const PreT& pre) const {
    one(b).put_t(0, j, i0, v, n, pre);
  }
  __device__ __forceinline__ void finish(int) const {}
};

}  // namespace pto
