// MFMA "NT" product core for gfx950:  C[b](i,j) = sum_k P[b](i,k) * Q[b](j,k)
//
// Both operands are row-major with K contiguous, which is the layout every
// product on the pytorch_opt.ops path can be put into (X·Xᵀ, S·S for
// symmetric S, B·X via a stored Xᵀ, ...). That keeps each lane's MFMA
// fragment a contiguous 16-byte run in LDS for all three element types.
//
// Operand contract (checked by the host launchers):
//   * K is a multiple of the tile's BK and the pad columns of both operands
//     are zero (workspace buffers are padded to kPadK elements);
//   * rows beyond M (P) or N (Q) are never read (masked to zero);
//   * operand base pointers and leading dimensions are 16-byte aligned.
//
// Grid: blockIdx.x enumerates output tiles, blockIdx.y the batch. In UPPER
// mode only tiles with tile_row <= tile_col are launched; the value computed
// for (i, j), i <= j, is stored at (i, j) and at (j, i), so the result is an
// exactly symmetric matrix at half the MFMA work.
//
// Pipeline: two LDS stages; the global loads of tile k+1 are issued into
// registers before the MFMAs of tile k and written to the other LDS stage
// afterwards, so one barrier per K tile suffices.
#pragma once

#include "pto_common.h"

namespace pto {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef double f64x4_t __attribute__((ext_vector_type(4)));

// Per element type: which MFMA, its fragment shapes and output lane map.
//   MN  : output block is MN x MN
//   KPL : consecutive k values one lane feeds per instruction
//   G   : lane groups along k (64 / MN)
template <typename T>
struct Mfma;

template <>
struct Mfma<bf16> {  // v_mfma_f32_32x32x16_bf16
  typedef float acc_t;
  typedef f32x16_t cvec_t;
  static constexpr int MN = 32, KPL = 8, G = 2, NACC = 16;
  __device__ static __forceinline__ cvec_t mma(const uint4& a, const uint4& b, int, cvec_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane, int r) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }
  __device__ static __forceinline__ int col(int lane, int) { return lane & 31; }
};

template <>
struct Mfma<float> {  // v_mfma_f32_32x32x2_f32
  typedef float acc_t;
  typedef f32x16_t cvec_t;
  static constexpr int MN = 32, KPL = 1, G = 2, NACC = 16;
  __device__ static __forceinline__ cvec_t mma(const uint4& a, const uint4& b, int ii, cvec_t c) {
    float av = __uint_as_float(ii == 0 ? a.x : ii == 1 ? a.y : ii == 2 ? a.z : a.w);
    float bv = __uint_as_float(ii == 0 ? b.x : ii == 1 ? b.y : ii == 2 ? b.z : b.w);
    return __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane, int r) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }
  __device__ static __forceinline__ int col(int lane, int) { return lane & 31; }
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

// Tile configuration: BM x BN output tile, BK deep, WM x WN waves.
template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int NT = 64 * WM * WN;
};

struct GemmArgs {
  const void* P;
  int64_t ldp, sP;  // row pitch and batch stride, in elements
  const void* Q;
  int64_t ldq, sQ;
  int M, N, K;
  int tiles_m, tiles_n;
  const int* guard;  // if non-null and *guard != 0 the launch does nothing
};

// Map the linear tile id to (tile_row, tile_col).
template <bool UPPER>
__device__ __forceinline__ void decode_tile(int t, int tiles_m, int tiles_n, int& ti, int& tj) {
  if (UPPER) {
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

template <typename T, class Cfg, bool UPPER, class Epi>
__global__ void __launch_bounds__(Cfg::NT) gemm_nt_kernel(GemmArgs g, Epi epi) {
  typedef Mfma<T> MF;
  typedef typename MF::cvec_t cvec_t;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, NT = Cfg::NT;
  constexpr int VEC = 16 / sizeof(T);       // elements per 16-byte chunk
  constexpr int CPR = BK / VEC;             // chunks per tile row
  constexpr int PITCH = BK + VEC;           // LDS row pitch (16-byte pad)
  constexpr int WTM = BM / Cfg::WM, WTN = BN / Cfg::WN;
  constexpr int FM = WTM / MF::MN, FN = WTN / MF::MN;
  constexpr int LP = BM * CPR / NT, LQ = BN * CPR / NT;
  constexpr int KSPAN = BK / MF::G;         // k values per lane group per tile
  constexpr int NRG = KSPAN / VEC;          // 16-byte reads per fragment per tile
  constexpr int IPR = VEC / MF::KPL;        // instructions per 16-byte read
  static_assert(BK * sizeof(T) == 128, "tiles are 128 bytes deep");
  static_assert(BM * CPR % NT == 0 && BN * CPR % NT == 0, "load split");
  static_assert(WTM % MF::MN == 0 && WTN % MF::MN == 0, "wave tile");
  static_assert(KSPAN % VEC == 0, "fragment runs");

  if (g.guard != nullptr && *g.guard != 0) return;

  __shared__ __attribute__((aligned(16))) T lds[2][(BM + BN) * PITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int b = blockIdx.y;
  int ti, tj;
  decode_tile<UPPER>(blockIdx.x, g.tiles_m, g.tiles_n, ti, tj);
  const int row0 = ti * BM, col0 = tj * BN;

  const T* __restrict__ P = static_cast<const T*>(g.P) + (int64_t)b * g.sP;
  const T* __restrict__ Q = static_cast<const T*>(g.Q) + (int64_t)b * g.sQ;

  // Per-thread global source pointers (nullptr = masked row).
  const T* src_p[LP];
  const T* src_q[LQ];
#pragma unroll
  for (int q = 0; q < LP; ++q) {
    int c = tid + q * NT, r = c / CPR, kc = c % CPR;
    int gr = row0 + r;
    src_p[q] = gr < g.M ? P + (int64_t)gr * g.ldp + kc * VEC : nullptr;
  }
#pragma unroll
  for (int q = 0; q < LQ; ++q) {
    int c = tid + q * NT, r = c / CPR, kc = c % CPR;
    int gr = col0 + r;
    src_q[q] = gr < g.N ? Q + (int64_t)gr * g.ldq + kc * VEC : nullptr;
  }

  uint4 rp[LP], rq[LQ];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < LP; ++q)
      rp[q] = src_p[q] ? *reinterpret_cast<const uint4*>(src_p[q] + k0) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int q = 0; q < LQ; ++q)
      rq[q] = src_q[q] ? *reinterpret_cast<const uint4*>(src_q[q] + k0) : make_uint4(0, 0, 0, 0);
  };
  auto lstore = [&](int s) {
    T* L = lds[s];
#pragma unroll
    for (int q = 0; q < LP; ++q) {
      int c = tid + q * NT, r = c / CPR, kc = c % CPR;
      *reinterpret_cast<uint4*>(L + r * PITCH + kc * VEC) = rp[q];
    }
#pragma unroll
    for (int q = 0; q < LQ; ++q) {
      int c = tid + q * NT, r = c / CPR, kc = c % CPR;
      *reinterpret_cast<uint4*>(L + (BM + r) * PITCH + kc * VEC) = rq[q];
    }
  };

  cvec_t acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int r = 0; r < MF::NACC; ++r) acc[fm][fn][r] = 0;

  const int lr = lane % MF::MN, lg = lane / MF::MN;
  auto compute = [&](int s) {
    const T* L = lds[s];
    const T* Pw = L + (wm * WTM + lr) * PITCH + lg * KSPAN;
    const T* Qw = L + (BM + wn * WTN + lr) * PITCH + lg * KSPAN;
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      uint4 a[FM], bq[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        a[fm] = *reinterpret_cast<const uint4*>(Pw + fm * MF::MN * PITCH + rg * VEC);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        bq[fn] = *reinterpret_cast<const uint4*>(Qw + fn * MF::MN * PITCH + rg * VEC);
#pragma unroll
      for (int ii = 0; ii < IPR; ++ii)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = MF::mma(a[fm], bq[fn], ii, acc[fm][fn]);
    }
  };

  const int KT = g.K / BK;
  if (KT > 0) {
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < KT) gload((kt + 1) * BK);
      compute(cur);
      if (kt + 1 < KT) lstore(cur ^ 1);
      __syncthreads();
    }
  }

  // Epilogue, staged through LDS (free after the last barrier above) in
  // chunks of CH tile rows, so every global access of the functor is a run
  // of up to 8 consecutive elements of one output row:
  //   1. waves owning the chunk's rows write raw accumulators to LDS;
  //   2. direct pass: runs along output rows (i, j..j+7) -> epi.put, which
  //      hands back the value the transposed pass should see;
  //   3. transposed pass (mirror of a symmetric tile, or the functor's
  //      transposed copy): runs along (j, i..i+7) -> epi.put_t.
  // In symmetric (UPPER) products only i <= j is taken from the MFMA result;
  // on diagonal tiles the direct pass stores i <= j and the transposed pass
  // i > j, so the stored matrix is exactly symmetric.
  typedef typename Epi::S S;
  constexpr int SP = BN + 1;  // staging pitch (≡ 1 mod 64 banks for BN >= 64)
  constexpr int LDS_BYTES = 2 * (BM + BN) * PITCH * (int)sizeof(T);
  constexpr int CH_FIT = LDS_BYTES / (SP * (int)sizeof(S));
  constexpr int CH = CH_FIT >= BM ? BM : (CH_FIT / WTM) * WTM;
  static_assert(CH >= WTM && BM % CH == 0, "epilogue chunk");
  constexpr int CPRW = BN / 8;                 // 8-element runs per tile row
  constexpr int LGD = CPRW < 8 ? CPRW : 8;     // lanes sharing a row in a 64-item block
  constexpr int RPB = 64 / LGD;                // rows per 64-item block
  constexpr int CBLK = CPRW / LGD;             // 64-item blocks across a row
  S* stg = reinterpret_cast<S*>(&lds[0][0]);
  const bool diag = UPPER && ti == tj;
  const bool need_t = UPPER || epi.has_t();
  const int mrem = g.M - row0, nrem = g.N - col0;  // valid extent of this tile

  for (int c0 = 0; c0 < BM; c0 += CH) {
    if (c0 >= mrem) break;
    const int wr0 = wm * WTM;
    if (wr0 >= c0 && wr0 < c0 + CH) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int r = 0; r < MF::NACC; ++r) {
            const int li = wr0 - c0 + fm * MF::MN + MF::row(lane, r);
            const int lj = wn * WTN + fn * MF::MN + MF::col(lane, r);
            stg[li * SP + lj] = static_cast<S>(acc[fm][fn][r]);
          }
    }
    __syncthreads();
    const int rows = min(CH, mrem - c0);
    // direct pass: item -> (row lr, run lc); 8 lanes cover 64 consecutive
    // columns of one row, and the odd pitch keeps the LDS reads conflict-free
    const int dblocks = ((rows + RPB - 1) / RPB) * CBLK;
    for (int t = tid; t < dblocks * 64; t += NT) {
      const int blk = t >> 6, w = t & 63;
      const int lr = (blk / CBLK) * RPB + w / LGD;
      const int lc = ((blk % CBLK) * LGD + w % LGD) * 8;
      if (lr >= rows || lc >= nrem) continue;
      const int n = min(8, nrem - lc);
      const int kbeg = diag ? max(0, c0 + lr - lc) : 0;  // skip i > j on diagonal tiles
      if (kbeg >= n) continue;
      S v[8], vo[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = stg[lr * SP + lc + k];
      epi.put(b, row0 + c0 + lr, col0 + lc, v, kbeg, n, vo);
      if (need_t) {
#pragma unroll
        for (int k = 0; k < 8; ++k) stg[lr * SP + lc + k] = vo[k];
      }
    }
    if (need_t) {
      __syncthreads();
      // transposed pass: output row j = col0 + lc, columns i = row0+c0+lr..+7;
      // 8 lanes share lc and cover 64 consecutive i
      const int rgroups = (rows + 7) / 8;
      const int tblocks = ((rgroups + 7) / 8) * CPRW;
      for (int t = tid; t < tblocks * 64; t += NT) {
        const int blk = t >> 6, w = t & 63;
        const int lc = (blk % CPRW) * 8 + w / 8;
        const int lr = ((blk / CPRW) * 8 + w % 8) * 8;
        if (lc >= nrem || lr >= rows) continue;
        int n = min(8, rows - lr);
        if (diag) n = min(n, lc - (c0 + lr));  // strictly below the diagonal
        if (n <= 0) continue;
        S v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = k < n ? stg[(lr + k) * SP + lc] : S(0);
        epi.put_t(b, col0 + lc, row0 + c0 + lr, v, n);
      }
    }
    __syncthreads();
  }
  epi.finish(b);
}

// ------------------------------------------------------------- host launch

// Tile choices per element type. "big" for large problems, "small" when
// the big tiles would leave most of the 256 CUs idle.
template <typename T>
struct TileSet;
template <>
struct TileSet<bf16> {
  typedef Tile<256, 256, 64, 2, 4> big;
  typedef Tile<128, 128, 64, 2, 2> small;
};
template <>
struct TileSet<float> {
  typedef Tile<128, 128, 32, 2, 2> big;
  typedef Tile<64, 64, 32, 2, 2> small;
};
template <>
struct TileSet<double> {
  typedef Tile<64, 64, 16, 2, 2> big;
  typedef Tile<32, 32, 16, 2, 2> small;
};

template <typename T, class Cfg, bool UPPER, class Epi>
int launch_gemm_cfg(GemmArgs g, const Epi& epi, int batch, hipStream_t stream, const char* name) {
  g.tiles_m = (g.M + Cfg::BM - 1) / Cfg::BM;
  g.tiles_n = (g.N + Cfg::BN - 1) / Cfg::BN;
  int64_t tiles = UPPER ? (int64_t)g.tiles_m * (g.tiles_m + 1) / 2 : (int64_t)g.tiles_m * g.tiles_n;
  if (tiles == 0 || batch == 0) return 0;
  PTO_REQUIRE(tiles < (1ll << 31) && batch < 65536, std::string(name) + ": grid too large");
  ProfScope ps(name, stream);
  hipLaunchKernelGGL((gemm_nt_kernel<T, Cfg, UPPER, Epi>), dim3((unsigned)tiles, (unsigned)batch),
                     dim3(Cfg::NT), 0, stream, g, epi);
  PTO_LAUNCHED(name);
  return 0;
}

// Validate the operand contract and pick a tile size.
template <typename T, bool UPPER, class Epi>
int launch_gemm(const GemmArgs& g, const Epi& epi, int batch, hipStream_t stream, const char* name) {
  typedef typename TileSet<T>::big Big;
  typedef typename TileSet<T>::small Small;
  PTO_REQUIRE(g.M >= 0 && g.N >= 0 && g.K >= 0, std::string(name) + ": negative extent");
  PTO_REQUIRE(!UPPER || g.M == g.N, std::string(name) + ": symmetric product needs M == N");
  PTO_REQUIRE(g.K % Small::BK == 0 && g.K % Big::BK == 0, std::string(name) + ": K not padded");
  PTO_REQUIRE(g.ldp % (16 / sizeof(T)) == 0 && g.ldq % (16 / sizeof(T)) == 0 &&
                  (reinterpret_cast<uintptr_t>(g.P) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(g.Q) & 15) == 0,
              std::string(name) + ": operands not 16-byte aligned");
  int64_t tm = (g.M + Big::BM - 1) / Big::BM, tn = (g.N + Big::BN - 1) / Big::BN;
  int64_t big_tiles = (UPPER ? tm * (tm + 1) / 2 : tm * tn) * batch;
  if (big_tiles >= 512) return launch_gemm_cfg<T, Big, UPPER, Epi>(g, epi, batch, stream, name);
  return launch_gemm_cfg<T, Small, UPPER, Epi>(g, epi, batch, stream, name);
}

// ------------------------------------------------------------- epilogues
// Functor interface (S = staging/accumulation type):
//   put(b, i, j0, v[8], kbeg, n, vo[8])  output row i, columns j0+k for
//       k in [kbeg, n); vo receives what the transposed pass should see;
//   put_t(b, j, i0, v[8], n)             output row j, columns i0+k, k < n
//       (the mirror of a symmetric product, or a transposed copy);
//   has_t()                              whether put_t is needed outside
//       symmetric products;
//   finish(b)                            once per thread at the end.
// j0 and i0 are multiples of 8; `vec` (set by the host when the row pitch,
// batch stride and base allow) enables 16-byte accesses for full runs.

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
  __device__ __forceinline__ bool has_t() const { return false; }
  __device__ __forceinline__ void put(int b, int i, int j0, const S* v, int kbeg, int n, S* vo) const {
    st8<TO, S>(dst + (int64_t)b * sd + (int64_t)i * ld + j0, v, kbeg, n, vec);
#pragma unroll
    for (int k = 0; k < 8; ++k) vo[k] = v[k];
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const S* v, int n) const {
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
  __device__ __forceinline__ bool has_t() const { return false; }
  __device__ __forceinline__ void blend(TO* p, const S* v, int kbeg, int n) const {
    S r[8];
    if (beta != A(0)) {
      S old[8];
      ld8<TO, S>(p, old, kbeg, n, vec);
#pragma unroll
      for (int k = 0; k < 8; ++k) r[k] = beta * old[k] + alpha * v[k];
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) r[k] = alpha * v[k];
    }
    st8<TO, S>(p, r, kbeg, n, vec);
  }
  __device__ __forceinline__ void put(int b, int i, int j0, const S* v, int kbeg, int n, S* vo) const {
    blend(dst + (int64_t)b * sd + (int64_t)i * ld + j0, v, kbeg, n);
#pragma unroll
    for (int k = 0; k < 8; ++k) vo[k] = v[k];
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const S* v, int n) const {
    blend(dst + (int64_t)b * sd + (int64_t)j * ld + i0, v, 0, n);
  }
  __device__ __forceinline__ void finish(int) const {}
};

}  // namespace pto
