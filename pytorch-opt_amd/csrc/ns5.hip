// Quintic Newton–Schulz orthogonalization on gfx950.
//
// Replaces _NATIVE.newton_schulz_orthogonalize
// (pytorch_opt/ops/__init__.py:67-71, csrc/pytorch_opt_ops.cpp:65-81) with
// the same semantics as pytorch_opt/ops/reference.py:71-97:
//   X = G (work precision); if rows > cols, X = Xᵀ;  X /= (‖X‖_F + eps);
//   repeat `steps` times:  A = X·Xᵀ;  B = b·A + c·A·A;  X = a·X + B·X;
//   undo the transpose; cast back.
//
// Per iteration three MFMA launches, each with a fused epilogue:
//   1. A = X·Xᵀ                    symmetric: upper tiles only, mirrored store
//   2. B' = a·I + b·A + c·(A·A)    symmetric: upper tiles only, mirrored store
//   3. X' = B'·X  (= a·X + B·X)    full
// Folding a·X into the product as a·I on the diagonal of B' spares the
// update a read of X; the extra rounding is that of one bf16 store of
// a + B_ii, the same size as the rounding of a·X itself in a bf16 chain.
// Layouts: the gram reads X's K-contiguous rows on both sides ("NT"). In
// bf16 the square and the update read their operands from [K][·] arrays
// through transposing LDS loads (A and B' are symmetric, so each is its own
// transpose; X' = B'·X reads X as stored), so X is kept in one layout; the
// first iteration reads a caller's 128-aligned bf16 G in place, with the
// 1/(‖G‖+eps) scale applied in the gram's and update's epilogues. In fp32
// and fp64 the update reads a stored Xᵀ, which its epilogue writes beside
// X'. bf16 inputs keep X, A, B in bf16 between launches with fp32
// accumulation (short side 128 or more; smaller ones run the fp32 chain,
// see ns5_bf16); fp32 and fp64 inputs stay in their own precision.
#include <algorithm>

#include "aux_kernels.h"
#include "gemm_nt.h"

namespace pto {

namespace {

// 1 / (sqrt(sum of partial squares) + eps), one block per matrix.
template <typename A>
__global__ void __launch_bounds__(256) ns_scale_kernel(const double* __restrict__ partial, double eps,
                                                       A* __restrict__ scale) {
  const double s = block_sum_partials(partial, blockIdx.x);
  if (threadIdx.x == 0) scale[blockIdx.x] = A(1) / (static_cast<A>(sqrt(s)) + static_cast<A>(eps));
}

// A = s²·v: the first gram reads the input itself when no pack is needed,
// so the 1/(‖G‖ + eps) scale lands here (scale == nullptr: A = v).
template <typename T, typename A>
struct EpiNsGram {
  typedef A S;
  T* dst;
  int64_t ld, sd;
  const A* scale;
  bool vec;
  typedef NoPre Pre;
  typedef NoPre PreT;
  static constexpr bool kVoIsV = true;
  __device__ __forceinline__ bool has_t() const { return false; }
  __device__ __forceinline__ void load(int, int, int, int, int, Pre&) const {}
  __device__ __forceinline__ void load_t(int, int, int, int, PreT&) const {}
  __device__ __forceinline__ void store(T* p, int b, const S* v, int kbeg, int n) const {
    if (scale == nullptr) {
      st8<T, S>(p, v, kbeg, n, vec);
      return;
    }
    const S s2 = scale[b] * scale[b];
    S w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = s2 * v[k];
    st8<T, S>(p, w, kbeg, n, vec);
  }
  __device__ __forceinline__ void put(int b, int i, int j0, const S* v, int kbeg, int n, const Pre&, S* vo) const {
    store(dst + (int64_t)b * sd + (int64_t)i * ld + j0, b, v, kbeg, n);
#pragma unroll
    for (int k = 0; k < 8; ++k) vo[k] = v[k];
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const S* v, int n, const PreT&) const {
    store(dst + (int64_t)b * sd + (int64_t)j * ld + i0, b, v, 0, n);
  }
  __device__ __forceinline__ void finish(int) const {}
};

// B' = a·I + b·A + c·v  (symmetric, so the mirror takes the same value)
template <typename T, typename A>
struct EpiNsSq {
  typedef A S;
  const T* Asrc;
  T* dst;
  int64_t ld, sd;
  A ac, bc, cc;
  bool vec;
  typedef Raw8<T> Pre;
  typedef NoPre PreT;
  static constexpr bool kVoIsV = false;  // the mirror stores B', not the raw product
  __device__ __forceinline__ bool has_t() const { return false; }
  __device__ __forceinline__ void load(int b, int i, int j0, int kbeg, int n, Pre& p) const {
    ld8_pre<T>(Asrc + (int64_t)b * sd + (int64_t)i * ld + j0, p, kbeg, n, vec);
  }
  __device__ __forceinline__ void load_t(int, int, int, int, PreT&) const {}
  __device__ __forceinline__ void put(int b, int i, int j0, const S* v, int kbeg, int n, const Pre& pre,
                                      S* vo) const {
    const int64_t o = (int64_t)b * sd + (int64_t)i * ld + j0;
    S a[8];
    ld8_use<T, S>(Asrc + o, pre, a, kbeg, n, vec);
    // explicit fused multiply-adds fix the rounding, so it cannot depend on
    // how the compiler contracts this expression in a given build
#pragma unroll
    for (int k = 0; k < 8; ++k) vo[k] = fma(cc, v[k], fma(bc, a[k], i == j0 + k ? ac : A(0)));
    st8<T, S>(dst + o, vo, kbeg, n, vec);
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const S* v, int n, const PreT&) const {
    st8<T, S>(dst + (int64_t)b * sd + (int64_t)j * ld + i0, v, 0, n, vec);
  }
  __device__ __forceinline__ void finish(int) const {}
};

// X' = s·v (s per matrix, scale == nullptr: s = 1; the first update of an
// unpacked input applies 1/(‖G‖ + eps) here), stored to dst (row-major)
// and/or dstT (transposed copy).
template <typename T, typename A>
struct EpiNsUpdate {
  typedef A S;
  T* dst;
  int64_t ld_d, s_d;
  T* dstT;
  int64_t ld_t, s_t;
  bool vec_d, vec_t;
  const A* scale;
  typedef NoPre Pre;
  typedef NoPre PreT;
  static constexpr bool kVoIsV = true;
  __device__ __forceinline__ bool has_t() const { return dstT != nullptr; }
  __device__ __forceinline__ void load(int, int, int, int, int, Pre&) const {}
  __device__ __forceinline__ void load_t(int, int, int, int, PreT&) const {}
  __device__ __forceinline__ void store(T* p, int b, const S* v, int kbeg, int n, bool vec) const {
    if (scale == nullptr) {
      st8<T, S>(p, v, kbeg, n, vec);
      return;
    }
    const S s = scale[b];
    S w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = s * v[k];
    st8<T, S>(p, w, kbeg, n, vec);
  }
  __device__ __forceinline__ void put(int b, int i, int j0, const S* v, int kbeg, int n, const Pre&, S* vo) const {
#pragma unroll
    for (int k = 0; k < 8; ++k) vo[k] = v[k];
    if (dst) store(dst + (int64_t)b * s_d + (int64_t)i * ld_d + j0, b, v, kbeg, n, vec_d);
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const S* v, int n, const PreT&) const {
    store(dstT + (int64_t)b * s_t + (int64_t)j * ld_t + i0, b, v, 0, n, vec_t);
  }
  __device__ __forceinline__ void finish(int) const {}
};

template <typename T>
struct NsLayout {
  int64_t m, n, ldm, ldn;
  bool transposed;
};

// bf16 updates read X itself as the [K][N] operand of X' = B'·X (QN
// layout), ping-ponging between two X buffers with ldm rows whose pad rows
// are zero. fp32 and fp64 keep one X and a ping-pong pair of stored Xᵀ.
template <typename T>
constexpr bool ns5_qn() {
  return sizeof(T) == 2;
}

template <typename T>
size_t ns5_ws_bytes_t(int64_t batch, int64_t rows, int64_t cols) {
  int64_t m = std::min(rows, cols), n = std::max(rows, cols);
  int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  size_t e = sizeof(T);
  size_t bytes = 0;
  auto add = [&](size_t b) { bytes = round_up(bytes, 256) + b; };
  typedef typename AccOf<T>::type A;
  add(sizeof(double) * kRedBlocks * batch);   // partial sums
  add(sizeof(A) * batch);                      // scales
  add(e * batch * ldm * ldm);                  // A (ldm rows: pad rows for the transposed read)
  add(e * batch * ldm * ldm);                  // B'
  if (ns5_qn<T>()) {
    add(e * batch * ldm * ldn);                // X ping
    add(e * batch * ldm * ldn);                // X pong
  } else {
    add(e * batch * m * ldn);                  // X
    add(e * batch * n * ldm);                  // Xᵀ ping
    add(e * batch * n * ldm);                  // Xᵀ pong
  }
  return bytes + 256;
}

template <typename T>
int ns5_t(const T* G, T* out, int64_t batch, int64_t rows, int64_t cols, int64_t steps, double a, double b, double c,
          double eps, void* ws, size_t ws_bytes, hipStream_t stream) {
  typedef typename AccOf<T>::type A;
  const bool transposed = rows > cols;
  const int64_t m = std::min(rows, cols), n = std::max(rows, cols);
  const int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  PTO_REQUIRE(m <= INT32_MAX && n <= INT32_MAX && batch <= 65535, "newton_schulz_orthogonalize: shape too large");
  if (batch == 0 || rows == 0 || cols == 0) return 0;

  constexpr bool QN = ns5_qn<T>();
  Carver cv(ws, ws_bytes);
  double* partial = cv.take<double>(kRedBlocks * batch);
  A* scale = cv.take<A>(batch);
  // A and B' hold ldm rows so that the bf16 update can read the symmetric
  // B' as its own transpose ([K][M], K = ldm, pad rows zero)
  const int64_t sAB = ldm * ldm;
  T* Ab = cv.take<T>(batch * sAB);
  T* Bb = cv.take<T>(batch * sAB);
  const int64_t sX = QN ? ldm * ldn : m * ldn;  // batch stride of X
  T* X[2];
  T* XT[2] = {nullptr, nullptr};
  X[0] = cv.take<T>(batch * sX);
  if (QN) {
    X[1] = cv.take<T>(batch * sX);
  } else {
    X[1] = X[0];
    XT[0] = cv.take<T>(batch * n * ldm);
    XT[1] = cv.take<T>(batch * n * ldm);
  }
  PTO_REQUIRE(!cv.overflow, "newton_schulz_orthogonalize: workspace too small");
  const int nb = (int)batch;
  const int64_t sG = rows * cols;

  // ‖X‖_F per matrix (deterministic two-stage sum), then 1/(‖X‖+eps).
  if (launch_sumsq<T>(G, rows, cols, cols, sG, nb, partial, stream)) return -1;
  hipLaunchKernelGGL(ns_scale_kernel<A>, dim3(nb), dim3(256), 0, stream, partial, eps, scale);
  PTO_LAUNCHED("ns_scale");

  // `out` may alias G exactly or not at all: every path below reads G only
  // in kernels that end before `out` is written, except the steps == 0
  // pack, which is tile-local (each element read before it is rewritten
  // in place) only when the two coincide.
  const uintptr_t g0 = reinterpret_cast<uintptr_t>(G), g1 = g0 + sizeof(T) * (uintptr_t)(batch * sG);
  const uintptr_t o0 = reinterpret_cast<uintptr_t>(out), o1 = o0 + sizeof(T) * (uintptr_t)(batch * sG);
  const bool aliased = g0 < o1 && o0 < g1;
  PTO_REQUIRE(!aliased || g0 == o0, "newton_schulz_orthogonalize: out partially overlaps G");

  if (steps == 0) {  // the normalised input, in the input's layout
    if (launch_pack<T, T, A>(G, rows, cols, cols, sG, scale, out, cols, sG, nullptr, 0, 0, false, nb, stream)) return -1;
    return 0;
  }

  // X0 = s·X (and, without the QN layout, X0ᵀ), pads zeroed. bf16 inputs
  // that need neither padding nor a transpose skip the copy: the first
  // gram and update read G itself and apply s² and s in their epilogues.
  // The MFMA operand loads are 16-byte accesses, so G must be 16-byte
  // aligned (a view at an odd element offset is packed instead), and the
  // first update reads G while its epilogue writes `out` (with one
  // iteration, the only update), so an aliased call is packed as well.
  const bool direct = QN && !transposed && m == ldm && n == ldn && (g0 & 15) == 0 && !aliased;
  if (QN && direct) {
    // no pads: X[1] is written in full by the first update
  } else if (QN) {
    if (!transposed) {
      if (launch_pack<T, T, A>(G, rows, cols, cols, sG, scale, X[0], ldn, sX, nullptr, 0, 0, false, nb, stream))
        return -1;
    } else {
      if (launch_pack<T, T, A>(G, rows, cols, cols, sG, scale, nullptr, 0, 0, X[0], ldn, sX, false, nb, stream))
        return -1;
    }
    // pad columns of the pong buffer, pad rows of both
    if (launch_zero_cols<T>(X[1], m, ldn, n, sX, nb, stream)) return -1;
    for (int i = 0; i < 2; ++i)
      if (launch_zero_cols<T>(X[i] + m * ldn, ldm - m, ldn, 0, sX, nb, stream)) return -1;
  } else {
    if (!transposed) {
      if (launch_pack<T, T, A>(G, rows, cols, cols, sG, scale, X[0], ldn, sX, XT[0], ldm, n * ldm, false, nb, stream))
        return -1;
    } else {
      if (launch_pack<T, T, A>(G, rows, cols, cols, sG, scale, XT[0], ldm, n * ldm, X[0], ldn, sX, false, nb, stream))
        return -1;
    }
    if (launch_zero_cols<T>(XT[1], n, ldm, m, n * ldm, nb, stream)) return -1;
  }
  if (launch_zero_cols<T>(Ab, m, ldm, m, sAB, nb, stream)) return -1;
  if (launch_zero_cols<T>(Bb, m, ldm, m, sAB, nb, stream)) return -1;
  if (launch_zero_cols<T>(Ab + m * ldm, ldm - m, ldm, 0, sAB, nb, stream)) return -1;  // pad rows
  if (launch_zero_cols<T>(Bb + m * ldm, ldm - m, ldm, 0, sAB, nb, stream)) return -1;

  int cur = 0;  // X[cur] (QN) or XT[cur] holds the current iterate
  for (int64_t t = 0; t < steps; ++t) {
    const bool last = t == steps - 1;
    // iteration 0 of an unpacked input reads G (stride sG == sX, no pads)
    const bool from_g = direct && t == 0;
    const T* Xc = from_g ? G : X[cur];
    const A* s0 = from_g ? scale : nullptr;
    // 1. A = X·Xᵀ
    {
      GemmArgs g{Xc, ldn, sX, Xc, ldn, sX, (int)m, (int)m, (int)ldn, 0, 0, nullptr};
      EpiNsGram<T, A> e{Ab, ldm, sAB, s0, vec_ok<T>(Ab, ldm, sAB)};
      if (launch_gemm<T, true>(g, e, nb, stream, "ns5_gram")) return -1;
    }
    // 2. B' = a·I + b·A + c·A·A
    {
      GemmArgs g{Ab, ldm, sAB, Ab, ldm, sAB, (int)m, (int)m, (int)ldm, 0, 0, nullptr};
      EpiNsSq<T, A> e{Ab, Bb, ldm, sAB, static_cast<A>(a), static_cast<A>(b), static_cast<A>(c),
                      vec_ok<T>(Ab, ldm, sAB) && vec_ok<T>(Bb, ldm, sAB)};
      // A is symmetric: both operands read as its own transpose (PT), on
      // any of the three symmetric tiles; without the transposing reads
      // (fp32, fp64) A's rows are its columns, so the NT launch reads A too
      if constexpr (QN) {
        if (launch_gemm_qn<EpiNsSq<T, A>, true, true>(g, e, nb, stream, "ns5_square")) return -1;
      } else {
        if (launch_gemm<T, true>(g, e, nb, stream, "ns5_square")) return -1;
      }
    }
    // 3. X' = B'·X   (QN: over X itself; else as B'·(Xᵀ)ᵀ over the stored
    //    transpose, X written in place since this product does not read it)
    {
      EpiNsUpdate<T, A> e{};
      e.scale = s0;
      if (!last && QN) {
        e.dst = X[cur ^ 1]; e.ld_d = ldn; e.s_d = sX;
        e.dstT = nullptr;
      } else if (!last) {
        e.dst = X[0]; e.ld_d = ldn; e.s_d = sX;
        e.dstT = XT[cur ^ 1]; e.ld_t = ldm; e.s_t = n * ldm;
      } else if (!transposed) {
        e.dst = out; e.ld_d = cols; e.s_d = sG;
        e.dstT = nullptr;
      } else {
        e.dst = nullptr;
        e.dstT = out; e.ld_t = cols; e.s_t = sG;
      }
      e.vec_d = e.dst && vec_ok<T>(e.dst, e.ld_d, e.s_d);
      e.vec_t = e.dstT && vec_ok<T>(e.dstT, e.ld_t, e.s_t);
      if constexpr (QN) {
        // B' is symmetric: read as its own transpose (PT), like X (QN)
        GemmArgs g{Bb, ldm, sAB, Xc, ldn, sX, (int)m, (int)n, (int)ldm, 0, 0, nullptr};
        if (launch_gemm_qn<EpiNsUpdate<T, A>, true>(g, e, nb, stream, "ns5_update")) return -1;
      } else {
        GemmArgs g{Bb, ldm, sAB, XT[cur], ldm, n * ldm, (int)m, (int)n, (int)ldm, 0, 0, nullptr};
        if (launch_gemm<T, false>(g, e, nb, stream, "ns5_update")) return -1;
      }
    }
    cur ^= 1;
  }
  return 0;
}

// bf16 inputs whose short side is below kNs5Bf16MinSide run in fp32 work
// precision, as the reference runs every bf16 input (they are small, so
// the fp32 chain costs little): G is widened to fp32, the fp32 chain runs,
// and the result is rounded to bf16 once. Keeping X, A and B' in bf16
// between launches costs few-row matrices the most accuracy (relative
// Frobenius error against the fp32 chain up to 0.057 at 3-4 rows, 0.026 at
// 32 and 0.019 at 48 on Gaussian inputs in a CPU emulation of the bf16
// chain, against <= 0.0115 from 96 rows up and ~0.01 at 4096).
constexpr int64_t kNs5Bf16MinSide = 128;

inline bool ns5_bf16_in_f32(int64_t rows, int64_t cols) { return std::min(rows, cols) < kNs5Bf16MinSide; }

size_t ns5_ws_bytes_bf16(int64_t batch, int64_t rows, int64_t cols) {
  if (!ns5_bf16_in_f32(rows, cols)) return ns5_ws_bytes_t<bf16>(batch, rows, cols);
  const size_t copy = round_up(sizeof(float) * (size_t)(batch * rows * cols), 256);
  return 2 * copy + ns5_ws_bytes_t<float>(batch, rows, cols) + 3 * 256;
}

int ns5_bf16(const bf16* G, bf16* out, int64_t batch, int64_t rows, int64_t cols, int64_t steps, double a, double b,
             double c, double eps, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!ns5_bf16_in_f32(rows, cols))
    return ns5_t<bf16>(G, out, batch, rows, cols, steps, a, b, c, eps, ws, ws_bytes, stream);
  PTO_REQUIRE(batch <= 65535, "newton_schulz_orthogonalize: shape too large");
  if (batch == 0 || rows == 0 || cols == 0) return 0;
  Carver cv(ws, ws_bytes);
  const int64_t sG = rows * cols;
  float* Gf = cv.take<float>(batch * sG);
  float* Of = cv.take<float>(batch * sG);
  const size_t rest = ns5_ws_bytes_t<float>(batch, rows, cols);
  char* wf = cv.take<char>((int64_t)rest);
  PTO_REQUIRE(!cv.overflow, "newton_schulz_orthogonalize: workspace too small");
  const int nb = (int)batch;
  // G is read in full before `out` (which may be G itself) is written
  if (launch_pack<bf16, float, float>(G, rows, cols, cols, sG, nullptr, Gf, cols, sG, nullptr, 0, 0, false, nb,
                                      stream))
    return -1;
  if (ns5_t<float>(Gf, Of, batch, rows, cols, steps, a, b, c, eps, wf, rest, stream)) return -1;
  return launch_pack<float, bf16, float>(Of, rows, cols, cols, sG, nullptr, out, cols, sG, nullptr, 0, 0, false, nb,
                                         stream);
}

}  // namespace
}  // namespace pto

extern "C" {

size_t pto_ns5_workspace_bytes(int dtype, int64_t batch, int64_t rows, int64_t cols) {
  switch (dtype) {
    case pto::kBF16: return pto::ns5_ws_bytes_bf16(batch, rows, cols);
    case pto::kF32: return pto::ns5_ws_bytes_t<float>(batch, rows, cols);
    case pto::kF64: return pto::ns5_ws_bytes_t<double>(batch, rows, cols);
    default: return 0;
  }
}

int pto_ns5(const void* G, void* out, int dtype, int64_t batch, int64_t rows, int64_t cols, int64_t steps, double a,
            double b, double c, double eps, void* workspace, size_t ws_bytes, void* stream) {
  PTO_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0 && steps >= 0,
              "newton_schulz_orthogonalize: negative extent or steps");
  PTO_REQUIRE(batch * rows * cols == 0 || (G && out && workspace),
              "newton_schulz_orthogonalize: null input, output or workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case pto::kBF16:
      return pto::ns5_bf16(static_cast<const pto::bf16*>(G), static_cast<pto::bf16*>(out), batch, rows, cols, steps, a,
                           b, c, eps, workspace, ws_bytes, s);
    case pto::kF32:
      return pto::ns5_t<float>(static_cast<const float*>(G), static_cast<float*>(out), batch, rows, cols, steps, a, b,
                               c, eps, workspace, ws_bytes, s);
    case pto::kF64:
      return pto::ns5_t<double>(static_cast<const double*>(G), static_cast<double*>(out), batch, rows, cols, steps, a,
                                b, c, eps, workspace, ws_bytes, s);
    default:
      PTO_REQUIRE(false, "newton_schulz_orthogonalize: unsupported dtype code");
  }
}

}  // extern "C"
