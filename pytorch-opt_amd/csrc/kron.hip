// Kronecker-factor statistics on gfx950.
//
// pto_kron_factor_update replaces _NATIVE.kron_factor_update_
// (pytorch_opt/ops/__init__.py:74-78, csrc/pytorch_opt_ops.cpp:83-94),
// following pytorch_opt/ops/reference.py:100-114:
//     L <- beta·L + (1-beta)·G·Gᵀ,   R <- beta·R + (1-beta)·Gᵀ·G
// (beta == 1 is the plain sum L += G·Gᵀ, R += Gᵀ·G), in place.
//
// pto_gram_update is the additive boundary for the K-FAC activation and
// gradient factors (pytorch_opt/curvature/kron.py:105-113 and the
// clone/EMA/running-mean step at :95-103):
//     F <- beta·F + alpha·X̃ᵀ·X̃,   X̃ = [X, 1] when append_ones is set,
// with beta == 0 meaning "overwrite".
//
// Each factor is one symmetric MFMA launch: only upper tiles are computed,
// the blend with the old factor is fused into the epilogue, and both
// (i, j) and (j, i) are written, so each factor is read and written once.
#include <algorithm>

#include "aux_kernels.h"
#include "gemm_nt.h"

namespace pto {
namespace {

template <typename T>
size_t kron_ws_bytes_t(int64_t m, int64_t n) {
  int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  size_t bytes = 0;
  auto add = [&](size_t b) { bytes = round_up(bytes, 256) + b; };
  add(sizeof(T) * m * ldn);  // G padded (only when n is not a pad multiple)
  add(sizeof(T) * n * ldm);  // Gᵀ
  return bytes + 256;
}

template <typename T>
int kron_t(T* L, T* R, const T* G, int64_t m, int64_t n, double beta2, void* ws, size_t ws_bytes,
           hipStream_t stream) {
  typedef typename AccOf<T>::type A;
  PTO_REQUIRE(m <= INT32_MAX && n <= INT32_MAX, "kron_factor_update_: shape too large");
  if (m == 0 || n == 0) return 0;
  const int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  Carver cv(ws, ws_bytes);
  T* Gp = cv.take<T>(m * ldn);
  T* GT = cv.take<T>(n * ldm);
  PTO_REQUIRE(!cv.overflow, "kron_factor_update_: workspace too small");

  const bool direct = (n % kPadK == 0) && (reinterpret_cast<uintptr_t>(G) & 15) == 0;
  const T* Grows = direct ? G : Gp;
  const int64_t ldg = direct ? n : ldn;
  if (launch_pack<T, T, A>(G, m, n, n, m * n, nullptr, direct ? nullptr : Gp, ldn, m * ldn, GT, ldm, n * ldm, false, 1,
                           stream))
    return -1;

  const A beta = beta2 == 1.0 ? A(1) : static_cast<A>(beta2);
  const A alpha = beta2 == 1.0 ? A(1) : static_cast<A>(1.0 - beta2);
  {
    GemmArgs g{Grows, ldg, 0, Grows, ldg, 0, (int)m, (int)m, (int)ldn, 0, 0, nullptr};
    EpiBlend<T, A> e{L, m, 0, beta, alpha, vec_ok<T>(L, m, 0)};
    if (launch_gemm<T, true>(g, e, 1, stream, "kron_left")) return -1;
  }
  {
    GemmArgs g{GT, ldm, 0, GT, ldm, 0, (int)n, (int)n, (int)ldm, 0, 0, nullptr};
    EpiBlend<T, A> e{R, n, 0, beta, alpha, vec_ok<T>(R, n, 0)};
    if (launch_gemm<T, true>(g, e, 1, stream, "kron_right")) return -1;
  }
  return 0;
}

// Batched form for the optimizers, which update many same-shape factors per
// step: G is one stacked tensor [batch][m][n] (the caller stacks the
// gradients), L[b] and R[b] are separate tensors reached through a pointer
// table. Each side is one launch over the whole batch; every fp32/fp64 tile
// sums a position's products in the same order, so each factor gets exactly
// the bits a single-matrix call gives.
template <typename T>
size_t kron_batched_ws_bytes_t(int64_t batch, int64_t m, int64_t n) {
  int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  size_t bytes = 0;
  auto add = [&](size_t b) { bytes = round_up(bytes, 256) + b; };
  add(sizeof(T) * batch * m * ldn);  // G padded (only when n is not a pad multiple)
  add(sizeof(T) * batch * n * ldm);  // Gᵀ
  return bytes + 256;
}

template <typename T>
int kron_batched_t(T* const* L, T* const* R, const T* G, int64_t batch, int64_t m, int64_t n, double beta2, void* ws,
                   size_t ws_bytes, hipStream_t stream) {
  typedef typename AccOf<T>::type A;
  PTO_REQUIRE(m <= INT32_MAX && n <= INT32_MAX, "kron_factor_update_batched_: shape too large");
  PTO_REQUIRE(batch >= 0 && batch <= kBlendTab, "kron_factor_update_batched_: at most 64 matrices per call");
  if (batch == 0 || m == 0 || n == 0) return 0;
  for (int64_t b = 0; b < batch; ++b) {
    PTO_REQUIRE(L[b] && R[b], "kron_factor_update_batched_: null factor");
    for (int64_t c = 0; c < batch; ++c)
      PTO_REQUIRE(L[b] != R[c] && (c == b || (L[b] != L[c] && R[b] != R[c])),
                  "kron_factor_update_batched_: factors must be distinct tensors");
  }
  const int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  Carver cv(ws, ws_bytes);
  T* Gp = cv.take<T>(batch * m * ldn);
  T* GT = cv.take<T>(batch * n * ldm);
  PTO_REQUIRE(!cv.overflow, "kron_factor_update_batched_: workspace too small");

  const bool direct = (n % kPadK == 0) && (reinterpret_cast<uintptr_t>(G) & 15) == 0;
  const T* Grows = direct ? G : Gp;
  const int64_t ldg = direct ? n : ldn, sg = direct ? m * n : m * ldn;
  if (launch_pack<T, T, A>(G, m, n, n, m * n, nullptr, direct ? nullptr : Gp, ldn, m * ldn, GT, ldm, n * ldm, false,
                           (int)batch, stream))
    return -1;

  const A beta = beta2 == 1.0 ? A(1) : static_cast<A>(beta2);
  const A alpha = beta2 == 1.0 ? A(1) : static_cast<A>(1.0 - beta2);
  auto table = [&](T* const* F, int64_t d) {
    EpiBlendTab<T, A> e{};
    e.ld = d;
    e.beta = beta;
    e.alpha = alpha;
    e.vec = true;
    for (int64_t b = 0; b < batch; ++b) {
      e.dst[b] = F[b];
      e.vec = e.vec && vec_ok<T>(F[b], d, 0);
    }
    return e;
  };
  {
    GemmArgs g{Grows, ldg, sg, Grows, ldg, sg, (int)m, (int)m, (int)ldn, 0, 0, nullptr};
    if (launch_gemm<T, true>(g, table(L, m), (int)batch, stream, "kron_left")) return -1;
  }
  {
    GemmArgs g{GT, ldm, n * ldm, GT, ldm, n * ldm, (int)n, (int)n, (int)ldm, 0, 0, nullptr};
    if (launch_gemm<T, true>(g, table(R, n), (int)batch, stream, "kron_right")) return -1;
  }
  return 0;
}

// bf16 X without the ones column is already the [K][M] operand of the
// transposing-read layout (K = tokens, M = features), for both sides of
// X̃ᵀX̃: it is read in place, with no Xᵀ pass and no workspace, when the
// token count needs no pad rows, the rows are whole 16-byte chunks and the
// tile model picks the 192² or 128² tile (the 256² tile spills with the
// fp32 blend epilogue on this layout). Returns that tile (pick_tile's code)
// or -1 for the packed path. X's 16-byte alignment is the caller's part of
// the contract (checked at launch).
template <typename TX>
int gram_direct_tile(int64_t rows, int64_t d, int append_ones) {
  if (sizeof(TX) != 2 || append_ones || rows % kPadK != 0 || d % 8 != 0 || d == 0) return -1;
  const int pick = pick_tile<TX, true>(d, d, 1);
  return pick == 0 || pick == 2 ? pick : -1;
}

template <typename TX>
size_t gram_ws_bytes_t(int64_t rows, int64_t d, int append_ones) {
  if (gram_direct_tile<TX>(rows, d, append_ones) >= 0) return 0;
  int64_t dd = d + (append_ones ? 1 : 0);
  return sizeof(TX) * dd * round_up(rows, kPadK) + 512;
}

// F (TF, [dd][dd]) <- beta·F + alpha·X̃ᵀX̃ with X (TX, [rows][d]).
template <typename TX, typename TF>
int gram_t(TF* F, const TX* X, int64_t rows, int64_t d, int append_ones, double beta, double alpha, void* ws,
           size_t ws_bytes, hipStream_t stream) {
  typedef typename AccOf<TX>::type A;
  const int64_t dd = d + (append_ones ? 1 : 0);
  PTO_REQUIRE(dd <= INT32_MAX && rows <= INT32_MAX, "gram_update_: shape too large");
  if (dd == 0) return 0;
  const int64_t ldr = round_up(rows, kPadK);
  if constexpr (sizeof(TX) == 2) {
    const int tile = gram_direct_tile<TX>(rows, d, append_ones);
    if (tile >= 0) {
      PTO_REQUIRE((reinterpret_cast<uintptr_t>(X) & 15) == 0,
                  "gram_update_: X must be 16-byte aligned (it is read in place)");
      GemmArgs g{X, d, 0, X, d, 0, (int)dd, (int)dd, (int)rows, 0, 0, nullptr};
      EpiBlend<TF, A> e{F, dd, 0, static_cast<A>(beta), static_cast<A>(alpha), vec_ok<TF>(F, dd, 0)};
      return launch_gemm_qn<EpiBlend<TF, A>, true, true>(g, e, 1, stream, "gram_update_direct", tile);
    }
  }
  Carver cv(ws, ws_bytes);
  TX* XT = cv.take<TX>(dd * ldr);
  PTO_REQUIRE(!cv.overflow, "gram_update_: workspace too small");
  // X̃ᵀ, [dd][ldr], with the ones row appended and the token pad zeroed.
  if (launch_pack<TX, TX, A>(X, rows, d, d, 0, nullptr, nullptr, 0, 0, XT, ldr, 0, append_ones != 0, 1, stream))
    return -1;
  GemmArgs g{XT, ldr, 0, XT, ldr, 0, (int)dd, (int)dd, (int)ldr, 0, 0, nullptr};
  EpiBlend<TF, A> e{F, dd, 0, static_cast<A>(beta), static_cast<A>(alpha), vec_ok<TF>(F, dd, 0)};
  return launch_gemm<TX, true>(g, e, 1, stream, "gram_update");
}

}  // namespace
}  // namespace pto

extern "C" {

size_t pto_kron_workspace_bytes(int dtype, int64_t m, int64_t n) {
  switch (dtype) {
    case pto::kBF16: return pto::kron_ws_bytes_t<pto::bf16>(m, n);
    case pto::kF32: return pto::kron_ws_bytes_t<float>(m, n);
    case pto::kF64: return pto::kron_ws_bytes_t<double>(m, n);
    default: return 0;
  }
}

int pto_kron_factor_update(void* L, void* R, const void* G, int dtype, int64_t m, int64_t n, double beta2,
                           void* workspace, size_t ws_bytes, void* stream) {
  PTO_REQUIRE(m >= 0 && n >= 0, "kron_factor_update_: negative extent");
  PTO_REQUIRE(m * n == 0 || (L && R && G && workspace), "kron_factor_update_: null factor, gradient or workspace");
  PTO_REQUIRE(L != G && R != G, "kron_factor_update_: G must not alias L or R");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case pto::kBF16:
      return pto::kron_t<pto::bf16>(static_cast<pto::bf16*>(L), static_cast<pto::bf16*>(R),
                                    static_cast<const pto::bf16*>(G), m, n, beta2, workspace, ws_bytes, s);
    case pto::kF32:
      return pto::kron_t<float>(static_cast<float*>(L), static_cast<float*>(R), static_cast<const float*>(G), m, n,
                                beta2, workspace, ws_bytes, s);
    case pto::kF64:
      return pto::kron_t<double>(static_cast<double*>(L), static_cast<double*>(R), static_cast<const double*>(G), m,
                                 n, beta2, workspace, ws_bytes, s);
    default:
      PTO_REQUIRE(false, "kron_factor_update_: unsupported dtype code");
  }
}

size_t pto_kron_batched_workspace_bytes(int dtype, int64_t batch, int64_t m, int64_t n) {
  switch (dtype) {
    case pto::kBF16: return pto::kron_batched_ws_bytes_t<pto::bf16>(batch, m, n);
    case pto::kF32: return pto::kron_batched_ws_bytes_t<float>(batch, m, n);
    case pto::kF64: return pto::kron_batched_ws_bytes_t<double>(batch, m, n);
    default: return 0;
  }
}

int pto_kron_factor_update_batched(void* const* L, void* const* R, const void* G, int dtype, int64_t batch, int64_t m,
                                   int64_t n, double beta2, void* workspace, size_t ws_bytes, void* stream) {
  PTO_REQUIRE(batch >= 0 && m >= 0 && n >= 0, "kron_factor_update_batched_: negative extent");
  PTO_REQUIRE(batch * m * n == 0 || (L && R && G && workspace),
              "kron_factor_update_batched_: null factor table, gradient stack or workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case pto::kBF16:
      return pto::kron_batched_t<pto::bf16>(reinterpret_cast<pto::bf16* const*>(L),
                                            reinterpret_cast<pto::bf16* const*>(R),
                                            static_cast<const pto::bf16*>(G), batch, m, n, beta2, workspace, ws_bytes, s);
    case pto::kF32:
      return pto::kron_batched_t<float>(reinterpret_cast<float* const*>(L), reinterpret_cast<float* const*>(R),
                                        static_cast<const float*>(G), batch, m, n, beta2, workspace, ws_bytes, s);
    case pto::kF64:
      return pto::kron_batched_t<double>(reinterpret_cast<double* const*>(L), reinterpret_cast<double* const*>(R),
                                         static_cast<const double*>(G), batch, m, n, beta2, workspace, ws_bytes, s);
    default:
      PTO_REQUIRE(false, "kron_factor_update_batched_: unsupported dtype code");
  }
}

size_t pto_gram_workspace_bytes(int x_dtype, int64_t rows, int64_t d, int append_ones) {
  switch (x_dtype) {
    case pto::kBF16: return pto::gram_ws_bytes_t<pto::bf16>(rows, d, append_ones);
    case pto::kF32: return pto::gram_ws_bytes_t<float>(rows, d, append_ones);
    case pto::kF64: return pto::gram_ws_bytes_t<double>(rows, d, append_ones);
    default: return 0;
  }
}

int pto_gram_update(void* F, int f_dtype, const void* X, int x_dtype, int64_t rows, int64_t d, int append_ones,
                    double beta, double alpha, void* workspace, size_t ws_bytes, void* stream) {
  PTO_REQUIRE(rows >= 0 && d >= 0, "gram_update_: negative extent");
  PTO_REQUIRE((d == 0 && !append_ones) || (F && (rows == 0 || X)), "gram_update_: null factor or input");
  PTO_REQUIRE(workspace || ws_bytes == 0, "gram_update_: null workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == pto::kBF16 && f_dtype == pto::kF32)
    return pto::gram_t<pto::bf16, float>(static_cast<float*>(F), static_cast<const pto::bf16*>(X), rows, d,
                                         append_ones, beta, alpha, workspace, ws_bytes, s);
  if (x_dtype == pto::kF32 && f_dtype == pto::kF32)
    return pto::gram_t<float, float>(static_cast<float*>(F), static_cast<const float*>(X), rows, d, append_ones, beta,
                                     alpha, workspace, ws_bytes, s);
  if (x_dtype == pto::kF64 && f_dtype == pto::kF64)
    return pto::gram_t<double, double>(static_cast<double*>(F), static_cast<const double*>(X), rows, d, append_ones,
                                       beta, alpha, workspace, ws_bytes, s);
  PTO_REQUIRE(false, "gram_update_: unsupported (x dtype, factor dtype) pair");
}

}  // extern "C"
