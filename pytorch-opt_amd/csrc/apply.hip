// Two-sided preconditioner application on gfx950.
//
// Replaces _NATIVE.precond_apply_two_sided
// (pytorch_opt/ops/__init__.py:81-84, csrc/pytorch_opt_ops.cpp:96-99),
// following pytorch_opt/ops/reference.py:117-121: out = (L_root·G)·R_root,
// associated left to right with the intermediate held in the op dtype.
// Both products run as MFMA "NT" launches over packed transposes of G and
// R_root (an O(n²) pass each, small next to the O(n³) products).
//
// The same code serves pto_two_sided_product, out = op(A)·X·op(B) with
// either factor transposed: SOAP's rotations into and out of the Shampoo
// eigenbasis, Q_Lᵀ·X·Q_R and Q_L·X·Q_Rᵀ (pytorch_opt/optim/soap.py:123-125),
// and its second-moment transport (C_L²)ᵀ·v·(C_R²) (:103-107).
#include <algorithm>

#include "aux_kernels.h"
#include "gemm_nt.h"

namespace pto {
namespace {

template <typename T>
size_t apply_ws_bytes_t(int64_t m, int64_t n) {
  int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  size_t bytes = 0;
  auto add = [&](size_t b) { bytes = round_up(bytes, 256) + b; };
  add(sizeof(T) * m * ldm);  // L_root padded
  add(sizeof(T) * n * ldm);  // Gᵀ
  add(sizeof(T) * m * ldn);  // L_root·G
  add(sizeof(T) * n * ldn);  // R_rootᵀ
  return bytes + 256;
}

// out = op(A)·X·op(B), op = identity or transpose, A [m,m], X [m,n],
// B [n,n], associated left to right with the intermediate in T.
// NT form: op(A)·X takes op(A)'s rows as P (A itself, or a packed Aᵀ) and
// Xᵀ's rows as Q; (op(A)·X)·op(B) takes op(B)ᵀ's rows as Q (a packed Bᵀ,
// or B itself).
template <typename T>
int two_sided_t(const T* Am, const T* X, const T* Bm, T* out, int64_t m, int64_t n, bool trans_a, bool trans_b,
                void* ws, size_t ws_bytes, hipStream_t stream, const char* name_left, const char* name_right) {
  typedef typename AccOf<T>::type A;
  PTO_REQUIRE(m <= INT32_MAX && n <= INT32_MAX, "two-sided product: shape too large");
  if (m == 0 || n == 0) return 0;
  const int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  Carver cv(ws, ws_bytes);
  T* Ap = cv.take<T>(m * ldm);  // op(A), padded
  T* XT = cv.take<T>(n * ldm);  // Xᵀ
  T* AX = cv.take<T>(m * ldn);  // op(A)·X
  T* Bq = cv.take<T>(n * ldn);  // op(B)ᵀ, padded
  PTO_REQUIRE(!cv.overflow, "two-sided product: workspace too small");

  const bool a_direct = !trans_a && (m % kPadK == 0) && (reinterpret_cast<uintptr_t>(Am) & 15) == 0;
  const bool b_direct = trans_b && (n % kPadK == 0) && (reinterpret_cast<uintptr_t>(Bm) & 15) == 0;
  if (!a_direct && launch_pack<T, T, A>(Am, m, m, m, 0, nullptr, trans_a ? nullptr : Ap, ldm, 0,
                                        trans_a ? Ap : nullptr, ldm, 0, false, 1, stream))
    return -1;
  if (launch_pack<T, T, A>(X, m, n, n, 0, nullptr, nullptr, 0, 0, XT, ldm, 0, false, 1, stream)) return -1;
  if (!b_direct && launch_pack<T, T, A>(Bm, n, n, n, 0, nullptr, trans_b ? Bq : nullptr, ldn, 0,
                                        trans_b ? nullptr : Bq, ldn, 0, false, 1, stream))
    return -1;
  if (launch_zero_cols<T>(AX, m, ldn, n, 0, 1, stream)) return -1;
  {
    const T* P = a_direct ? Am : Ap;
    GemmArgs g{P, a_direct ? m : ldm, 0, XT, ldm, 0, (int)m, (int)n, (int)ldm, 0, 0, nullptr};
    EpiStore<T, A> e{AX, ldn, 0, vec_ok<T>(AX, ldn, 0)};
    if (launch_gemm<T, false>(g, e, 1, stream, name_left)) return -1;
  }
  {
    const T* Q = b_direct ? Bm : Bq;
    GemmArgs g{AX, ldn, 0, Q, b_direct ? n : ldn, 0, (int)m, (int)n, (int)ldn, 0, 0, nullptr};
    EpiStore<T, A> e{out, n, 0, vec_ok<T>(out, n, 0)};
    if (launch_gemm<T, false>(g, e, 1, stream, name_right)) return -1;
  }
  return 0;
}

template <typename T>
int two_sided_dispatch(const void* Am, const void* X, const void* Bm, void* out, int64_t m, int64_t n, bool trans_a,
                       bool trans_b, void* ws, size_t ws_bytes, hipStream_t stream, const char* left,
                       const char* right) {
  return two_sided_t<T>(static_cast<const T*>(Am), static_cast<const T*>(X), static_cast<const T*>(Bm),
                        static_cast<T*>(out), m, n, trans_a, trans_b, ws, ws_bytes, stream, left, right);
}

int two_sided(const void* Am, const void* X, const void* Bm, void* out, int dtype, int64_t m, int64_t n, bool trans_a,
              bool trans_b, void* ws, size_t ws_bytes, hipStream_t stream, const char* what, const char* left,
              const char* right) {
  PTO_REQUIRE(m >= 0 && n >= 0, std::string(what) + ": negative extent");
  switch (dtype) {
    case kBF16:
      return two_sided_dispatch<bf16>(Am, X, Bm, out, m, n, trans_a, trans_b, ws, ws_bytes, stream, left, right);
    case kF32:
      return two_sided_dispatch<float>(Am, X, Bm, out, m, n, trans_a, trans_b, ws, ws_bytes, stream, left, right);
    case kF64:
      return two_sided_dispatch<double>(Am, X, Bm, out, m, n, trans_a, trans_b, ws, ws_bytes, stream, left, right);
    default:
      PTO_REQUIRE(false, std::string(what) + ": unsupported dtype code");
  }
}

}  // namespace
}  // namespace pto

extern "C" {

size_t pto_precond_apply_workspace_bytes(int dtype, int64_t m, int64_t n) {
  switch (dtype) {
    case pto::kBF16: return pto::apply_ws_bytes_t<pto::bf16>(m, n);
    case pto::kF32: return pto::apply_ws_bytes_t<float>(m, n);
    case pto::kF64: return pto::apply_ws_bytes_t<double>(m, n);
    default: return 0;
  }
}

int pto_precond_apply(const void* L_root, const void* G, const void* R_root, void* out, int dtype, int64_t m,
                      int64_t n, void* workspace, size_t ws_bytes, void* stream) {
  return pto::two_sided(L_root, G, R_root, out, dtype, m, n, false, false, workspace, ws_bytes,
                        static_cast<hipStream_t>(stream), "precond_apply_two_sided", "apply_left", "apply_right");
}

size_t pto_two_sided_product_workspace_bytes(int dtype, int64_t m, int64_t n) {
  return pto_precond_apply_workspace_bytes(dtype, m, n);
}

int pto_two_sided_product(const void* A, const void* X, const void* B, void* out, int dtype, int64_t m, int64_t n,
                          int trans_a, int trans_b, void* workspace, size_t ws_bytes, void* stream) {
  return pto::two_sided(A, X, B, out, dtype, m, n, trans_a != 0, trans_b != 0, workspace, ws_bytes,
                        static_cast<hipStream_t>(stream), "two_sided_product", "rotate_left", "rotate_right");
}

}  // extern "C"
