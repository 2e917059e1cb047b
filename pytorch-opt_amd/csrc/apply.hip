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
size_t apply_ws_bytes_t(int64_t m, int64_t n, int64_t batch = 1, bool shared_a = false, bool shared_b = false) {
  int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  size_t bytes = 0;
  auto add = [&](size_t b) { bytes = round_up(bytes, 256) + b; };
  add(sizeof(T) * m * ldm * (shared_a ? 1 : batch));  // op(A) padded
  add(sizeof(T) * n * ldm * batch);                   // Xᵀ
  add(sizeof(T) * m * ldn * batch);                   // op(A)·X
  add(sizeof(T) * n * ldn * (shared_b ? 1 : batch));  // op(B)ᵀ padded
  return bytes + 256;
}

// out[b] = op(A[b])·X[b]·op(B[b]) for b < batch, op = identity or
// transpose, A [m,m], X [m,n], B [n,n] at element strides sA, sX, sB (0:
// one matrix shared by the whole batch), out contiguous [batch][m][n];
// associated left to right with the intermediate in T. NT form: op(A)·X
// takes op(A)'s rows as P (A itself, or a packed Aᵀ) and Xᵀ's rows as Q;
// (op(A)·X)·op(B) takes op(B)ᵀ's rows as Q (a packed Bᵀ, or B itself).
// Each of the two products is one batched launch.
template <typename T>
int two_sided_t(const T* Am, const T* X, const T* Bm, T* out, int64_t batch, int64_t m, int64_t n, int64_t sA,
                int64_t sX, int64_t sB, bool trans_a, bool trans_b, void* ws, size_t ws_bytes, hipStream_t stream,
                const char* name_left, const char* name_right) {
  typedef typename AccOf<T>::type A;
  PTO_REQUIRE(m <= INT32_MAX && n <= INT32_MAX, "two-sided product: shape too large");
  PTO_REQUIRE(batch >= 0 && batch < 65536, "two-sided product: batch must be below 65536");
  PTO_REQUIRE(sA >= 0 && sX >= 0 && sB >= 0, "two-sided product: negative stride");
  if (m == 0 || n == 0 || batch == 0) return 0;
  const int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  const int nb = (int)batch, nA = sA ? nb : 1, nB = sB ? nb : 1;
  Carver cv(ws, ws_bytes);
  T* Ap = cv.take<T>(m * ldm * nA);  // op(A), padded
  T* XT = cv.take<T>(n * ldm * nb);  // Xᵀ
  T* AX = cv.take<T>(m * ldn * nb);  // op(A)·X
  T* Bq = cv.take<T>(n * ldn * nB);  // op(B)ᵀ, padded
  PTO_REQUIRE(!cv.overflow, "two-sided product: workspace too small");

  constexpr int64_t VEC = 16 / sizeof(T);
  const bool a_direct = !trans_a && (m % kPadK == 0) && sA % VEC == 0 && (reinterpret_cast<uintptr_t>(Am) & 15) == 0;
  const bool b_direct = trans_b && (n % kPadK == 0) && sB % VEC == 0 && (reinterpret_cast<uintptr_t>(Bm) & 15) == 0;
  if (!a_direct && launch_pack<T, T, A>(Am, m, m, m, sA, nullptr, trans_a ? nullptr : Ap, ldm, m * ldm,
                                        trans_a ? Ap : nullptr, ldm, m * ldm, false, nA, stream))
    return -1;
  if (launch_pack<T, T, A>(X, m, n, n, sX, nullptr, nullptr, 0, 0, XT, ldm, n * ldm, false, nb, stream)) return -1;
  if (!b_direct && launch_pack<T, T, A>(Bm, n, n, n, sB, nullptr, trans_b ? Bq : nullptr, ldn, n * ldn,
                                        trans_b ? nullptr : Bq, ldn, n * ldn, false, nB, stream))
    return -1;
  if (launch_zero_cols<T>(AX, m, ldn, n, m * ldn, nb, stream)) return -1;
  {
    const T* P = a_direct ? Am : Ap;
    const int64_t sP = a_direct ? sA : (nA > 1 ? m * ldm : 0);
    GemmArgs g{P, a_direct ? m : ldm, sP, XT, ldm, n * ldm, (int)m, (int)n, (int)ldm, 0, 0, nullptr};
    EpiStore<T, A> e{AX, ldn, m * ldn, vec_ok<T>(AX, ldn, m * ldn)};
    if (launch_gemm<T, false>(g, e, nb, stream, name_left)) return -1;
  }
  {
    const T* Q = b_direct ? Bm : Bq;
    const int64_t sQ = b_direct ? sB : (nB > 1 ? n * ldn : 0);
    GemmArgs g{AX, ldn, m * ldn, Q, b_direct ? n : ldn, sQ, (int)m, (int)n, (int)ldn, 0, 0, nullptr};
    EpiStore<T, A> e{out, n, m * n, vec_ok<T>(out, n, m * n)};
    if (launch_gemm<T, false>(g, e, nb, stream, name_right)) return -1;
  }
  return 0;
}

template <typename T>
int two_sided_dispatch(const void* Am, const void* X, const void* Bm, void* out, int64_t batch, int64_t m, int64_t n,
                       int64_t sA, int64_t sX, int64_t sB, bool trans_a, bool trans_b, void* ws, size_t ws_bytes,
                       hipStream_t stream, const char* left, const char* right) {
  return two_sided_t<T>(static_cast<const T*>(Am), static_cast<const T*>(X), static_cast<const T*>(Bm),
                        static_cast<T*>(out), batch, m, n, sA, sX, sB, trans_a, trans_b, ws, ws_bytes, stream, left,
                        right);
}

int two_sided(const void* Am, const void* X, const void* Bm, void* out, int dtype, int64_t batch, int64_t m, int64_t n,
              int64_t sA, int64_t sX, int64_t sB, bool trans_a, bool trans_b, void* ws, size_t ws_bytes,
              hipStream_t stream, const char* what, const char* left, const char* right) {
  PTO_REQUIRE(m >= 0 && n >= 0 && batch >= 0, std::string(what) + ": negative extent");
  PTO_REQUIRE(batch * m * n == 0 || (Am && X && Bm && out && ws), std::string(what) + ": null operand or workspace");
  switch (dtype) {
    case kBF16:
      return two_sided_dispatch<bf16>(Am, X, Bm, out, batch, m, n, sA, sX, sB, trans_a, trans_b, ws, ws_bytes, stream,
                                      left, right);
    case kF32:
      return two_sided_dispatch<float>(Am, X, Bm, out, batch, m, n, sA, sX, sB, trans_a, trans_b, ws, ws_bytes, stream,
                                       left, right);
    case kF64:
      return two_sided_dispatch<double>(Am, X, Bm, out, batch, m, n, sA, sX, sB, trans_a, trans_b, ws, ws_bytes,
                                        stream, left, right);
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
  return pto::two_sided(L_root, G, R_root, out, dtype, 1, m, n, 0, 0, 0, false, false, workspace, ws_bytes,
                        static_cast<hipStream_t>(stream), "precond_apply_two_sided", "apply_left", "apply_right");
}

size_t pto_two_sided_product_workspace_bytes(int dtype, int64_t m, int64_t n) {
  return pto_precond_apply_workspace_bytes(dtype, m, n);
}

int pto_two_sided_product(const void* A, const void* X, const void* B, void* out, int dtype, int64_t m, int64_t n,
                          int trans_a, int trans_b, void* workspace, size_t ws_bytes, void* stream) {
  return pto::two_sided(A, X, B, out, dtype, 1, m, n, 0, 0, 0, trans_a != 0, trans_b != 0, workspace, ws_bytes,
                        static_cast<hipStream_t>(stream), "two_sided_product", "rotate_left", "rotate_right");
}

size_t pto_two_sided_product_batched_workspace_bytes(int dtype, int64_t batch, int64_t m, int64_t n, int shared_a,
                                                     int shared_b) {
  switch (dtype) {
    case pto::kBF16: return pto::apply_ws_bytes_t<pto::bf16>(m, n, batch, shared_a != 0, shared_b != 0);
    case pto::kF32: return pto::apply_ws_bytes_t<float>(m, n, batch, shared_a != 0, shared_b != 0);
    case pto::kF64: return pto::apply_ws_bytes_t<double>(m, n, batch, shared_a != 0, shared_b != 0);
    default: return 0;
  }
}

int pto_two_sided_product_batched(const void* A, const void* X, const void* B, void* out, int dtype, int64_t batch,
                                  int64_t m, int64_t n, int64_t stride_a, int64_t stride_x, int64_t stride_b,
                                  int trans_a, int trans_b, void* workspace, size_t ws_bytes, void* stream) {
  return pto::two_sided(A, X, B, out, dtype, batch, m, n, stride_a, stride_x, stride_b, trans_a != 0, trans_b != 0,
                        workspace, ws_bytes, static_cast<hipStream_t>(stream), "two_sided_product", "rotate_left",
                        "rotate_right");
}

}  // extern "C"
