// Two-sided preconditioner application on gfx950.
//
// Replaces _NATIVE.precond_apply_two_sided
// (pytorch_opt/ops/__init__.py:81-84, csrc/pytorch_opt_ops.cpp:96-99),
// following pytorch_opt/ops/reference.py:117-121: out = (L_root·G)·R_root,
// associated left to right with the intermediate held in the op dtype.
// Both products run as MFMA "NT" launches over packed transposes of G and
// R_root (an O(n²) pass each, small next to the O(n³) products).
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

template <typename T>
int apply_t(const T* Lr, const T* G, const T* Rr, T* out, int64_t m, int64_t n, void* ws, size_t ws_bytes,
            hipStream_t stream) {
  typedef typename AccOf<T>::type A;
  PTO_REQUIRE(m <= INT32_MAX && n <= INT32_MAX, "precond_apply_two_sided: shape too large");
  if (m == 0 || n == 0) return 0;
  const int64_t ldm = round_up(m, kPadK), ldn = round_up(n, kPadK);
  Carver cv(ws, ws_bytes);
  T* Lp = cv.take<T>(m * ldm);
  T* GT = cv.take<T>(n * ldm);
  T* LG = cv.take<T>(m * ldn);
  T* RT = cv.take<T>(n * ldn);
  PTO_REQUIRE(!cv.overflow, "precond_apply_two_sided: workspace too small");

  const bool l_direct = (m % kPadK == 0) && (reinterpret_cast<uintptr_t>(Lr) & 15) == 0;
  if (!l_direct && launch_pack<T, T, A>(Lr, m, m, m, 0, nullptr, Lp, ldm, 0, nullptr, 0, 0, false, 1, stream))
    return -1;
  if (launch_pack<T, T, A>(G, m, n, n, 0, nullptr, nullptr, 0, 0, GT, ldm, 0, false, 1, stream)) return -1;
  if (launch_pack<T, T, A>(Rr, n, n, n, 0, nullptr, nullptr, 0, 0, RT, ldn, 0, false, 1, stream)) return -1;
  if (launch_zero_cols<T>(LG, m, ldn, n, 0, 1, stream)) return -1;
  {
    const T* P = l_direct ? Lr : Lp;
    GemmArgs g{P, l_direct ? m : ldm, 0, GT, ldm, 0, (int)m, (int)n, (int)ldm, 0, 0, nullptr};
    EpiStore<T, A> e{LG, ldn, 0, vec_ok<T>(LG, ldn, 0)};
    if (launch_gemm<T, false>(g, e, 1, stream, "apply_left")) return -1;
  }
  {
    GemmArgs g{LG, ldn, 0, RT, ldn, 0, (int)m, (int)n, (int)ldn, 0, 0, nullptr};
    EpiStore<T, A> e{out, n, 0, vec_ok<T>(out, n, 0)};
    if (launch_gemm<T, false>(g, e, 1, stream, "apply_right")) return -1;
  }
  return 0;
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
  PTO_REQUIRE(m >= 0 && n >= 0, "precond_apply_two_sided: negative extent");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case pto::kBF16:
      return pto::apply_t<pto::bf16>(static_cast<const pto::bf16*>(L_root), static_cast<const pto::bf16*>(G),
                                     static_cast<const pto::bf16*>(R_root), static_cast<pto::bf16*>(out), m, n,
                                     workspace, ws_bytes, s);
    case pto::kF32:
      return pto::apply_t<float>(static_cast<const float*>(L_root), static_cast<const float*>(G),
                                 static_cast<const float*>(R_root), static_cast<float*>(out), m, n, workspace,
                                 ws_bytes, s);
    case pto::kF64:
      return pto::apply_t<double>(static_cast<const double*>(L_root), static_cast<const double*>(G),
                                  static_cast<const double*>(R_root), static_cast<double*>(out), m, n, workspace,
                                  ws_bytes, s);
    default:
      PTO_REQUIRE(false, "precond_apply_two_sided: unsupported dtype code");
  }
}

}  // extern "C"
