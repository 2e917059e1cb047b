// Fused AdamW step on gfx950 — the shared fallback of the matrix optimizers.
//
// The reference runs this step as ten torch elementwise ops
// (pytorch_opt/optim/_common.py:56-79: lerp_, mul_, addcmul_, sqrt, a divide,
// add_, two divides, mul_, add_), about 24 array passes per element. Here one
// HBM-bound pass reads p, g, m, v and writes p, m, v: 7 arrays per element.
// Each op's result is rounded to the tensor's dtype in the reference's order,
// so bf16 state follows torch's op-by-op rounding; fp32 and fp64 run the same
// operations in their own precision. The scalars are formed as the reference
// forms them (in double, then cast to the op's compute type).
//
// Optionally Σ update² (the Muon diagnostic, pytorch_opt/optim/muon.py:97) as
// a fixed-order fp64 reduction: per-block partials, then one block sums them.
#include <algorithm>
#include <cmath>

#include "pto_common.h"

namespace pto {
namespace {

template <typename T>
struct Rounding;  // compute type C and the rounding of one op's result
template <>
struct Rounding<float> {
  typedef float C;
  __device__ static __forceinline__ float r(float x) { return x; }
};
template <>
struct Rounding<double> {
  typedef double C;
  __device__ static __forceinline__ double r(double x) { return x; }
};
template <>
struct Rounding<bf16> {
  typedef float C;
  __device__ static __forceinline__ float r(float x) { return static_cast<float>(static_cast<bf16>(x)); }
};

template <typename C>
struct AdamwScalars {
  C w1;      // lerp weight 1 - beta1
  C b2, w2;  // beta2, 1 - beta2
  C sbc2;    // (1 - beta2^t) ** 0.5
  C eps;
  C bc1;     // 1 - beta1^t
  C decay;   // 1 - lr * weight_decay
  C neg_lr;  // -lr
};

constexpr int kEwThreads = 256;
constexpr int kEwMaxBlocks = 1024;

template <typename T>
__device__ __forceinline__ void adamw_one(T& p, T g, T& m, T& v, const AdamwScalars<typename Rounding<T>::C>& k,
                                          double& acc) {
  typedef Rounding<T> R;
  typedef typename R::C C;
  const C gi = to_f(g);
  C mi = to_f(m), vi = to_f(v), pi = to_f(p);
  // torch's lerp: self + w·(end − self) for |w| < 0.5, else end − (end − self)·(1 − w)
  mi = R::r(k.w1 < C(0.5) && k.w1 > C(-0.5) ? mi + k.w1 * (gi - mi) : gi - (gi - mi) * (C(1) - k.w1));
  vi = R::r(vi * k.b2);
  vi = R::r(vi + k.w2 * gi * gi);
  C d = R::r(sqrt(vi));
  d = R::r(d / k.sbc2);
  d = R::r(d + k.eps);
  C u = R::r(mi / k.bc1);
  u = R::r(u / d);
  pi = R::r(pi * k.decay);
  pi = R::r(pi + k.neg_lr * u);
  m = static_cast<T>(mi);
  v = static_cast<T>(vi);
  p = static_cast<T>(pi);
  acc += static_cast<double>(u) * static_cast<double>(u);
}

// Elements are taken in 16-byte chunks when all four arrays are 16-byte
// aligned (vec), then one at a time for the tail.
template <typename T>
__global__ void __launch_bounds__(kEwThreads) adamw_kernel(T* __restrict__ p, const T* __restrict__ g,
                                                           T* __restrict__ m, T* __restrict__ v, int64_t n, bool vec,
                                                           AdamwScalars<typename Rounding<T>::C> k,
                                                           double* __restrict__ partial) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int64_t stride = (int64_t)gridDim.x * kEwThreads;
  const int64_t tid = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  double acc = 0.0;
  const int64_t nv = vec ? n / VEC : 0;
  for (int64_t c = tid; c < nv; c += stride) {
    uint4 pu = reinterpret_cast<const uint4*>(p)[c];
    const uint4 gu = reinterpret_cast<const uint4*>(g)[c];
    uint4 mu = reinterpret_cast<const uint4*>(m)[c];
    uint4 vu = reinterpret_cast<const uint4*>(v)[c];
    T* pe = reinterpret_cast<T*>(&pu);
    const T* ge = reinterpret_cast<const T*>(&gu);
    T* me = reinterpret_cast<T*>(&mu);
    T* ve = reinterpret_cast<T*>(&vu);
#pragma unroll
    for (int e = 0; e < VEC; ++e) adamw_one<T>(pe[e], ge[e], me[e], ve[e], k, acc);
    reinterpret_cast<uint4*>(p)[c] = pu;
    reinterpret_cast<uint4*>(m)[c] = mu;
    reinterpret_cast<uint4*>(v)[c] = vu;
  }
  for (int64_t i = nv * VEC + tid; i < n; i += stride) adamw_one<T>(p[i], g[i], m[i], v[i], k, acc);
  if (partial == nullptr) return;
  __shared__ double red[kEwThreads];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kEwThreads / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

__global__ void __launch_bounds__(kEwThreads) sum_partials_kernel(const double* __restrict__ partial, int count,
                                                                  double* __restrict__ out) {
  __shared__ double red[kEwThreads];
  double acc = 0.0;
  for (int i = threadIdx.x; i < count; i += kEwThreads) acc += partial[i];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kEwThreads / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) *out = red[0];
}

template <typename T>
int adamw_t(T* p, const T* g, T* m, T* v, int64_t n, double lr, double wd, double beta1, double beta2, double eps,
            int64_t step, double* update_sq, void* ws, size_t ws_bytes, hipStream_t stream) {
  typedef typename Rounding<T>::C C;
  PTO_REQUIRE(n >= 0 && step >= 1, "adamw_step: n must be >= 0 and step >= 1");
  PTO_REQUIRE(p && g && m && v, "adamw_step: null tensor pointer");
  const double bc1 = 1.0 - std::pow(beta1, (double)step);
  const double bc2 = 1.0 - std::pow(beta2, (double)step);
  AdamwScalars<C> k;
  k.w1 = static_cast<C>(1.0 - beta1);
  k.b2 = static_cast<C>(beta2);
  k.w2 = static_cast<C>(1.0 - beta2);
  k.sbc2 = static_cast<C>(std::pow(bc2, 0.5));
  k.eps = static_cast<C>(eps);
  k.bc1 = static_cast<C>(bc1);
  k.decay = static_cast<C>(1.0 - lr * wd);
  k.neg_lr = static_cast<C>(-lr);
  Carver cv(ws, ws_bytes);
  double* partial = update_sq ? cv.take<double>(kEwMaxBlocks) : nullptr;
  PTO_REQUIRE(!cv.overflow, "adamw_step: workspace too small");
  constexpr int VEC = 16 / (int)sizeof(T);
  auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool vec = al(p) && al(g) && al(m) && al(v);
  const int64_t units = vec ? (n + VEC - 1) / VEC : n;
  const int blocks = (int)std::max<int64_t>(1, std::min<int64_t>((units + kEwThreads - 1) / kEwThreads, kEwMaxBlocks));
  hipLaunchKernelGGL(adamw_kernel<T>, dim3(blocks), dim3(kEwThreads), 0, stream, p, g, m, v, n, vec, k, partial);
  PTO_LAUNCHED("adamw");
  if (update_sq) {
    hipLaunchKernelGGL(sum_partials_kernel, dim3(1), dim3(kEwThreads), 0, stream, partial, blocks, update_sq);
    PTO_LAUNCHED("adamw_sum");
  }
  return 0;
}

}  // namespace
}  // namespace pto

extern "C" {

size_t pto_adamw_workspace_bytes(void) { return sizeof(double) * pto::kEwMaxBlocks + 256; }

int pto_adamw_step(void* p, const void* g, void* m, void* v, int dtype, int64_t n, double lr, double weight_decay,
                   double beta1, double beta2, double eps, int64_t step, double* update_sq, void* workspace,
                   size_t ws_bytes, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case pto::kF32:
      return pto::adamw_t<float>(static_cast<float*>(p), static_cast<const float*>(g), static_cast<float*>(m),
                                 static_cast<float*>(v), n, lr, weight_decay, beta1, beta2, eps, step, update_sq,
                                 workspace, ws_bytes, s);
    case pto::kF64:
      return pto::adamw_t<double>(static_cast<double*>(p), static_cast<const double*>(g), static_cast<double*>(m),
                                  static_cast<double*>(v), n, lr, weight_decay, beta1, beta2, eps, step, update_sq,
                                  workspace, ws_bytes, s);
    case pto::kBF16:
      return pto::adamw_t<pto::bf16>(static_cast<pto::bf16*>(p), static_cast<const pto::bf16*>(g),
                                     static_cast<pto::bf16*>(m), static_cast<pto::bf16*>(v), n, lr, weight_decay,
                                     beta1, beta2, eps, step, update_sq, workspace, ws_bytes, s);
    default:
      PTO_REQUIRE(false, "adamw_step: unsupported dtype code");
  }
}

}  // extern "C"
