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

// ------------------------------------------------- Muon and Shampoo graft
//
// Muon's elementwise work around NS5 (pytorch_opt/optim/muon.py:79-83: the
// momentum buffer and the Nesterov input; :87-92: decay, update and the
// Σ update² diagnostic) and Shampoo's AdaGrad graft with its update
// (shampoo.py:133-151), each as one HBM pass (the graft as two, with its
// two norms in between). Every op is rounded as the torch op it replaces:
// `a.mul_(s)`, `a.add_(b)`, sqrt and divide as separately rounded steps
// (products and sums formed with contraction off, so the compiler cannot
// fuse them; sqrt and divide correctly rounded), `a.add(b, alpha=s)` as
// one fused multiply-add and `a.addcmul_(b, c)` as a rounded product b·c
// then that fused op (as torch's GPU kernels compute them); bf16 tensors
// round each result to bf16. The norms and
// Σ update² are fixed-order float64 sums (per-block partials, summed in
// block order).
template <typename C>
__device__ __forceinline__ C mul_rn(C a, C b) {
#pragma clang fp contract(off)
  return a * b;
}
template <typename C>
__device__ __forceinline__ C add_rn(C a, C b) {
#pragma clang fp contract(off)
  return a + b;
}
template <typename C>
__device__ __forceinline__ C div_rn(C a, C b) {
#pragma clang fp contract(off)
  return a / b;
}
__device__ __forceinline__ float sqrt_rn(float a) { return __builtin_sqrtf(a); }
__device__ __forceinline__ double sqrt_rn(double a) { return __builtin_sqrt(a); }
__device__ __forceinline__ float fma_rn(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_rn(double a, double b, double c) { return __builtin_fma(a, b, c); }

// Block sum of one double per thread into out[blockIdx.x] (fixed order).
__device__ __forceinline__ void block_partial(double acc, double* __restrict__ out) {
  __shared__ double red[kEwThreads];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kEwThreads / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = red[0];
  __syncthreads();
}

// Sum of count partials in fixed order, the same in every block and thread.
__device__ __forceinline__ double block_total(const double* __restrict__ partial, int count) {
  __shared__ double red[kEwThreads];
  double acc = 0.0;
  for (int i = threadIdx.x; i < count; i += kEwThreads) acc += partial[i];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kEwThreads / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  const double t = red[0];
  __syncthreads();
  return t;
}

// buf <- buf·mu + g (mul_ then add_); u <- g + mu·buf (Nesterov, one fused
// op) or u <- buf. u is a separate array (the caller's NS5 input).
template <typename T>
__device__ __forceinline__ void momentum_one(T& b, T g, T& u, typename Rounding<T>::C mu, bool nesterov) {
  typedef Rounding<T> R;
  typedef typename R::C C;
  const C gi = to_f(g);
  C bi = R::r(mul_rn(to_f(b), mu));
  bi = R::r(add_rn(bi, gi));
  b = static_cast<T>(bi);
  u = nesterov ? static_cast<T>(R::r(fma_rn(mu, bi, gi))) : static_cast<T>(bi);
}

template <typename T>
__global__ void __launch_bounds__(kEwThreads) muon_momentum_kernel(T* __restrict__ buf, const T* __restrict__ g,
                                                                   T* __restrict__ u, int64_t n, bool vec,
                                                                   typename Rounding<T>::C mu, bool nesterov) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int64_t stride = (int64_t)gridDim.x * kEwThreads;
  const int64_t tid = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  const int64_t nv = vec ? n / VEC : 0;
  for (int64_t c = tid; c < nv; c += stride) {
    uint4 bu = reinterpret_cast<const uint4*>(buf)[c];
    const uint4 gu = reinterpret_cast<const uint4*>(g)[c];
    uint4 uu;
    T* be = reinterpret_cast<T*>(&bu);
    const T* ge = reinterpret_cast<const T*>(&gu);
    T* ue = reinterpret_cast<T*>(&uu);
#pragma unroll
    for (int e = 0; e < VEC; ++e) momentum_one<T>(be[e], ge[e], ue[e], mu, nesterov);
    reinterpret_cast<uint4*>(buf)[c] = bu;
    reinterpret_cast<uint4*>(u)[c] = uu;
  }
  for (int64_t i = nv * VEC + tid; i < n; i += stride) momentum_one<T>(buf[i], g[i], u[i], mu, nesterov);
}

// p <- p·decay (when decay != 1) then p <- p + neg_lr·o (one fused op);
// Σ o² into per-block partials.
template <typename T>
__device__ __forceinline__ void update_one(T& p, T o, typename Rounding<T>::C decay, bool scale,
                                           typename Rounding<T>::C neg_lr, double& acc) {
  typedef Rounding<T> R;
  typedef typename R::C C;
  const C oi = to_f(o);
  C pi = to_f(p);
  if (scale) pi = R::r(mul_rn(pi, decay));
  p = static_cast<T>(R::r(fma_rn(neg_lr, oi, pi)));
  acc += static_cast<double>(oi) * static_cast<double>(oi);
}

template <typename T>
__global__ void __launch_bounds__(kEwThreads) muon_update_kernel(T* __restrict__ p, const T* __restrict__ o, int64_t n,
                                                                 bool vec, typename Rounding<T>::C decay, bool scale,
                                                                 typename Rounding<T>::C neg_lr,
                                                                 double* __restrict__ partial) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int64_t stride = (int64_t)gridDim.x * kEwThreads;
  const int64_t tid = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  const int64_t nv = vec ? n / VEC : 0;
  double acc = 0.0;
  for (int64_t c = tid; c < nv; c += stride) {
    uint4 pu = reinterpret_cast<const uint4*>(p)[c];
    const uint4 ou = reinterpret_cast<const uint4*>(o)[c];
    T* pe = reinterpret_cast<T*>(&pu);
    const T* oe = reinterpret_cast<const T*>(&ou);
#pragma unroll
    for (int e = 0; e < VEC; ++e) update_one<T>(pe[e], oe[e], decay, scale, neg_lr, acc);
    reinterpret_cast<uint4*>(p)[c] = pu;
  }
  for (int64_t i = nv * VEC + tid; i < n; i += stride) update_one<T>(p[i], o[i], decay, scale, neg_lr, acc);
  block_partial(acc, partial);
}

// Graft pass 1: acc <- acc + g·g (addcmul_: torch forms a + value·(b·c), the
// product b·c rounded, then one fused op, which for value 1 is a rounded
// sum); Σ (g / (sqrt(acc) + eps))² and Σ P² into per-block partials
// (partial[0..B), [B..2B)).
template <typename T>
__device__ __forceinline__ void graft_stats_one(T g, T& a, T P, typename Rounding<T>::C eps, double& s1,
                                                double& s2) {
  typedef Rounding<T> R;
  typedef typename R::C C;
  const C gi = to_f(g);
  const C ai = R::r(add_rn(to_f(a), mul_rn(gi, gi)));
  a = static_cast<T>(ai);
  C d = R::r(sqrt_rn(ai));
  d = R::r(add_rn(d, eps));
  const C q = R::r(div_rn(gi, d));
  const C pi = to_f(P);
  s1 += static_cast<double>(q) * static_cast<double>(q);
  s2 += static_cast<double>(pi) * static_cast<double>(pi);
}

template <typename T>
__global__ void __launch_bounds__(kEwThreads) graft_stats_kernel(const T* __restrict__ g, T* __restrict__ acc,
                                                                 const T* __restrict__ P, int64_t n, bool vec,
                                                                 typename Rounding<T>::C eps,
                                                                 double* __restrict__ partial) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int64_t stride = (int64_t)gridDim.x * kEwThreads;
  const int64_t tid = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  const int64_t nv = vec ? n / VEC : 0;
  double s1 = 0.0, s2 = 0.0;
  for (int64_t c = tid; c < nv; c += stride) {
    const uint4 gu = reinterpret_cast<const uint4*>(g)[c];
    uint4 au = reinterpret_cast<const uint4*>(acc)[c];
    const uint4 pu = reinterpret_cast<const uint4*>(P)[c];
    const T* ge = reinterpret_cast<const T*>(&gu);
    T* ae = reinterpret_cast<T*>(&au);
    const T* pe = reinterpret_cast<const T*>(&pu);
#pragma unroll
    for (int e = 0; e < VEC; ++e) graft_stats_one<T>(ge[e], ae[e], pe[e], eps, s1, s2);
    reinterpret_cast<uint4*>(acc)[c] = au;
  }
  for (int64_t i = nv * VEC + tid; i < n; i += stride) graft_stats_one<T>(g[i], acc[i], P[i], eps, s1, s2);
  block_partial(s1, partial);
  block_partial(s2, partial + gridDim.x);
}

// Graft pass 2: ratio = ‖g/(sqrt(acc)+eps)‖ / (‖P‖ + 1e-30) from pass 1's
// partials (each norm rounded to the dtype, as torch's norm returns it);
// upd = P·ratio; with momentum buf <- buf·mu + upd and upd = buf; p <- p·decay
// (when decay != 1); p <- p + neg_lr·upd. Block 0 stores the ratio.
template <typename T>
__global__ void __launch_bounds__(kEwThreads) graft_apply_kernel(T* __restrict__ p, const T* __restrict__ P,
                                                                 T* __restrict__ buf, int64_t n, bool vec,
                                                                 const double* __restrict__ partial, int blocks1,
                                                                 typename Rounding<T>::C mu,
                                                                 typename Rounding<T>::C decay, bool scale,
                                                                 typename Rounding<T>::C neg_lr,
                                                                 T* __restrict__ ratio_out) {
  typedef Rounding<T> R;
  typedef typename R::C C;
  constexpr int VEC = 16 / (int)sizeof(T);
  const C target = R::r(static_cast<C>(sqrt(block_total(partial, blocks1))));
  const C pnorm = R::r(static_cast<C>(sqrt(block_total(partial + blocks1, blocks1))));
  const C ratio = R::r(div_rn(target, R::r(add_rn(pnorm, static_cast<C>(1e-30)))));
  if (blockIdx.x == 0 && threadIdx.x == 0 && ratio_out != nullptr) *ratio_out = static_cast<T>(ratio);
  const bool mom = buf != nullptr;
  auto one = [&](T& pv, T Pv, T* bv) {
    C u = R::r(mul_rn(to_f(Pv), ratio));
    if (mom) {
      C b = R::r(mul_rn(to_f(*bv), mu));
      b = R::r(add_rn(b, u));
      *bv = static_cast<T>(b);
      u = b;
    }
    C pi = to_f(pv);
    if (scale) pi = R::r(mul_rn(pi, decay));
    pv = static_cast<T>(R::r(fma_rn(neg_lr, u, pi)));
  };
  const int64_t stride = (int64_t)gridDim.x * kEwThreads;
  const int64_t tid = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  const int64_t nv = vec ? n / VEC : 0;
  for (int64_t c = tid; c < nv; c += stride) {
    uint4 pu = reinterpret_cast<const uint4*>(p)[c];
    const uint4 Pu = reinterpret_cast<const uint4*>(P)[c];
    uint4 bu = mom ? reinterpret_cast<const uint4*>(buf)[c] : make_uint4(0, 0, 0, 0);
    T* pe = reinterpret_cast<T*>(&pu);
    const T* Pe = reinterpret_cast<const T*>(&Pu);
    T* be = reinterpret_cast<T*>(&bu);
#pragma unroll
    for (int e = 0; e < VEC; ++e) one(pe[e], Pe[e], be + e);
    reinterpret_cast<uint4*>(p)[c] = pu;
    if (mom) reinterpret_cast<uint4*>(buf)[c] = bu;
  }
  for (int64_t i = nv * VEC + tid; i < n; i += stride) {
    T dummy = T(0);
    one(p[i], P[i], mom ? buf + i : &dummy);
  }
}

inline bool aligned16(const void* q) { return q == nullptr || (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

template <typename T>
int grid_for(int64_t n, bool vec) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int64_t units = vec ? (n + VEC - 1) / VEC : n;
  return (int)std::max<int64_t>(1, std::min<int64_t>((units + kEwThreads - 1) / kEwThreads, kEwMaxBlocks));
}

template <typename T>
int muon_momentum_t(T* buf, const T* g, T* u, int64_t n, double mu, bool nesterov, hipStream_t stream) {
  PTO_REQUIRE(n >= 0 && buf && g && u, "muon_momentum: null tensor pointer or negative size");
  if (n == 0) return 0;
  const bool vec = aligned16(buf) && aligned16(g) && aligned16(u);
  hipLaunchKernelGGL(muon_momentum_kernel<T>, dim3(grid_for<T>(n, vec)), dim3(kEwThreads), 0, stream, buf, g, u, n,
                     vec, static_cast<typename Rounding<T>::C>(mu), nesterov);
  PTO_LAUNCHED("muon_momentum");
  return 0;
}

template <typename T>
int muon_update_t(T* p, const T* o, int64_t n, double decay, double neg_lr, double* update_sq, void* ws,
                  size_t ws_bytes, hipStream_t stream) {
  typedef typename Rounding<T>::C C;
  PTO_REQUIRE(n >= 0 && p && o && update_sq, "muon_update: null pointer or negative size");
  Carver cv(ws, ws_bytes);
  double* partial = cv.take<double>(kEwMaxBlocks);
  PTO_REQUIRE(!cv.overflow, "muon_update: workspace too small");
  const bool vec = aligned16(p) && aligned16(o);
  const int blocks = grid_for<T>(n, vec);
  hipLaunchKernelGGL(muon_update_kernel<T>, dim3(blocks), dim3(kEwThreads), 0, stream, p, o, n, vec,
                     static_cast<C>(decay), decay != 1.0, static_cast<C>(neg_lr), partial);
  PTO_LAUNCHED("muon_update");
  hipLaunchKernelGGL(sum_partials_kernel, dim3(1), dim3(kEwThreads), 0, stream, partial, blocks, update_sq);
  PTO_LAUNCHED("muon_update_sum");
  return 0;
}

template <typename T>
int graft_t(T* p, const T* g, T* acc, const T* P, T* buf, int64_t n, double diag_eps, double momentum, double decay,
            double neg_lr, T* ratio_out, void* ws, size_t ws_bytes, hipStream_t stream) {
  typedef typename Rounding<T>::C C;
  PTO_REQUIRE(n >= 0 && p && g && acc && P, "shampoo_graft: null tensor pointer or negative size");
  PTO_REQUIRE((buf != nullptr) == (momentum != 0.0), "shampoo_graft: momentum buffer iff momentum != 0");
  Carver cv(ws, ws_bytes);
  double* partial = cv.take<double>(2 * kEwMaxBlocks);
  PTO_REQUIRE(!cv.overflow, "shampoo_graft: workspace too small");
  const bool vec = aligned16(p) && aligned16(g) && aligned16(acc) && aligned16(P) && aligned16(buf);
  const int blocks = grid_for<T>(n, vec);
  hipLaunchKernelGGL(graft_stats_kernel<T>, dim3(blocks), dim3(kEwThreads), 0, stream, g, acc, P, n, vec,
                     static_cast<C>(diag_eps), partial);
  PTO_LAUNCHED("graft_stats");
  hipLaunchKernelGGL(graft_apply_kernel<T>, dim3(blocks), dim3(kEwThreads), 0, stream, p, P, buf, n, vec, partial,
                     blocks, static_cast<C>(momentum), static_cast<C>(decay), decay != 1.0, static_cast<C>(neg_lr),
                     ratio_out);
  PTO_LAUNCHED("graft_apply");
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

size_t pto_muon_update_workspace_bytes(void) { return sizeof(double) * pto::kEwMaxBlocks + 256; }
size_t pto_shampoo_graft_workspace_bytes(void) { return sizeof(double) * 2 * pto::kEwMaxBlocks + 256; }

int pto_muon_momentum(void* buf, const void* g, void* u, int dtype, int64_t n, double momentum, int nesterov,
                      void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case pto::kF32:
      return pto::muon_momentum_t<float>(static_cast<float*>(buf), static_cast<const float*>(g),
                                         static_cast<float*>(u), n, momentum, nesterov != 0, s);
    case pto::kF64:
      return pto::muon_momentum_t<double>(static_cast<double*>(buf), static_cast<const double*>(g),
                                          static_cast<double*>(u), n, momentum, nesterov != 0, s);
    case pto::kBF16:
      return pto::muon_momentum_t<pto::bf16>(static_cast<pto::bf16*>(buf), static_cast<const pto::bf16*>(g),
                                             static_cast<pto::bf16*>(u), n, momentum, nesterov != 0, s);
    default:
      PTO_REQUIRE(false, "muon_momentum: unsupported dtype code");
  }
}

int pto_muon_update(void* p, const void* o, int dtype, int64_t n, double decay, double neg_lr, double* update_sq,
                    void* workspace, size_t ws_bytes, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case pto::kF32:
      return pto::muon_update_t<float>(static_cast<float*>(p), static_cast<const float*>(o), n, decay, neg_lr,
                                       update_sq, workspace, ws_bytes, s);
    case pto::kF64:
      return pto::muon_update_t<double>(static_cast<double*>(p), static_cast<const double*>(o), n, decay, neg_lr,
                                        update_sq, workspace, ws_bytes, s);
    case pto::kBF16:
      return pto::muon_update_t<pto::bf16>(static_cast<pto::bf16*>(p), static_cast<const pto::bf16*>(o), n, decay,
                                           neg_lr, update_sq, workspace, ws_bytes, s);
    default:
      PTO_REQUIRE(false, "muon_update: unsupported dtype code");
  }
}

int pto_shampoo_graft(void* p, const void* g, void* acc, const void* P, void* buf, int dtype, int64_t n,
                      double diag_eps, double momentum, double decay, double neg_lr, void* ratio_out, void* workspace,
                      size_t ws_bytes, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case pto::kF32:
      return pto::graft_t<float>(static_cast<float*>(p), static_cast<const float*>(g), static_cast<float*>(acc),
                                 static_cast<const float*>(P), static_cast<float*>(buf), n, diag_eps, momentum, decay,
                                 neg_lr, static_cast<float*>(ratio_out), workspace, ws_bytes, s);
    case pto::kF64:
      return pto::graft_t<double>(static_cast<double*>(p), static_cast<const double*>(g), static_cast<double*>(acc),
                                  static_cast<const double*>(P), static_cast<double*>(buf), n, diag_eps, momentum,
                                  decay, neg_lr, static_cast<double*>(ratio_out), workspace, ws_bytes, s);
    case pto::kBF16:
      return pto::graft_t<pto::bf16>(static_cast<pto::bf16*>(p), static_cast<const pto::bf16*>(g),
                                     static_cast<pto::bf16*>(acc), static_cast<const pto::bf16*>(P),
                                     static_cast<pto::bf16*>(buf), n, diag_eps, momentum, decay, neg_lr,
                                     static_cast<pto::bf16*>(ratio_out), workspace, ws_bytes, s);
    default:
      PTO_REQUIRE(false, "shampoo_graft: unsupported dtype code");
  }
}

}  // extern "C"
