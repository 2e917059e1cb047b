// Inverse p-th matrix root by the coupled Newton iteration, on gfx950.
//
// Replaces the "newton" branch of _NATIVE.inverse_matrix_root
// (pytorch_opt/ops/__init__.py:58-64, csrc/pytorch_opt_ops.cpp:15-63),
// following pytorch_opt/ops/reference.py:17-40 and :43-68:
//   M  = sym(A in root precision) + damping·I
//   z  = (1 + p) / (2·max(‖M‖_F, tiny));  X = z^(1/p)·I;  Mk = z·M
//   loop up to max_iter:
//     Mi = (1 + 1/p)·I − Mk/p;  X = X·Mi;  Mk = Mi^p·Mk;  err = max|Mk − I|
//     stop keeping the previous X if err > 1.2·previous err; stop if err < tol
//   return sym(X) in the input dtype
// `err` is one maximum over the whole batch, as in the reference's batched
// call. pto_inverse_root_each instead runs every matrix of the batch by its
// own rule (own err, divergence guard, stop and returned iterate), exactly
// as one call per matrix would: the optimizers stack independent factors
// into one launch sequence that way.
//
// Symmetric formulation. In exact arithmetic X, Mk, Mi and every power of
// Mi are symmetric (all are polynomials in M). Here X·Mi, Mi^p and Mi^p·Mk
// are symmetric by construction: computed on upper tiles only and
// mirrored. That halves their MFMA work and is also what
// keeps fp32 stable: with full products (the reference's form) but
// symmetrised powers, Mk's antisymmetric rounding part is never corrected
// and X drifts; with Mk kept symmetric the iteration converges like the
// reference's (same err floor) with a smaller final residual.
//
// fp32 products accumulate in blocks (the GEMM core's COMP mode): at
// cond ~1e6 the returned iterate's residual is set by product rounding in
// the small-eigenvalue directions (a plain fp32 MFMA chain over K, which
// rounds like a sequential FMA loop, ends config-size runs at 2-10x the
// residual of the blocked sums).
//
// Device-side control: every kernel of an iteration checks a device flag
// and exits at once after the stop decision. The decision for iteration it
// is made by every wave of iteration it + 1's first launch (from the state
// after it - 1 and err of it; its first workgroup records the new state),
// so no launch sits between iterations; states alternate between two slots
// by iteration parity, so a launch never reads the slot it writes. The host
// enqueues iterations in chunks, ends each chunk with a one-block decide
// kernel, and reads the state once per chunk instead of once per
// iteration, one chunk behind the enqueued work (a chunk enqueued past the
// stop only runs skipping launches). X ping-pongs between two buffers, so the "previous iterate"
// is still intact when the divergence guard fires.
#include <algorithm>
#include <limits>
#include <vector>

#include "aux_kernels.h"
#include "gemm_nt.h"

namespace pto {
namespace {

// Stop state of one iteration run. Global mode: one state. Per-matrix
// mode: state 0 summarises (stopped once every matrix has stopped; iters =
// loop iterations run) and state 1 + b belongs to matrix b.
template <typename R>
struct RootState {
  int stopped;
  int result;  // index k of the iterate X_k to return
  int iters;   // loop iterations executed
  int pad;
  R prev_err;
};
static_assert(sizeof(RootState<float>) % sizeof(int) == 0 && sizeof(RootState<double>) % sizeof(int) == 0,
              "state stride in ints");

template <typename R>
struct Bits;
template <>
struct Bits<float> {
  typedef unsigned int U;
  __device__ static U of(float v) { return __float_as_uint(v); }
};
template <>
struct Bits<double> {
  typedef unsigned long long U;
  __device__ static U of(double v) { return (U)__double_as_longlong(v); }
};

// Separately rounded product and sum (never contracted into one fused
// operation), so the elementwise steps round as the reference's torch ops
// do: M = 0.5·(A + Aᵀ) then + damping·I; Mi = (1 − α)·I + α·Mk.
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ double mul_rn(double a, double b) { return __dmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ double add_rn(double a, double b) { return __dadd_rn(a, b); }

// M = sym(A) + damping·I in precision R, [n][ld] with zeroed pads.
template <typename TI, typename R>
__global__ void __launch_bounds__(256) root_sym_kernel(const TI* __restrict__ A, int64_t n, int64_t sA, R damping,
                                                       R* __restrict__ M, int64_t ld, int64_t sM) {
  __shared__ R t1[32][33], t2[32][33];
  const int b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const TI* Ab = A + (int64_t)b * sA;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int rr = ty; rr < 32; rr += 8) {
    int64_t r = r0 + rr, c = c0 + tx;
    t1[rr][tx] = (r < n && c < n) ? convert<R>(Ab[r * n + c]) : R(0);
    int64_t r2 = c0 + rr, c2 = r0 + tx;  // the mirrored tile A[c0.., r0..]
    t2[rr][tx] = (r2 < n && c2 < n) ? convert<R>(Ab[r2 * n + c2]) : R(0);
  }
  __syncthreads();
  R* Mb = M + (int64_t)b * sM;
  for (int rr = ty; rr < 32; rr += 8) {
    int64_t r = r0 + rr, c = c0 + tx;
    if (r >= n || c >= ld) continue;
    R v = R(0);
    if (c < n) {
      v = mul_rn(R(0.5), add_rn(t1[rr][tx], t2[tx][rr]));
      if (r == c && damping != R(0)) v = add_rn(v, damping);
    }
    Mb[r * ld + c] = v;
  }
}

// z = (1+p)/(2·max(‖M‖_F, tiny)), xs = z^(1/p), per matrix.
template <typename R>
__global__ void __launch_bounds__(256) root_scale_kernel(const double* __restrict__ partial, int p, R tiny,
                                                         R* __restrict__ z, R* __restrict__ xs) {
  const int b = blockIdx.x;
  const double s = block_sum_partials(partial, b);
  if (threadIdx.x != 0) return;
  R fro = static_cast<R>(sqrt(s));
  if (fro < tiny) fro = tiny;  // clamp_min; NaN compares false and passes through
  R zz = static_cast<R>(1.0 + p) / (R(2) * fro);
  z[b] = zz;
  xs[b] = pow(zz, static_cast<R>(1.0 / p));
}

// X0 = xs·I, Mk0 = z·M, Mi0 = c1·I + alpha·Mk0.
template <typename R>
__global__ void root_init_kernel(const R* __restrict__ M, int64_t n, int64_t ld, int64_t sb, const R* __restrict__ z,
                                 const R* __restrict__ xs, R c1, R alpha, R* __restrict__ X0, R* __restrict__ Mk,
                                 R* __restrict__ Mi) {
  const int b = blockIdx.y;
  const int64_t total = n * ld;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = e / ld, c = e - r * ld;
    int64_t o = (int64_t)b * sb + e;
    R x = R(0), mk = R(0), mi = R(0);
    if (c < n) {
      mk = M[o] * z[b];
      mi = mul_rn(alpha, mk);
      if (r == c) {
        mi = add_rn(c1, mi);
        x = xs[b];
      }
    }
    X0[o] = x;
    Mk[o] = mk;
    Mi[o] = mi;
  }
}

// Error slots: each (iteration, matrix) maximum is spread over kErrSub
// words, one per group of waves, and the decide kernel reduces them (one
// word for every wave of a launch serialised thousands of atomics: 20-45 us
// per iteration at n = 1024-2048).
constexpr int kErrSub = 64;

// Epilogue of Mk' = Mi^p·Mk (upper tiles + mirror): writes Mk' and the next
// Mi and folds max|Mk' − I| into err[b * err_stride + sub] (bitwise max of
// non-negative values, which keeps NaN; err_stride 0 = one batch maximum;
// sub spreads the workgroups over kErrSub words).
template <typename R>
struct EpiMk {
  typedef R S;
  R* Mk;
  R* Mi;
  int64_t ld, sb;
  R c1, alpha;
  typename Bits<R>::U* err;
  int err_stride;
  typename Bits<R>::U mx;
  bool vec;
  typedef NoPre Pre;
  typedef NoPre PreT;
  static constexpr bool kVoIsV = true;
  __device__ __forceinline__ bool has_t() const { return false; }
  __device__ __forceinline__ void load(int, int, int, int, int, Pre&) const {}
  __device__ __forceinline__ void load_t(int, int, int, int, PreT&) const {}
  // Row `row`, columns c0+k for k in [kbeg, n).
  __device__ __forceinline__ void run(int b, int row, int c0, const R* v, int kbeg, int n) {
    const int64_t o = (int64_t)b * sb + (int64_t)row * ld + c0;
    R mi[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      R d = v[k];
      mi[k] = mul_rn(alpha, v[k]);
      if (row == c0 + k) {
        mi[k] = add_rn(c1, mi[k]);
        d = v[k] - R(1);
      }
      if (k >= kbeg && k < n) {
        typename Bits<R>::U u = Bits<R>::of(fabs(d));
        mx = u > mx ? u : mx;
      }
    }
    st8<R, R>(Mk + o, v, kbeg, n, vec);
    st8<R, R>(Mi + o, mi, kbeg, n, vec);
  }
  __device__ __forceinline__ void put(int b, int i, int j0, const R* v, int kbeg, int n, const Pre&, R* vo) {
    run(b, i, j0, v, kbeg, n);
#pragma unroll
    for (int k = 0; k < 8; ++k) vo[k] = v[k];
  }
  __device__ __forceinline__ void put_t(int b, int j, int i0, const R* v, int n, const PreT&) {
    run(b, j, i0, v, 0, n);
  }
  // Every thread of the workgroup calls this once at the end of the
  // kernel: wave maxima, then one atomic per workgroup (one per wave
  // queued ~33 deep on each word at n = 1024).
  __device__ __forceinline__ void finish(int b) {
    typedef typename Bits<R>::U U;
    for (int off = 32; off > 0; off >>= 1) {
      U o = __shfl_xor(mx, off, 64);
      mx = o > mx ? o : mx;
    }
    __shared__ U wmax[16];
    const int nw = (int)(blockDim.x >> 6);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
      U m = wmax[0];
      for (int w = 1; w < nw; ++w) m = wmax[w] > m ? wmax[w] : m;
      atomicMax(err + (int64_t)b * err_stride + (blockIdx.x & (kErrSub - 1)), m);
    }
  }
};

// The stop rule for one run after loop iteration `it` with error e.
template <typename R>
__device__ void decide_one(RootState<R>& st, R e, int it, R tol) {
  if (st.stopped) return;
  st.iters = it + 1;
  if (it > 0 && e > st.prev_err * R(1.2)) {  // diverging: keep the last good iterate
    st.stopped = 1;
    st.result = it;
  } else {
    st.prev_err = e;
    st.result = it + 1;
    if (e < tol) st.stopped = 1;
  }
}

// Maximum of one slot's kErrSub words (bit patterns of non-negative values).
template <typename R>
__device__ R err_slot_max(const R* slot) {
  typedef typename Bits<R>::U U;
  const U* w = reinterpret_cast<const U*>(slot);
  U m = 0;
  for (int j = 0; j < kErrSub; ++j) m = w[j] > m ? w[j] : m;
  R r;
  __builtin_memcpy(&r, &m, sizeof(R));
  return r;
}

// States after iteration it (`out`) from those after it - 1 (`in`) and
// err of it. Global mode: one thread applies the rule to slot it.
// Per-matrix mode: the block applies it to each matrix (slot it·nb + b)
// and then to the summary (only these chunk-end launches refresh the
// summary; its stop flag is all the host reads of it).
template <typename R>
__global__ void __launch_bounds__(256) root_decide_kernel(const RootState<R>* in, RootState<R>* out,
                                                          const R* __restrict__ err, int it, R tol, int nb, int each) {
  if (!each) {
    if (threadIdx.x == 0) {
      RootState<R> d = in[0];
      decide_one(d, err_slot_max(err + (int64_t)it * kErrSub), it, tol);
      out[0] = d;
    }
    return;
  }
  __shared__ int live;
  if (threadIdx.x == 0) live = 0;
  __syncthreads();
  int mine = 0;
  for (int b = threadIdx.x; b < nb; b += blockDim.x) {
    RootState<R> d = in[1 + b];
    decide_one(d, err_slot_max(err + ((int64_t)it * nb + b) * kErrSub), it, tol);
    out[1 + b] = d;
    mine |= !d.stopped;
  }
  if (mine) atomicOr(&live, 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    RootState<R> d = in[0];
    if (!d.stopped) {
      d.iters = it + 1;
      if (!live) d.stopped = 1;
    }
    out[0] = d;
  }
}

// Store epilogue of iteration it + 1's first launch (X·Mi, paired with
// Mi·Mi for one matrix) that makes the stop decision of iteration `it`
// itself: every wave reduces the kErrSub error words (one per lane) and
// applies the rule to the state after it - 1, all waves alike; the first
// workgroup of each run records the state after `it` for the later
// launches. A stopped run skips the product.
template <typename R>
struct EpiStoreDecide : EpiStore<R, R> {
  const RootState<R>* prev;  // states after iteration it - 1
  RootState<R>* next;        // states after iteration it (written here)
  const R* err;              // error words of iteration it
  int it;
  R tol;
  int state0;      // state index of run 0 (1 in per-matrix mode, else 0)
  int per_matrix;  // batch entry b is run b (own state and error words);
                   // else every entry belongs to run 0 (one batch-wide
                   // rule, or the X·Mi / Mi·Mi pair of one matrix)
  __device__ __forceinline__ bool skip(int b, bool first) const {
    typedef typename Bits<R>::U U;
    static_assert(kErrSub == 64, "one error word per lane");
    const int r = per_matrix ? b : 0;
    const int s = state0 + r;
    const U* w = reinterpret_cast<const U*>(err + (int64_t)r * kErrSub);
    U m = w[threadIdx.x & (kErrSub - 1)];
    for (int off = 32; off > 0; off >>= 1) {
      const U o = __shfl_xor(m, off, 64);
      m = o > m ? o : m;
    }
    R e;
    __builtin_memcpy(&e, &m, sizeof(R));
    RootState<R> d = prev[s];
    decide_one(d, e, it, tol);
    if (first && b == r && threadIdx.x == 0) next[s] = d;
    return d.stopped != 0;
  }
};

// out = sym(X_result) cast to the input dtype.
template <typename R, typename TO>
__global__ void __launch_bounds__(256) root_final_kernel(const R* __restrict__ X0, const R* __restrict__ X1,
                                                         const RootState<R>* st, int each, int64_t n, int64_t ld,
                                                         int64_t sb, TO* __restrict__ out) {
  __shared__ R t1[32][33], t2[32][33];
  const int b = blockIdx.z;
  const R* X = (st[each ? 1 + b : 0].result & 1) ? X1 : X0;
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const R* Xb = X + (int64_t)b * sb;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int rr = ty; rr < 32; rr += 8) {
    int64_t r = r0 + rr, c = c0 + tx;
    t1[rr][tx] = (r < n && c < n) ? Xb[r * ld + c] : R(0);
    int64_t r2 = c0 + rr, c2 = r0 + tx;
    t2[rr][tx] = (r2 < n && c2 < n) ? Xb[r2 * ld + c2] : R(0);
  }
  __syncthreads();
  TO* ob = out + (int64_t)b * n * n;
  for (int rr = ty; rr < 32; rr += 8) {
    int64_t r = r0 + rr, c = c0 + tx;
    if (r < n && c < n) ob[r * n + c] = convert<TO>(R(0.5) * (t1[rr][tx] + t2[tx][rr]));
  }
}

constexpr int kRootBufs = 10;

// Host copies of the stop state after each chunk of iterations, two per
// host thread, in pinned memory so that the copies are asynchronous and the
// host can enqueue the next chunk before it waits for this one's state.
// Allocated on first use and kept until the process ends.
constexpr size_t kPinSlot = 64;
static_assert(sizeof(RootState<double>) <= kPinSlot && sizeof(RootState<float>) <= kPinSlot, "state copy slot");
static char* pinned_states() {
  static thread_local char* buf = nullptr;
  if (buf == nullptr) {
    void* p = nullptr;
    if (hipHostMalloc(&p, 2 * kPinSlot, hipHostMallocPortable) != hipSuccess) return nullptr;
    buf = static_cast<char*>(p);
  }
  return buf;
}

// each: per-matrix stop mode (err slots and states per matrix).
template <typename R>
size_t root_ws_bytes_t(int64_t batch, int64_t n, int64_t max_iter, bool each) {
  int64_t ld = round_up(n, kPadK);
  size_t bytes = 0;
  auto add = [&](size_t b) { bytes = round_up(bytes, 256) + b; };
  add(sizeof(double) * kRedBlocks * batch);
  add(sizeof(R) * batch);
  add(sizeof(R) * batch);
  add(sizeof(R) * std::max<int64_t>(max_iter, 1) * (each ? batch : 1) * kErrSub);
  add(sizeof(RootState<R>) * 2 * (each ? 1 + batch : 1));
  for (int i = 0; i < kRootBufs; ++i) add(sizeof(R) * batch * n * ld);
  return bytes + 256;
}

// iters_out: one count (global mode) or one per matrix (each).
template <typename TI, typename R>
int root_t(const TI* A, TI* out, int64_t batch, int64_t n, int64_t p, double damping, int64_t max_iter, double tol,
           bool each, void* ws, size_t ws_bytes, int64_t* iters_out, hipStream_t stream) {
  typedef typename Bits<R>::U U;
  PTO_REQUIRE(p >= 1, "inverse_matrix_root: p must be a positive integer");
  PTO_REQUIRE(n <= INT32_MAX && batch <= 65535 && max_iter <= INT32_MAX && max_iter * batch <= INT32_MAX,
              "inverse_matrix_root: shape too large");
  if (iters_out)
    for (int64_t b = 0; b < (each ? batch : 1); ++b) iters_out[b] = 0;
  if (batch == 0 || n == 0) return 0;
  const int64_t ld = round_up(n, kPadK), sb = n * ld;
  const int nb = (int)batch;
  Carver cv(ws, ws_bytes);
  double* partial = cv.take<double>(kRedBlocks * batch);
  R* z = cv.take<R>(batch);
  R* xs = cv.take<R>(batch);
  const int64_t n_err = std::max<int64_t>(max_iter, 1) * (each ? batch : 1) * kErrSub;
  const int64_t n_st = each ? 1 + batch : 1;
  R* err = cv.take<R>(n_err);
  RootState<R>* st = cv.take<RootState<R>>(2 * n_st);  // two slots of n_st
  R* buf[kRootBufs];
  for (int i = 0; i < kRootBufs; ++i) buf[i] = cv.take<R>(batch * sb);
  PTO_REQUIRE(!cv.overflow, "inverse_matrix_root: workspace too small");
  R* M = buf[0];
  R* X[2] = {buf[1], buf[2]};
  R* Mi[2] = {buf[3], buf[4]};
  R* Mk[2] = {buf[5], buf[6]};
  R* tmp[3] = {buf[7], buf[8], buf[9]};

  const R c1 = static_cast<R>(1.0 + 1.0 / (double)p);
  const R alpha = static_cast<R>(-1.0 / (double)p);
  {
    dim3 grid((unsigned)((ld + 31) / 32), (unsigned)((n + 31) / 32), (unsigned)nb);
    hipLaunchKernelGGL((root_sym_kernel<TI, R>), grid, dim3(256), 0, stream, A, n, n * n, static_cast<R>(damping), M,
                       ld, sb);
    PTO_LAUNCHED("root_sym");
  }
  if (launch_sumsq<R>(M, n, n, ld, sb, nb, partial, stream)) return -1;
  hipLaunchKernelGGL(root_scale_kernel<R>, dim3(nb), dim3(256), 0, stream, partial, (int)p,
                     std::numeric_limits<R>::min(), z, xs);
  PTO_LAUNCHED("root_scale");
  {
    unsigned blocks = (unsigned)std::min<int64_t>((sb + 255) / 256, 2048);
    hipLaunchKernelGGL(root_init_kernel<R>, dim3(blocks, nb), dim3(256), 0, stream, M, n, ld, sb, z, xs, c1, alpha,
                       X[0], Mk[0], Mi[0]);
    PTO_LAUNCHED("root_init");
  }
  // Pads of the buffers written only by MFMA epilogues must read as zero.
  for (R* q : {X[1], Mi[1], Mk[1], tmp[0], tmp[1], tmp[2]})
    if (launch_zero_cols<R>(q, n, ld, n, sb, nb, stream)) return -1;
  if (launch_fill<R>(err, n_err, R(0), stream)) return -1;
  if (launch_fill<int>(reinterpret_cast<int*>(st), 2 * n_st * (int64_t)(sizeof(RootState<R>) / sizeof(int)), 0,
                      stream))
    return -1;
  // states after iteration i (slot of i = -1: the zeroed initial state)
  auto slot = [&](int64_t i) -> RootState<R>* { return st + (i & 1) * n_st; };

  // GEMMs skip a stopped run: the one state, or matrix b's own (set per
  // iteration to the states after the previous one)
  const int* guard = nullptr;
  const int guard_stride = each ? (int)(sizeof(RootState<R>) / sizeof(int)) : 0;
  // dst = P·Q for symmetric Q (Q's rows are its columns); upper = the
  // product is symmetric too, computed on upper tiles and mirrored.
  auto product = [&](const R* P, const R* Q, R* dst, bool upper, const char* name) -> int {
    GemmArgs g{P, ld, sb, Q, ld, sb, (int)n, (int)n, (int)ld, 0, 0, guard, guard_stride};
    EpiStore<R, R> e{dst, ld, sb, vec_ok<R>(dst, ld, sb)};
    if (upper) return launch_gemm<R, true, EpiStore<R, R>, true>(g, e, nb, stream, name);
    return launch_gemm<R, false, EpiStore<R, R>, true>(g, e, nb, stream, name);
  };

  // One matrix, p >= 2: X·Mi and the first power product Mi·Mi share their
  // Q operand (Mi), so they run as one launch of two "matrices" whose P and
  // output strides are the buffers' distances (twice the workgroups for a
  // one-matrix launch that would leave CUs idle; each product's arithmetic
  // is unchanged).
  const bool pair = nb == 1 && p >= 2;
  // The first launch of iteration it >= 1 decides iteration it - 1 itself.
  auto decider = [&](int it, R* dst, int64_t sd, bool per_matrix) {
    return EpiStoreDecide<R>{{dst, ld, sd, vec_ok<R>(dst, ld, sd)},
                             slot(it - 2),
                             slot(it - 1),
                             err + (int64_t)(it - 1) * (each ? nb : 1) * kErrSub,
                             it - 1,
                             static_cast<R>(tol),
                             each ? 1 : 0,
                             per_matrix ? 1 : 0};
  };
  auto product_pair = [&](int it, const R* P0, R* d0, const R* P1, R* d1, const R* Q, const char* name) -> int {
    GemmArgs g{P0, ld, (int64_t)(P1 - P0), Q, ld, 0, (int)n, (int)n, (int)ld, 0, 0, guard, 0};
    const int64_t sd = (int64_t)(d1 - d0);
    if (it > 0) {
      g.guard = nullptr;
      return launch_gemm<R, true, EpiStoreDecide<R>, true>(g, decider(it, d0, sd, false), 2, stream, name);
    }
    EpiStore<R, R> e{d0, ld, sd, vec_ok<R>(d0, ld, sd)};
    return launch_gemm<R, true, EpiStore<R, R>, true>(g, e, 2, stream, name);
  };

  auto iteration = [&](int it) -> int {
    const int cur = it & 1, nxt = cur ^ 1;
    guard = &slot(it - 1)[each ? 1 : 0].stopped;
    // X_{it+1} = X_it · Mi (symmetric: both are polynomials in M); with
    // `pair`, tmp[0] = Mi·Mi in the same launch
    if (pair) {
      if (product_pair(it, X[cur], X[nxt], Mi[cur], tmp[0], Mi[cur], "root_xmi_pow")) return -1;
    } else if (it > 0) {
      GemmArgs g{X[cur], ld, sb, Mi[cur], ld, sb, (int)n, (int)n, (int)ld, 0, 0, nullptr, 0};
      if (launch_gemm<R, true, EpiStoreDecide<R>, true>(g, decider(it, X[nxt], sb, each), nb, stream, "root_xmi"))
        return -1;
    } else if (product(X[cur], Mi[cur], X[nxt], true, "root_xmi")) {
      return -1;
    }
    // S = Mi^p (torch.linalg.matrix_power order: direct for p <= 3, else
    // binary powering from the least significant bit; its first product is
    // always Mi·Mi, into tmp[0])
    const R* S = nullptr;
    if (p == 1) {
      S = Mi[cur];
    } else if (p == 2) {
      if (!pair && product(Mi[cur], Mi[cur], tmp[0], true, "root_pow")) return -1;
      S = tmp[0];
    } else if (p == 3) {
      if (!pair && product(Mi[cur], Mi[cur], tmp[0], true, "root_pow")) return -1;
      if (product(tmp[0], Mi[cur], tmp[1], true, "root_pow")) return -1;
      S = tmp[1];
    } else {
      const R* zp = nullptr;   // current power Mi^(2^k)
      const R* res = nullptr;  // accumulated result
      int64_t k = p;
      auto free_tmp = [&]() -> R* {
        for (R* t : tmp)
          if (t != zp && t != res) return t;
        return nullptr;
      };
      while (k > 0) {
        const int64_t bit = k & 1;
        k >>= 1;
        if (zp == nullptr) {
          zp = Mi[cur];
        } else {
          R* d = free_tmp();
          if (pair && zp == Mi[cur]) {
            PTO_REQUIRE(d == tmp[0], "inverse_matrix_root: power buffers");  // Mi·Mi is there already
          } else if (product(zp, zp, d, true, "root_pow")) {
            return -1;
          }
          zp = d;
        }
        if (bit) {
          if (res == nullptr) {
            res = zp;
          } else {
            R* d = free_tmp();
            if (product(res, zp, d, true, "root_pow")) return -1;
            res = d;
          }
        }
      }
      S = res;
    }
    // Mk_{it+1} = S · Mk_it, with the fused next-Mi / error epilogue.
    {
      GemmArgs g{S, ld, sb, Mk[cur], ld, sb, (int)n, (int)n, (int)ld, 0, 0, guard, guard_stride};
      EpiMk<R> e{Mk[nxt], Mi[nxt], ld, sb, c1, alpha,
                 reinterpret_cast<U*>(err + (int64_t)it * (each ? nb : 1) * kErrSub), each ? kErrSub : 0, U(0), vec_ok<R>(Mk[nxt], ld, sb) && vec_ok<R>(Mi[nxt], ld, sb)};
      if (launch_gemm<R, true, EpiMk<R>, true>(g, e, nb, stream, "root_mk")) return -1;
    }
    return 0;
  };

  // Each recorded event marks a state copy into this thread's pinned slots;
  // leaving (an error included) waits for it, so no copy lands after the
  // slots are reused.
  struct Events {
    hipEvent_t e[2] = {nullptr, nullptr};
    bool recorded[2] = {false, false};
    ~Events() {
      for (int i = 0; i < 2; ++i) {
        if (!e[i]) continue;
        if (recorded[i]) (void)hipEventSynchronize(e[i]);
        (void)hipEventDestroy(e[i]);
      }
    }
  } ev;
  for (hipEvent_t& x : ev.e) PTO_HIP(hipEventCreateWithFlags(&x, hipEventDisableTiming));
  char* pin = pinned_states();
  PTO_REQUIRE(pin != nullptr, "inverse_matrix_root: pinned host buffer allocation failed");
  RootState<R>* hs[2] = {reinterpret_cast<RootState<R>*>(pin), reinterpret_cast<RootState<R>*>(pin + kPinSlot)};

  RootState<R> host{};
  int64_t it = 0;
  int64_t chunk = 2;
  // Enqueue the next chunk of iterations, the chunk-end decide and the copy
  // of the state after the chunk into hs[k].
  auto enqueue_chunk = [&](int k) -> int {
    const int64_t end = std::min<int64_t>(max_iter, it + chunk);
    for (; it < end; ++it)
      if (iteration((int)it)) return -1;
    hipLaunchKernelGGL(root_decide_kernel<R>, dim3(1), dim3(each ? 256 : 64), 0, stream, slot(it - 2),
                       slot(it - 1), err, (int)(it - 1), static_cast<R>(tol), nb, (int)each);
    PTO_LAUNCHED("root_decide");
    PTO_HIP(hipMemcpyAsync(hs[k], slot(it - 1), sizeof(RootState<R>), hipMemcpyDeviceToHost, stream));
    PTO_HIP(hipEventRecord(ev.e[k], stream));
    ev.recorded[k] = true;
    chunk = std::min<int64_t>(chunk * 2, 16);
    return 0;
  };
  if (max_iter > 0) {
    if (enqueue_chunk(0)) return -1;
    for (int k = 0;; k ^= 1) {
      // the next chunk is enqueued before the host waits for this one, so
      // the device does not idle while the host reads the state
      const bool ahead = it < max_iter;
      if (ahead && enqueue_chunk(k ^ 1)) return -1;
      PTO_HIP(hipEventSynchronize(ev.e[k]));
      host = *hs[k];
      if (!ahead || host.stopped) break;  // a chunk enqueued past a stop only skips
    }
  }
  const RootState<R>* last = slot(it - 1);  // states after the last iteration run
  {
    dim3 grid((unsigned)((n + 31) / 32), (unsigned)((n + 31) / 32), (unsigned)nb);
    hipLaunchKernelGGL((root_final_kernel<R, TI>), grid, dim3(256), 0, stream, X[0], X[1], last, (int)each, n, ld,
                       sb, out);
    PTO_LAUNCHED("root_final");
  }
  if (iters_out && !each) *iters_out = host.iters;
  if (iters_out && each) {
    std::vector<RootState<R>> all((size_t)nb);
    PTO_HIP(hipMemcpyAsync(all.data(), last + 1, sizeof(RootState<R>) * nb, hipMemcpyDeviceToHost, stream));
    PTO_HIP(hipStreamSynchronize(stream));
    for (int b = 0; b < nb; ++b) iters_out[b] = all[b].iters;
  }
  return 0;
}

template <typename TI>
int root_dispatch(const TI* A, TI* out, int root_f64, int64_t batch, int64_t n, int64_t p, double damping,
                  int64_t max_iter, double tol, bool each, void* ws, size_t ws_bytes, int64_t* iters_out,
                  hipStream_t s) {
  if (root_f64)
    return root_t<TI, double>(A, out, batch, n, p, damping, max_iter, tol, each, ws, ws_bytes, iters_out, s);
  return root_t<TI, float>(A, out, batch, n, p, damping, max_iter, tol, each, ws, ws_bytes, iters_out, s);
}

int root_entry(const void* A, void* out, int dtype, int root_f64, int64_t batch, int64_t n, int64_t p,
               double damping, int64_t max_iter, double tol, bool each, void* workspace, size_t ws_bytes,
               int64_t* iters_out, void* stream) {
  PTO_REQUIRE(batch >= 0 && n >= 0 && max_iter >= 0, "inverse_matrix_root: negative extent or max_iter");
  PTO_REQUIRE(batch * n == 0 || (A && out && workspace), "inverse_matrix_root: null input, output or workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case kF32:
      return root_dispatch<float>(static_cast<const float*>(A), static_cast<float*>(out), root_f64, batch, n, p,
                                  damping, max_iter, tol, each, workspace, ws_bytes, iters_out, s);
    case kF64:
      return root_dispatch<double>(static_cast<const double*>(A), static_cast<double*>(out), root_f64, batch, n, p,
                                   damping, max_iter, tol, each, workspace, ws_bytes, iters_out, s);
    case kBF16:
      return root_dispatch<bf16>(static_cast<const bf16*>(A), static_cast<bf16*>(out), root_f64, batch, n, p,
                                 damping, max_iter, tol, each, workspace, ws_bytes, iters_out, s);
    default:
      PTO_REQUIRE(false, "inverse_matrix_root: unsupported dtype code");
  }
}

}  // namespace
}  // namespace pto

extern "C" {

size_t pto_inverse_root_workspace_bytes(int root_f64, int64_t batch, int64_t n, int64_t max_iter) {
  return root_f64 ? pto::root_ws_bytes_t<double>(batch, n, max_iter, false)
                  : pto::root_ws_bytes_t<float>(batch, n, max_iter, false);
}

int pto_inverse_root(const void* A, void* out, int dtype, int root_f64, int64_t batch, int64_t n, int64_t p,
                     double damping, int64_t max_iter, double tol, void* workspace, size_t ws_bytes,
                     int64_t* iters_out, void* stream) {
  return pto::root_entry(A, out, dtype, root_f64, batch, n, p, damping, max_iter, tol, false, workspace, ws_bytes,
                         iters_out, stream);
}

size_t pto_inverse_root_each_workspace_bytes(int root_f64, int64_t batch, int64_t n, int64_t max_iter) {
  return root_f64 ? pto::root_ws_bytes_t<double>(batch, n, max_iter, true)
                  : pto::root_ws_bytes_t<float>(batch, n, max_iter, true);
}

int pto_inverse_root_each(const void* A, void* out, int dtype, int root_f64, int64_t batch, int64_t n, int64_t p,
                          double damping, int64_t max_iter, double tol, void* workspace, size_t ws_bytes,
                          int64_t* iters_out, void* stream) {
  return pto::root_entry(A, out, dtype, root_f64, batch, n, p, damping, max_iter, tol, true, workspace, ws_bytes,
                         iters_out, stream);
}

}  // extern "C"
