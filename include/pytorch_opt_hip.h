/*
 * pytorch_opt_hip.h — C ABI of the MI355X (gfx950) backend for pytorch_opt.ops.
 *
 * One shared library, libpytorch_opt_hip.so, built from the .hip sources in
 * pytorch-opt_amd/csrc. It replaces the reference's compiled
 * backend object `_NATIVE` (pytorch_opt/ops/__init__.py:18, built by
 * pytorch_opt/ops/native_build.py:10-21 from
 * pytorch_opt/ops/csrc/pytorch_opt_ops.cpp). The Python adapter
 * (pytorch_opt/ops/_hip.py) turns tensors into the plain pointers below.
 *
 * Conventions for every compute entry point:
 *  - Pointers are device pointers to contiguous row-major data. Batched
 *    arguments are `batch` matrices laid out back to back.
 *  - `dtype` is one of PTO_F32, PTO_F64, PTO_BF16.
 *  - `workspace` is caller-owned device memory of at least the size the
 *    matching *_workspace_bytes query returns, at any alignment (the
 *    library aligns its blocks inside it; the sizes include that slack).
 *    The library never allocates device memory and keeps no state between
 *    calls (the coupled-Newton roots keep two small pinned host slots per
 *    host thread for their stop state). A null operand, output or
 *    workspace of a non-empty call is an error reported before any launch.
 *  - `stream` is a hipStream_t; all kernels are enqueued on it and the call
 *    returns without synchronising, except pto_inverse_root and
 *    pto_inverse_root_each, which read their stop state back once per chunk
 *    of iterations, one chunk behind the enqueued work (the reference syncs
 *    once per iteration: csrc/pytorch_opt_ops.cpp:29).
 *  - Return value 0 means success. A non-zero value means failure, and
 *    pto_last_error() returns a message (thread-local).
 */
#ifndef PYTORCH_OPT_HIP_H_
#define PYTORCH_OPT_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { PTO_F32 = 0, PTO_F64 = 1, PTO_BF16 = 2 };

/* Message of the last failed call on this thread ("" if none). */
const char* pto_last_error(void);
/* Library version as major*10000 + minor*100 + patch. */
int pto_version(void);
/* HIP runtime version the library is bound to, or -1. */
int pto_runtime_version(void);

/*
 * Newton–Schulz orthogonalization. Replaces
 *   _NATIVE.newton_schulz_orthogonalize(G, steps, a, b, c, eps)
 * called at pytorch_opt/ops/__init__.py:70; semantics of
 * pytorch_opt/ops/reference.py:71-97 and csrc/pytorch_opt_ops.cpp:65-81.
 * G and out are [batch, rows, cols] of `dtype`. bf16 computes with bf16
 * operands and fp32 accumulation when min(rows, cols) >= 128 (below that
 * the fp32 chain runs and the result is rounded once, as the reference
 * computes every bf16 input); f32/f64 stay in their own precision.
 * out may be G itself (in place) but must not otherwise overlap it. G may
 * sit at any element alignment (a G that is not 16-byte aligned is copied
 * into the workspace first).
 */
size_t pto_ns5_workspace_bytes(int dtype, int64_t batch, int64_t rows, int64_t cols);
int pto_ns5(const void* G, void* out, int dtype, int64_t batch, int64_t rows, int64_t cols, int64_t steps,
            double a, double b, double c, double eps, void* workspace, size_t ws_bytes, void* stream);

/*
 * pto_ns5 without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). It has no counterpart in the
 * reference. The workspace is a static 256 MiB device array in the library,
 * one per GPU. It sits in a code object of its own (no kernels), which the
 * runtime loads on a GPU at the first no-alloc call there (the call takes
 * the array's address), so processes that never call this entry point do
 * not hold it; once loaded it is held until the process ends. The first
 * call on a GPU is therefore the one to make outside graph capture or a
 * loop that must not allocate. A call whose pto_ns5_workspace_bytes exceeds
 * 256 MiB fails before any launch (bf16 up to one 4096x11008 matrix, fp32
 * up to 2048x8192). The call itself allocates nothing: no hipMalloc, no
 * events (kernel timing is off for it). Every call on a GPU shares that
 * GPU's array, so calls that overlap on one GPU (other streams, other
 * threads) race; serialise them. G, out and the result are as for pto_ns5.
 */
int pto_ns5_noalloc(const void* G, void* out, int dtype, int64_t batch, int64_t rows, int64_t cols, int64_t steps,
                    double a, double b, double c, double eps, void* stream);

/*
 * In-place Kronecker factor update. Replaces
 *   _NATIVE.kron_factor_update_(L, R, G, beta2)
 * called at pytorch_opt/ops/__init__.py:76; semantics of
 * pytorch_opt/ops/reference.py:100-114 and csrc/pytorch_opt_ops.cpp:83-94:
 *   L <- beta2*L + (1-beta2)*G*G^T,  R <- beta2*R + (1-beta2)*G^T*G
 * (beta2 == 1: L += G*G^T, R += G^T*G). G [m,n], L [m,m], R [n,n].
 */
size_t pto_kron_workspace_bytes(int dtype, int64_t m, int64_t n);
int pto_kron_factor_update(void* L, void* R, const void* G, int dtype, int64_t m, int64_t n, double beta2,
                           void* workspace, size_t ws_bytes, void* stream);

/*
 * Batched factor update (additive; the reference updates one parameter's
 * factors per call, pytorch_opt/optim/shampoo.py:98-100 and
 * pytorch_opt/optim/soap.py:88-90): for b < batch,
 *   L[b] <- beta2*L[b] + (1-beta2)*G[b]*G[b]^T,  R[b] <- ... G[b]^T*G[b].
 * G is one contiguous stack [batch][m][n]; L and R are host arrays of
 * batch device pointers to distinct [m,m] / [n,n] tensors. batch <= 64.
 * In f32 and f64 each factor gets exactly the bits pto_kron_factor_update
 * gives it. In bf16 the tile the library picks depends on the batch, and
 * the 192x192 tile sums even and odd K tiles in separate accumulators, so
 * a batched result may differ from the single call's in the last bits.
 */
size_t pto_kron_batched_workspace_bytes(int dtype, int64_t batch, int64_t m, int64_t n);
int pto_kron_factor_update_batched(void* const* L, void* const* R, const void* G, int dtype, int64_t batch, int64_t m,
                                   int64_t n, double beta2, void* workspace, size_t ws_bytes, void* stream);

/*
 * Gram update F <- beta*F + alpha * Xa^T Xa, Xa = [X, 1] if append_ones.
 * The reference has no compiled counterpart: it is the boundary added for
 * the K-FAC factor products pytorch_opt/curvature/kron.py:105-113 and the
 * EMA / running-mean step :95-103 (beta == 0 overwrites F).
 * X [rows, d] of x_dtype, F [d(+1), d(+1)] of f_dtype.
 * Supported (x, F) pairs: (bf16, f32), (f32, f32), (f64, f64).
 * The workspace size is 0 when X is read in place (bf16, rows % 128 == 0,
 * d % 8 == 0, no ones column, and the tile the library picks for d allows
 * it); X must then be 16-byte aligned, and workspace may be NULL.
 */
size_t pto_gram_workspace_bytes(int x_dtype, int64_t rows, int64_t d, int append_ones);
int pto_gram_update(void* F, int f_dtype, const void* X, int x_dtype, int64_t rows, int64_t d, int append_ones,
                    double beta, double alpha, void* workspace, size_t ws_bytes, void* stream);

/*
 * Inverse p-th root by the coupled Newton iteration. Replaces the "newton"
 * method of _NATIVE.inverse_matrix_root(A, p, damping, method, root_f64,
 * max_iter, tol) called at pytorch_opt/ops/__init__.py:61-62; semantics of
 * pytorch_opt/ops/reference.py:17-40,43-68 and csrc/pytorch_opt_ops.cpp:15-63.
 * A and out are [batch, n, n] of `dtype`; the iteration runs in f64 if
 * root_f64 else f32. *iters_out (may be NULL) receives the number of loop
 * iterations executed.
 */
size_t pto_inverse_root_workspace_bytes(int root_f64, int64_t batch, int64_t n, int64_t max_iter);
int pto_inverse_root(const void* A, void* out, int dtype, int root_f64, int64_t batch, int64_t n, int64_t p,
                     double damping, int64_t max_iter, double tol, void* workspace, size_t ws_bytes,
                     int64_t* iters_out, void* stream);

/*
 * The same iteration over a stack of independent matrices, each run by its
 * own rule: its own err, divergence guard, stop and returned iterate, so
 * out[b] and iters_out[b] (int64_t[batch], may be NULL) equal what one
 * pto_inverse_root call on matrix b alone returns. The reference calls
 * inverse_matrix_root once per factor (pytorch_opt/optim/shampoo.py:112-117);
 * this is that loop in one launch sequence, for callers that stack
 * same-shape factors. pto_inverse_root keeps the reference's batch-wide
 * rule for a batched A (pytorch_opt/ops/reference.py:34, one amax over all
 * dims). batch * max_iter must stay below 2^31.
 */
size_t pto_inverse_root_each_workspace_bytes(int root_f64, int64_t batch, int64_t n, int64_t max_iter);
int pto_inverse_root_each(const void* A, void* out, int dtype, int root_f64, int64_t batch, int64_t n, int64_t p,
                          double damping, int64_t max_iter, double tol, void* workspace, size_t ws_bytes,
                          int64_t* iters_out, void* stream);

/*
 * Two-sided preconditioner application. Replaces
 *   _NATIVE.precond_apply_two_sided(L_root, G, R_root)
 * called at pytorch_opt/ops/__init__.py:83; semantics of
 * pytorch_opt/ops/reference.py:117-121: out = (L_root*G)*R_root.
 * L_root [m,m], G [m,n], R_root [n,n], out [m,n].
 */
size_t pto_precond_apply_workspace_bytes(int dtype, int64_t m, int64_t n);
int pto_precond_apply(const void* L_root, const void* G, const void* R_root, void* out, int dtype, int64_t m,
                      int64_t n, void* workspace, size_t ws_bytes, void* stream);

/*
 * Two-sided product with optional transposes: out = op(A)*X*op(B),
 * op(M) = M, or Mᵀ when trans_* is non-zero, associated left to right.
 * A [m,m], X [m,n], B [n,n], out [m,n]. The reference has no compiled
 * counterpart: these are SOAP's eigenbasis rotations, Q_Lᵀ*X*Q_R and
 * Q_L*X*Q_Rᵀ (pytorch_opt/optim/soap.py:123-125, torch matmuls in the
 * reference), and its second-moment transport (C_L²)ᵀ*v*(C_R²) (:103-107).
 * pto_precond_apply is the case trans_a = trans_b = 0.
 */
size_t pto_two_sided_product_workspace_bytes(int dtype, int64_t m, int64_t n);
int pto_two_sided_product(const void* A, const void* X, const void* B, void* out, int dtype, int64_t m, int64_t n,
                          int trans_a, int trans_b, void* workspace, size_t ws_bytes, void* stream);

/*
 * The same over a batch, each of the two products one launch: out[b] =
 * op(A[b])*X[b]*op(B[b]) for b < batch (below 65536), A[b] = A + b*stride_a
 * (elements; 0 shares one matrix across the batch), likewise X and B; out
 * is contiguous [batch][m][n]. Serves the batched calls of
 * precond_apply_two_sided and two_sided_product (leading dims of
 * pytorch_opt/ops/reference.py:117-121, batched there by torch.matmul),
 * which the harnesses use for same-shape parameters (SOAP rotations,
 * K-FAC and EKFAC preconditioning, Shampoo's apply). shared_a / shared_b
 * in the workspace query: the matching stride is 0.
 */
size_t pto_two_sided_product_batched_workspace_bytes(int dtype, int64_t batch, int64_t m, int64_t n, int shared_a,
                                                     int shared_b);
int pto_two_sided_product_batched(const void* A, const void* X, const void* B, void* out, int dtype, int64_t batch,
                                  int64_t m, int64_t n, int64_t stride_a, int64_t stride_x, int64_t stride_b,
                                  int trans_a, int trans_b, void* workspace, size_t ws_bytes, void* stream);

/*
 * One AdamW step of a dense tensor, in place: the shared fallback of the
 * optimizers, pytorch_opt/optim/_common.py:56-79 (torch elementwise ops in
 * the reference; no compiled counterpart). With bc1 = 1 - beta1^step and
 * bc2 = 1 - beta2^step:
 *   m <- lerp(m, g, 1 - beta1);  v <- beta2*v + (1 - beta2)*g*g;
 *   u <- (m / bc1) / (sqrt(v) / bc2^0.5 + eps);  p <- p*(1 - lr*wd) - lr*u
 * each op rounded to the tensor dtype in that order. p, g, m, v hold n
 * elements of `dtype`. update_sq (device pointer, may be NULL) receives the
 * sum of u^2 in double (the Muon diagnostic, pytorch_opt/optim/muon.py:97).
 */
size_t pto_adamw_workspace_bytes(void);
int pto_adamw_step(void* p, const void* g, void* m, void* v, int dtype, int64_t n, double lr, double weight_decay,
                   double beta1, double beta2, double eps, int64_t step, double* update_sq, void* workspace,
                   size_t ws_bytes, void* stream);

/*
 * Muon's elementwise work around NS5, pytorch_opt/optim/muon.py:79-92
 * (torch elementwise ops in the reference; no compiled counterpart).
 * pto_muon_momentum: buf <- buf*mu + g (mul_ then add_), then
 *   u <- g + mu*buf (nesterov != 0; one fused multiply-add, as torch's
 *   g.add(buf, alpha=mu)) or u <- buf; u is a separate array of n elements
 *   (the caller's stacked NS5 input), buf and g are updated/read in place.
 * pto_muon_update: p <- p*decay (skipped when decay == 1), then
 *   p <- p + neg_lr*o (one fused multiply-add, as p.add_(o, alpha=neg_lr));
 *   update_sq (device pointer) receives the sum of o^2 in double, summed in
 *   a fixed order (the update_rms diagnostic, muon.py:92).
 * Each result is rounded to `dtype` in the reference's op order.
 */
size_t pto_muon_update_workspace_bytes(void);
int pto_muon_momentum(void* buf, const void* g, void* u, int dtype, int64_t n, double momentum, int nesterov,
                      void* stream);
int pto_muon_update(void* p, const void* o, int dtype, int64_t n, double decay, double neg_lr, double* update_sq,
                    void* workspace, size_t ws_bytes, void* stream);

/*
 * Shampoo's AdaGrad graft and parameter update, pytorch_opt/optim/
 * shampoo.py:133-151 (torch elementwise ops and two norms in the reference;
 * no compiled counterpart), over n elements of `dtype`:
 *   acc <- acc + g*g (addcmul_: g*g rounded, then the sum);
 *   t <- ||g / (sqrt(acc) + diag_eps)||;
 *   ratio <- t / (||P|| + 1e-30);  u <- P*ratio;
 *   momentum != 0: buf <- buf*momentum + u, u <- buf (buf must be non-NULL
 *   exactly when momentum != 0);
 *   p <- p*decay (skipped when decay == 1);  p <- p + neg_lr*u.
 * The norms are fixed-order double sums rounded to `dtype`; ratio_out
 * (device pointer to one `dtype` element, may be NULL) receives the ratio.
 */
size_t pto_shampoo_graft_workspace_bytes(void);
int pto_shampoo_graft(void* p, const void* g, void* acc, const void* P, void* buf, int dtype, int64_t n,
                      double diag_eps, double momentum, double decay, double neg_lr, void* ratio_out, void* workspace,
                      size_t ws_bytes, void* stream);

/*
 * Kernel timing with HIP events. The reference has no counterpart (its
 * StepTimer, pytorch_opt/optim/_common.py:82-98, is host wall-clock). While
 * enabled, every MFMA launch is bracketed by events on its stream;
 * pto_prof_query waits for them and returns the summed milliseconds and
 * launch count for one kernel class ("ns5_gram", "ns5_square",
 * "ns5_update", "kron_left", "kron_right", "gram_update", "root_xmi",
 * "root_pow", "root_mk", "apply_left", "apply_right", "rotate_left",
 * "rotate_right").
 */
int pto_prof_enable(int on);
int pto_prof_reset(void);
int pto_prof_query(const char* name, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* PYTORCH_OPT_HIP_H_ */
