"""CPU oracle for the pytorch_opt.ops hot path — TEST INFRASTRUCTURE ONLY.

Plain numpy restatement of the reference algorithms, against which
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg check the
HIP kernels. Nothing in
the product imports this module.

Every function cites the reference lines it restates (paths relative to
the reference checkout). Arrays are numpy; ``dtype`` selects the working
precision (np.float32 mirrors the reference's fp32 path, np.float64 gives a
high-precision check). bf16 inputs are passed as float32 arrays holding
bf16-representable values.

Pinning (tests/test_oracle.py):
  ns5                  closed form via SVD (NS acts per singular value),
                       semi-orthogonal input -> scalar multiple, transpose
                       symmetry, batched == loop, the reference's band test
  kron_factor_update   closed form sums / EMA (tests/test_ops_reference.py:92-108),
                       brute-force outer products
  inverse_root         closed form Q diag(l^(-1/p)) Qᵀ (tests/test_ops_reference.py:16-21),
                       newton ~ eigh (:24-29), damping (:32-38), residual
  coupled_newton       values through inverse_root's closed forms; the stop
                       rule's iteration count is pinned in float64 (where
                       convergence, not rounding noise, ends the loop) by the
                       iteration bound of the quadratic phase; in float32,
                       run with the root kernels' product order
                       (gemm_emu.c as ``matmul``), its iterate, err sequence
                       and iteration count equal the kernels' bit for bit
                       on the config-4 inputs (tests/test_root_emulated.py),
                       which pins both sides against each other
  gram_update          brute-force sum of outer products, clone/EMA/mean
  precond_apply        associativity / brute force in float64
  two_sided_product    orthogonal round trip Q·(QᵀXQ)·Qᵀ = X, permutation
                       and sign-flip closed forms, transpose identities
"""

from __future__ import annotations

import numpy as np

NS_COEFFS = (3.4445, -4.7750, 2.0315)


def _t(x: np.ndarray) -> np.ndarray:
    return np.swapaxes(x, -1, -2)


def sym(x: np.ndarray) -> np.ndarray:
    """(X + Xᵀ)/2 — pytorch_opt/ops/reference.py:13-14."""
    return x.dtype.type(0.5) * (x + _t(x))


def ns5(G, steps=5, coeffs=NS_COEFFS, eps=1e-7, dtype=None):
    """Quintic Newton–Schulz — pytorch_opt/ops/reference.py:71-97.

    Returns the work-precision result (the caller casts to its dtype).
    """
    G = np.asarray(G)
    if G.ndim < 2:
        raise ValueError("newton_schulz_orthogonalize expects a matrix (ndim >= 2)")
    if dtype is None:
        dtype = np.float64 if G.dtype == np.float64 else np.float32
    a, b, c = (dtype(v) for v in coeffs)
    X = G.astype(dtype)
    flip = X.shape[-2] > X.shape[-1]
    if flip:
        X = _t(X)
    nrm = np.sqrt(np.sum(X.astype(np.float64) ** 2, axis=(-2, -1), keepdims=True)).astype(dtype)
    X = X / (nrm + dtype(eps))
    for _ in range(steps):
        A = X @ _t(X)
        B = b * A + c * (A @ A)
        X = a * X + B @ X
    if flip:
        X = _t(X)
    return np.ascontiguousarray(X)


def ns5_flops(m, n, steps=5):
    """Algorithmic FLOPs of NS5 on an m x n matrix (LAWN-41: symmetric
    products m(m+1)k, others 2mnk), after the rows <= cols transpose."""
    m, n = min(m, n), max(m, n)
    return steps * (m * (m + 1) * n + m * m * (m + 1) + 2 * m * m * n)


def kron_factor_update(L, R, G, beta2=1.0, dtype=None):
    """L ← β·L + (1−β)·G·Gᵀ, R ← β·R + (1−β)·Gᵀ·G — reference.py:100-114.

    Functional: returns new (L, R).
    """
    G = np.asarray(G)
    if G.ndim != 2:
        raise ValueError(f"G must be 2D, got shape {G.shape}")
    dtype = dtype or G.dtype.type
    G = G.astype(dtype)
    L = np.asarray(L, dtype=dtype)
    R = np.asarray(R, dtype=dtype)
    left, right = G @ G.T, G.T @ G
    if beta2 == 1.0:
        return L + left, R + right
    bb, aa = dtype(beta2), dtype(1.0 - beta2)
    return L * bb + aa * left, R * bb + aa * right


def coupled_newton(M, p, max_iter=100, tol=1e-10, matmul=np.matmul, errors=None):
    """Coupled Newton for M^(-1/p) — pytorch_opt/ops/reference.py:17-40.

    Returns (X, iterations executed). M is [..., n, n] in the root dtype.
    ``matmul`` computes every product (a test can change the summation
    order; the default is numpy's BLAS). ``errors``, a list, receives each
    iteration's err = max|Mk − I|.
    """
    dt = M.dtype.type
    n = M.shape[-1]
    eye = np.broadcast_to(np.eye(n, dtype=M.dtype), M.shape)
    inv_p = 1.0 / p
    fro = np.sqrt(np.sum(M.astype(np.float64) ** 2, axis=(-2, -1))).astype(M.dtype)
    fro = np.maximum(fro, np.finfo(M.dtype).tiny)
    z = (dt(1.0 + p) / (dt(2.0) * fro))[..., None, None]
    X = eye * np.power(z, dt(inv_p))
    Mk = M * z
    good, good_err = X, None
    iters = 0
    for _ in range(max_iter):
        iters += 1
        Mi = dt(1.0 + inv_p) * eye + dt(-inv_p) * Mk
        X = matmul(X, Mi)
        Mk = matmul(matrix_power(Mi, p, matmul), Mk)
        err = np.max(np.abs(Mk - eye))
        if errors is not None:
            errors.append(float(err))
        if good_err is not None and err > good_err * dt(1.2):
            return good, iters
        good, good_err = X, err
        if err < dt(tol):
            break
    return X, iters


def matrix_power(A, p, matmul=np.matmul):
    """A**p with the product order of torch.linalg.matrix_power: direct for
    p <= 3, else binary powering from the least significant bit."""
    if p == 1:
        return A.copy()
    if p == 2:
        return matmul(A, A)
    if p == 3:
        return matmul(matmul(A, A), A)
    z = res = None
    k = p
    while k > 0:
        bit, k = k & 1, k >> 1
        z = A if z is None else matmul(z, z)
        if bit:
            res = z if res is None else matmul(res, z)
    return res


def inverse_root(A, p, damping=0.0, method="auto", root_dtype=np.float64, max_iter=100, tol=1e-10,
                 matmul=np.matmul, errors=None):
    """(A + damping·I)^(-1/p) — pytorch_opt/ops/reference.py:43-68.

    Returns (root in the input dtype, iterations; 0 for eigh). ``matmul``
    and ``errors`` as in coupled_newton.
    """
    if int(p) != p or p < 1:
        raise ValueError(f"p must be a positive integer, got {p}")
    if method not in ("auto", "eigh", "newton"):
        raise ValueError(f"method must be one of ('auto', 'eigh', 'newton'), got {method!r}")
    A = np.asarray(A)
    M = sym(A.astype(root_dtype))
    if damping:
        M = M + root_dtype(damping) * np.eye(M.shape[-1], dtype=root_dtype)
    if method == "newton":
        X, iters = coupled_newton(M, int(p), max_iter, tol, matmul, errors)
    else:
        lam, V = np.linalg.eigh(M)
        lam = np.maximum(lam, 1e-30)
        X = (V * lam[..., None, :] ** (-1.0 / p)) @ _t(V)
        iters = 0
    return sym(X).astype(A.dtype), iters


def root_residual(X, A, p, damping=0.0):
    """‖X^p (A + damping·I) − I‖_F / √n in float64, per matrix."""
    X = np.asarray(X, dtype=np.float64)
    A = np.asarray(A, dtype=np.float64)
    n = A.shape[-1]
    M = A + damping * np.eye(n)
    P = np.linalg.matrix_power(X, p) if X.ndim == 2 else np.stack([np.linalg.matrix_power(x, p) for x in X])
    return np.sqrt(np.sum((P @ M - np.eye(n)) ** 2, axis=(-2, -1))) / np.sqrt(n)


def precond_apply(Lr, G, Rr):
    """(L_root·G)·R_root — pytorch_opt/ops/reference.py:117-121."""
    return (np.asarray(Lr) @ np.asarray(G)) @ np.asarray(Rr)


def two_sided_product(A, X, B, transpose_a=False, transpose_b=False):
    """op(A)·X·op(B), left to right — SOAP's rotations and transport,
    pytorch_opt/optim/soap.py:103-107 (C_L²ᵀ·v·C_R²) and :123-125
    (Q_Lᵀ·x·Q_R, Q_L·x·Q_Rᵀ)."""
    A, X, B = np.asarray(A), np.asarray(X), np.asarray(B)
    return ((_t(A) if transpose_a else A) @ X) @ (_t(B) if transpose_b else B)


def gram_update(F, X, beta=0.0, alpha=1.0, append_ones=False, dtype=np.float32):
    """F ← β·F + α·X̃ᵀX̃ (β = 0 overwrites), X̃ = [X, 1] if append_ones.

    The K-FAC batch factor and blend of pytorch_opt/curvature/kron.py:95-113
    (A_b = ãᵀã/n, clone / EMA / running mean) written as one update.
    """
    X2 = np.asarray(X, dtype=dtype).reshape(-1, np.shape(X)[-1])
    if append_ones:
        X2 = np.concatenate([X2, np.ones((X2.shape[0], 1), dtype=dtype)], axis=1)
    prod = X2.T @ X2
    if beta == 0.0:
        return dtype(alpha) * prod
    return np.asarray(F, dtype=dtype) * dtype(beta) + dtype(alpha) * prod
