"""Pure-torch implementations of the pytorch_opt.ops numerics.

This is the "reference" backend of the dispatch switch: it runs on any
device torch supports and is what ``set_backend("reference")`` (or ``auto``
without a loaded native library) executes. Semantics follow the reference
project's ``pytorch_opt/ops/reference.py`` line for line in meaning; each
function cites the lines it restates.
"""

from __future__ import annotations

import torch

ROOT_METHODS = ("auto", "eigh", "newton")


class OpsArgumentError(ValueError, RuntimeError):
    """Invalid op argument.

    The reference raises ValueError from its pure path
    (pytorch_opt/ops/reference.py:53-56,82-83,104-105) and RuntimeError from
    its compiled path (csrc/pytorch_opt_ops.cpp:44-46,67,84); this type is
    both, so callers written against either keep working.
    """


def _sym(A: torch.Tensor) -> torch.Tensor:
    """(A + Aᵀ)/2 over the last two dims (reference.py:13-14)."""
    return 0.5 * (A + A.mT)


def _identity_like(M: torch.Tensor) -> torch.Tensor:
    n = M.shape[-1]
    return torch.eye(n, dtype=M.dtype, device=M.device).expand_as(M)


def _matrix_power_lsb(Mi: torch.Tensor, p: int) -> torch.Tensor:
    """Mi**p with torch.linalg.matrix_power's product order."""
    return torch.linalg.matrix_power(Mi, p)


def coupled_newton(M: torch.Tensor, p: int, max_iter: int, tol: float):
    """Coupled Newton iteration for M^(-1/p); returns (X, iterations).

    Restates reference.py:17-40: scale by z = (1+p)/(2‖M‖_F), iterate
    Mi = (1+1/p)I − Mk/p, X ← X·Mi, Mk ← Mi^p·Mk and stop on
    max|Mk − I| < tol, or return the previous X when the error grows by more
    than 1.2×. The error is a single maximum over the whole batch.
    """
    eye = _identity_like(M)
    inv_p = 1.0 / p
    fro = torch.linalg.matrix_norm(M, ord="fro")
    z = (1.0 + p) / (2.0 * fro.clamp_min(torch.finfo(M.dtype).tiny))
    z = z[..., None, None]
    X = eye * z.pow(inv_p)
    Mk = M * z
    last_good, last_err = X, None
    iters = 0
    for _ in range(max_iter):
        iters += 1
        Mi = (1.0 + inv_p) * eye + (-inv_p) * Mk
        X = X @ Mi
        Mk = _matrix_power_lsb(Mi, p) @ Mk
        err = (Mk - eye).abs().amax()
        if last_err is not None and err > last_err * 1.2:
            return last_good, iters
        last_good, last_err = X, err
        if err < tol:
            break
    return X, iters


def _check_root_args(p, method):
    if int(p) != p or p < 1:
        raise OpsArgumentError(f"p must be a positive integer, got {p}")
    if method not in ROOT_METHODS:
        raise OpsArgumentError(f"method must be one of {ROOT_METHODS}, got {method!r}")


def inverse_matrix_root_with_iters(A, p, damping=0.0, method="auto", root_dtype=torch.float64,
                                   max_iter=100, tol=1e-10):
    """inverse_matrix_root plus the Newton iteration count (0 for eigh)."""
    _check_root_args(p, method)
    out_dtype = A.dtype
    M = _sym(A.to(root_dtype))
    if damping:
        M = M + damping * _identity_like(M)
    if method == "newton":
        root, iters = coupled_newton(M, int(p), max_iter, tol)
    else:  # "auto" and "eigh": eigendecomposition (reference.py:64-67)
        lam, V = torch.linalg.eigh(M)
        lam = lam.clamp_min(1e-30)
        root = V @ torch.diag_embed(lam.pow(-1.0 / p)) @ V.mT
        iters = 0
    return _sym(root).to(out_dtype), iters


def inverse_matrix_root(A, p, damping=0.0, method="auto", root_dtype=torch.float64,
                        max_iter=100, tol=1e-10):
    """(A + damping·I)^(-1/p) for symmetric PSD A, batched (reference.py:43-68)."""
    return inverse_matrix_root_with_iters(A, p, damping, method, root_dtype, max_iter, tol)[0]


def newton_schulz_orthogonalize(G, steps=5, coeffs=(3.4445, -4.7750, 2.0315), eps=1e-7):
    """Quintic Newton–Schulz polar-factor approximation (reference.py:71-97).

    Work precision is float64 for float64 input and float32 otherwise; the
    matrix is transposed so rows <= cols, Frobenius-normalised with eps added
    to the norm, iterated, transposed back and cast to the input dtype.
    """
    if G.ndim < 2:
        raise OpsArgumentError("newton_schulz_orthogonalize expects a matrix (ndim >= 2)")
    a, b, c = coeffs
    X = G.to(torch.float64 if G.dtype == torch.float64 else torch.float32)
    flip = X.shape[-2] > X.shape[-1]
    if flip:
        X = X.mT
    X = X / (torch.linalg.matrix_norm(X, ord="fro", keepdim=True) + eps)
    for _ in range(steps):
        A = X @ X.mT
        B = b * A + c * (A @ A)
        X = a * X + B @ X
    if flip:
        X = X.mT
    return X.to(G.dtype)


def kron_factor_update_(L, R, G, beta2=1.0):
    """In place: L ← β·L + (1−β)·G·Gᵀ, R ← β·R + (1−β)·Gᵀ·G (reference.py:100-114)."""
    if G.ndim != 2:
        raise OpsArgumentError(f"G must be 2D, got shape {tuple(G.shape)}")
    left = G @ G.mT
    right = G.mT @ G
    if beta2 == 1.0:
        L.add_(left)
        R.add_(right)
    else:
        L.mul_(beta2).add_(left, alpha=1.0 - beta2)
        R.mul_(beta2).add_(right, alpha=1.0 - beta2)
    return L, R


def precond_apply_two_sided(L_root, G, R_root):
    """(L_root·G)·R_root (reference.py:117-121)."""
    return L_root @ G @ R_root


def adamw_step_(p, grad, exp_avg, exp_avg_sq, lr, weight_decay, betas, eps, step, return_update_sq=False):
    """One AdamW step in place, the optimizers' shared fallback
    (optim/_common.py:56-79) from the moment updates on; `step` is the
    already-incremented step count. Returns Σ update² (a 0-dim tensor) when
    asked, else None."""
    b1, b2 = betas
    exp_avg.lerp_(grad, 1 - b1)
    exp_avg_sq.mul_(b2).addcmul_(grad, grad, value=1 - b2)
    bc1, bc2 = 1 - b1 ** step, 1 - b2 ** step
    denom = (exp_avg_sq.sqrt() / bc2 ** 0.5).add_(eps)
    update = (exp_avg / bc1) / denom
    p.mul_(1 - lr * weight_decay).add_(update, alpha=-lr)
    return update.pow(2).sum() if return_update_sq else None


def muon_momentum_(buf, grad, u, momentum, nesterov=True):
    """Muon's momentum step (optim/muon.py:79-83): buf ← buf·μ + g in place,
    then the NS5 input g + μ·buf (Nesterov) or buf, written into u (a tensor
    of buf's size, e.g. one slot of a stacked batch). Returns u."""
    buf.mul_(momentum).add_(grad)
    src = grad.add(buf, alpha=momentum) if nesterov else buf
    u.copy_(src.reshape(u.shape))
    return u


def muon_update_(p, O, decay, neg_lr):
    """Muon's parameter update (optim/muon.py:87-92): p ← p·decay (when
    decay ≠ 1), p ← p + neg_lr·O; returns Σ O² (the update_rms term)."""
    if decay != 1.0:
        p.mul_(decay)
    upd = O.reshape(p.shape)
    p.add_(upd, alpha=neg_lr)
    return upd.pow(2).sum()


def shampoo_graft_(p, grad, acc, P, buf, diag_eps, momentum, decay, neg_lr):
    """Shampoo's AdaGrad graft and update (optim/shampoo.py:133-151):
    acc ← acc + g·g; ratio = ‖g/(√acc + diag_eps)‖ / (‖P‖ + 1e-30); u = P·ratio;
    with momentum buf ← buf·μ + u, u = buf; p ← p·decay (when decay ≠ 1);
    p ← p + neg_lr·u. Returns the ratio as a 0-dim tensor."""
    acc.addcmul_(grad, grad)
    target = (grad / (acc.sqrt() + diag_eps)).norm()
    ratio = target / (P.norm() + 1e-30)
    upd = (P * ratio).reshape(p.shape)
    if momentum:
        buf.mul_(momentum).add_(upd)
        upd = buf
    if decay != 1.0:
        p.mul_(decay)
    p.add_(upd, alpha=neg_lr)
    return ratio


def two_sided_product(A, X, B, transpose_a=False, transpose_b=False):
    """op(A)·X·op(B), op = identity or transpose, associated left to right.

    SOAP's rotations into and out of the Shampoo eigenbasis, Q_Lᵀ·X·Q_R and
    Q_L·X·Q_Rᵀ (optim/soap.py:123-125), and its second-moment transport
    (C_L²)ᵀ·v·(C_R²) (:103-107), exposed as an op so a compiled backend can
    serve them. precond_apply_two_sided is the case without transposes.
    """
    return (A.mT if transpose_a else A) @ X @ (B.mT if transpose_b else B)


def gram_update_(F, X, beta=0.0, alpha=1.0, append_ones=False):
    """In place: F ← β·F + α·X̃ᵀX̃ with X̃ = [X, 1] if append_ones; β = 0 overwrites.

    X is flattened to rows over all leading dims. This is the product and
    blend of the K-FAC factor statistics (curvature/kron.py:95-113), exposed
    as an op so a compiled backend can serve it.
    """
    X2 = X.reshape(-1, X.shape[-1]).to(F.dtype)
    if append_ones:
        X2 = torch.cat([X2, X2.new_ones(X2.shape[0], 1)], dim=1)
    prod = X2.mT @ X2
    if beta == 0.0:
        F.copy_(prod.mul_(alpha))
    else:
        F.mul_(beta).add_(prod, alpha=alpha)
    return F
