"""pytorch_opt.ops — backend-dispatched numerics for the matrix optimizers.

Backends (the same switch as the reference's pytorch_opt/ops/__init__.py:16-88):
  "reference"  pure torch (pytorch_opt.ops.reference), any device;
  "native"     the gfx950 HIP library (libpytorch_opt_hip.so) for GPU
               tensors; CPU tensors take the pure-torch maths, as the
               reference's compiled backend served CPU tensors through ATen;
  "auto"       native once loaded, reference otherwise (the default).

``load_native()`` loads the prebuilt library; like the reference it never
raises (it warns and returns False). ``PYTORCH_OPT_NATIVE=1`` at import
calls it. Op signatures and defaults are the reference's
(pytorch_opt/ops/__init__.py:58-84); ``gram_update_`` (K-FAC factor
statistics), ``two_sided_product`` (SOAP's rotations), ``adamw_step_``
(the optimizers' shared AdamW fallback) and ``inverse_matrix_root_each``
(one root per matrix of a stack, the optimizers' per-factor calls) are
additive.
"""

from __future__ import annotations

import os
import warnings

import torch

from . import reference
from .reference import OpsArgumentError

_VALID_BACKENDS = ("auto", "native", "reference")
_BACKEND = "auto"
_NATIVE = None  # pytorch_opt.ops._hip.HipBackend once loaded


def get_backend() -> str:
    return _BACKEND


def native_available() -> bool:
    return _NATIVE is not None


def set_backend(name: str) -> None:
    """Select the backend (reference: pytorch_opt/ops/__init__.py:29-35)."""
    global _BACKEND
    if name not in _VALID_BACKENDS:
        raise ValueError(f"backend must be one of {_VALID_BACKENDS}, got {name!r}")
    if name == "native" and _NATIVE is None:
        raise RuntimeError("native backend not loaded; call pytorch_opt.ops.load_native() first")
    _BACKEND = name


def load_native(verbose: bool = False) -> bool:
    """Load the HIP library. True on success; never raises (warns instead)."""
    global _NATIVE
    if _NATIVE is not None:
        return True
    try:
        from . import native_build

        _NATIVE = native_build.load(verbose=verbose)
        return True
    except Exception as exc:  # keep the package usable without the library
        warnings.warn(f"pytorch-opt: native backend unavailable ({type(exc).__name__}: {exc}); "
                      f"using reference implementations", RuntimeWarning, stacklevel=2)
        return False


def _use_native() -> bool:
    return _BACKEND == "native" or (_BACKEND == "auto" and _NATIVE is not None)


def inverse_matrix_root(A, p, damping=0.0, method="auto", root_dtype=torch.float64,
                        max_iter=100, tol=1e-10):
    if _use_native():
        return _NATIVE.inverse_matrix_root(A, int(p), float(damping), str(method),
                                           root_dtype == torch.float64, int(max_iter), float(tol))
    return reference.inverse_matrix_root(A, p, damping=damping, method=method,
                                         root_dtype=root_dtype, max_iter=max_iter, tol=tol)


def inverse_matrix_root_each(A, p, damping=0.0, method="auto", root_dtype=torch.float64, max_iter=100, tol=1e-10):
    """inverse_matrix_root of each matrix of a stack A [k, n, n] on its own,
    i.e. the k separate calls the reference's optimizers make (each with its
    own Newton stop rule), as one call: the HIP backend runs the coupled
    Newton iterations of the whole stack in one launch sequence."""
    if A.dim() != 3:
        raise OpsArgumentError(f"inverse_matrix_root_each expects [k, n, n], got {tuple(A.shape)}")
    if _use_native() and A.is_cuda and _NATIVE.newton_for(method):
        out, _ = _NATIVE.inverse_matrix_root_each(A, int(p), float(damping), root_dtype == torch.float64,
                                                  int(max_iter), float(tol))
        return out
    return torch.stack([inverse_matrix_root(a, p, damping=damping, method=method, root_dtype=root_dtype,
                                            max_iter=max_iter, tol=tol) for a in A])


def newton_schulz_orthogonalize(G, steps=5, coeffs=(3.4445, -4.7750, 2.0315), eps=1e-7):
    if _use_native():
        a, b, c = coeffs
        return _NATIVE.newton_schulz_orthogonalize(G, int(steps), float(a), float(b), float(c), float(eps))
    return reference.newton_schulz_orthogonalize(G, steps=steps, coeffs=coeffs, eps=eps)


def kron_factor_update_(L, R, G, beta2=1.0):
    if _use_native():
        _NATIVE.kron_factor_update_(L, R, G, float(beta2))
        return L, R
    return reference.kron_factor_update_(L, R, G, beta2=beta2)


def kron_factor_update_batched_(Ls, Rs, Gs, beta2=1.0):
    """kron_factor_update_ of each (L, R, G) in three same-length lists of
    same-shape tensors (additive: the optimizers' per-step factor updates as
    one call); each pair gets what a separate kron_factor_update_ gives it."""
    if _use_native():
        _NATIVE.kron_factor_update_batched_(list(Ls), list(Rs), list(Gs), float(beta2))
        return Ls, Rs
    for L, R, G in zip(Ls, Rs, Gs):
        reference.kron_factor_update_(L, R, G, beta2=beta2)
    return Ls, Rs


def precond_apply_two_sided(L_root, G, R_root):
    if _use_native():
        return _NATIVE.precond_apply_two_sided(L_root, G, R_root)
    return reference.precond_apply_two_sided(L_root, G, R_root)


def two_sided_product(A, X, B, transpose_a=False, transpose_b=False):
    """op(A)·X·op(B) with op = identity or transpose (SOAP's eigenbasis rotations)."""
    if _use_native():
        return _NATIVE.two_sided_product(A, X, B, bool(transpose_a), bool(transpose_b))
    return reference.two_sided_product(A, X, B, transpose_a=transpose_a, transpose_b=transpose_b)


def adamw_step_(p, grad, exp_avg, exp_avg_sq, lr, weight_decay, betas, eps, step, return_update_sq=False):
    """One fused AdamW step in place (the optimizers' shared fallback); `step` is
    the already-incremented count. Returns Σ update² as a 0-dim tensor if asked."""
    if _use_native():
        b1, b2 = betas
        return _NATIVE.adamw_step_(p, grad, exp_avg, exp_avg_sq, float(lr), float(weight_decay), float(b1),
                                   float(b2), float(eps), int(step), bool(return_update_sq))
    return reference.adamw_step_(p, grad, exp_avg, exp_avg_sq, lr, weight_decay, betas, eps, step,
                                 return_update_sq=return_update_sq)


def muon_momentum_(buf, grad, u, momentum, nesterov=True):
    """(additive) Muon's momentum step in one pass: buf ← buf·μ + g in place,
    the NS5 input (g + μ·buf, or buf) into u. Returns u."""
    if _use_native():
        return _NATIVE.muon_momentum_(buf, grad, u, float(momentum), bool(nesterov))
    return reference.muon_momentum_(buf, grad, u, momentum, nesterov)


def muon_update_(p, O, decay, neg_lr):
    """(additive) Muon's parameter update in one pass: p ← p·decay + neg_lr·O
    (decay applied only when ≠ 1); returns Σ O² as a 0-dim tensor."""
    if _use_native():
        return _NATIVE.muon_update_(p, O, float(decay), float(neg_lr))
    return reference.muon_update_(p, O, decay, neg_lr)


def shampoo_graft_(p, grad, acc, P, buf, diag_eps, momentum, decay, neg_lr):
    """(additive) Shampoo's AdaGrad graft and parameter update in two passes;
    returns the graft ratio as a 0-dim tensor."""
    if _use_native():
        return _NATIVE.shampoo_graft_(p, grad, acc, P, buf, float(diag_eps), float(momentum), float(decay),
                                      float(neg_lr))
    return reference.shampoo_graft_(p, grad, acc, P, buf, diag_eps, momentum, decay, neg_lr)


def gram_update_(F, X, beta=0.0, alpha=1.0, append_ones=False):
    """F ← beta·F + alpha·X̃ᵀX̃ in place, X̃ = [X, 1] if append_ones (beta=0 overwrites)."""
    if _use_native():
        _NATIVE.gram_update_(F, X, float(beta), float(alpha), bool(append_ones))
        return F
    return reference.gram_update_(F, X, beta=beta, alpha=alpha, append_ones=append_ones)


__all__ = ["get_backend", "set_backend", "native_available", "load_native", "inverse_matrix_root",
           "inverse_matrix_root_each",
           "newton_schulz_orthogonalize", "kron_factor_update_", "kron_factor_update_batched_",
           "precond_apply_two_sided",
           "two_sided_product", "gram_update_", "adamw_step_", "muon_momentum_", "muon_update_", "shampoo_graft_",
           "OpsArgumentError", "reference"]

if os.environ.get("PYTORCH_OPT_NATIVE") == "1":
    load_native()
