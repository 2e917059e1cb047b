"""CPU oracle for the optimizer steps that drive the hot path — TEST
INFRASTRUCTURE ONLY (used by tests/ and bench.py's cpu_baseline leg).

numpy restatements of one Muon step (pytorch_opt/optim/muon.py:60-102),
the shared AdamW fallback (pytorch_opt/optim/_common.py:56-79), one
Shampoo step for a single matrix parameter
(pytorch_opt/optim/shampoo.py:70-160) and one SOAP step
(pytorch_opt/optim/soap.py:48-125), used for teacher-forced checks: given
the state a GPU run reached, the oracle computes the next state.

Pinning (tests/test_oracle.py): adamw_step against torch.optim.Adam/AdamW;
soap_matrix_step against the same Adam when the factors stay diagonal (the
eigenbases are signed permutations, SOAP's analytic identity,
tests/test_soap.py:8-24 of the reference) and against its own rotation-
free form when Q_L, Q_R are fixed arbitrary orthogonal matrices;
muon_matrix_step over two steps on gradients sharing singular vectors
(Nesterov momentum, NS5 per singular value and the aspect-ratio lr factor
in closed form); shampoo_matrix_step's first step on g = U·diag(s)·Vᵀ
(P = U·diag(s·(s²+ε)^-½)·Vᵀ, with and without the AdaGrad graft);
kfac_direction against the dense Kronecker solve; ekfac_direction with
the factors' eigenvalue products as scales against kfac_direction.
"""

from __future__ import annotations

import numpy as np

from . import ops_oracle as oo


def muon_matrix_step(p, g, buf, lr=0.02, momentum=0.95, nesterov=True, ns_steps=5, weight_decay=0.0,
                     lr_adjust="spectral"):
    """One Muon update of a routed matrix; returns (p_new, buf_new, O)."""
    buf = buf * np.float32(momentum) + g
    u = g + np.float32(momentum) * buf if nesterov else buf
    u2 = u if u.ndim == 2 else u.reshape(u.shape[0], -1)
    O = oo.ns5(u2, steps=ns_steps).astype(np.float32)
    rows, cols = O.shape[-2], O.shape[-1]
    if lr_adjust == "spectral":
        scale = max(1.0, rows / cols) ** 0.5
    elif lr_adjust == "match_rms_adam":
        scale = 0.2 * max(rows, cols) ** 0.5
    else:
        scale = 1.0
    if weight_decay:
        p = p * np.float32(1.0 - lr * weight_decay)
    p = p - np.float32(lr * scale) * O.reshape(p.shape)
    return p, buf, O


def adamw_step(p, g, m, v, t, lr, betas=(0.9, 0.95), eps=1e-8, wd=0.0):
    """One AdamW fallback step at step count t (1-based); returns (p, m, v)."""
    b1, b2 = betas
    m = m + np.float32(1 - b1) * (g - m)
    v = v * np.float32(b2) + np.float32(1 - b2) * g * g
    bc1, bc2 = 1 - b1 ** t, 1 - b2 ** t
    denom = np.sqrt(v) / np.float32(bc2 ** 0.5) + np.float32(eps)
    upd = (m / np.float32(bc1)) / denom
    p = p * np.float32(1 - lr * wd) - np.float32(lr) * upd
    return p, m, v


def shampoo_matrix_step(p, g, L, R, L_root, R_root, graft_acc, step, factor_updates, lr=0.03, beta2=0.999,
                        eps=1e-8, precondition_frequency=20, graft="adagrad", diag_eps=1e-10, root_dtype=np.float64,
                        root_method="auto", factors=None, roots=None):
    """One Shampoo update of a selected matrix (no momentum / wd / bootstrap).

    Returns the new (p, L, R, L_root, R_root, graft_acc). Teacher forcing
    per stage: ``factors`` = (L, R) after this step's update replaces the
    oracle's own factor update, ``roots`` = (L_root, R_root) this step's
    roots (on a refresh step), so each stage can start from a GPU run's
    result of the stage before.
    """
    g2 = g.reshape(g.shape[0], -1)
    L, R = oo.kron_factor_update(L, R, g2, beta2) if factors is None else factors
    factor_updates += 1
    if roots is not None and step % precondition_frequency == 0:
        L_root, R_root = roots
    elif step % precondition_frequency == 0:
        bc = 1.0 - beta2 ** factor_updates if beta2 < 1.0 else 1.0
        L_root = oo.inverse_root(L / np.float32(bc), 4, damping=eps, method=root_method, root_dtype=root_dtype)[0]
        R_root = oo.inverse_root(R / np.float32(bc), 4, damping=eps, method=root_method, root_dtype=root_dtype)[0]
    P = oo.precond_apply(L_root, g2, R_root)
    if graft == "adagrad":
        graft_acc = graft_acc + g2 * g2
        target = np.linalg.norm(g2 / (np.sqrt(graft_acc) + np.float32(diag_eps)))
        P = P * np.float32(target / (np.linalg.norm(P) + 1e-30))
    elif graft == "sgd":
        P = P * np.float32(np.linalg.norm(g2) / (np.linalg.norm(P) + 1e-30))
    p = p - np.float32(lr) * P.reshape(p.shape)
    return p, L, R, L_root, R_root, graft_acc


def soap_power_basis(F, Q):
    """One subspace-iteration step of a SOAP eigenbasis from its current
    estimate Q (the power-iteration refresh of Vyas et al., "SOAP", 2024,
    Algorithm 4; the library's SOAP(basis_refresh="power"), which has no
    counterpart in the reference): the columns of Q ordered by descending
    Rayleigh quotient diag(Qᵀ·F·Q) (ties in index order), then the
    orthonormal factor of W = F·Q whose R has a positive diagonal. Here by
    Householder QR (numpy, float64) with the signs of R's diagonal moved
    into Q; the library computes the same factor by shifted CholeskyQR3.
    Returned in F's dtype."""
    Fd, Qd = F.astype(np.float64), Q.astype(np.float64)
    W = Fd @ Qd
    order = np.argsort(-np.einsum("ij,ij->j", Qd, W), kind="stable")
    Qn, R = np.linalg.qr(W[:, order])
    return (Qn * np.where(np.diag(R) < 0, -1.0, 1.0)).astype(F.dtype)


def soap_matrix_step(p, g, state, lr=3e-3, betas=(0.95, 0.95), shampoo_beta=0.95, eps=1e-8,
                     precondition_frequency=10, weight_decay=0.0, basis_refresh="eigh"):
    """One SOAP update of a selected matrix (pytorch_opt/optim/soap.py:48-66,
    :80-125): factor EMA, eigenbasis refresh every `precondition_frequency`
    steps with the second moment transported through the squared
    basis-change matrices, then Adam in the eigenbasis.

    `state` holds L, R, exp_avg, exp_avg_sq, step and (after the first
    refresh) Q_L, Q_R, as numpy arrays; a new dict is returned with p.
    Eigenvectors come from numpy's eigh (ascending, as torch's): the update
    is unchanged by the sign of each eigenvector and the transport maps the
    second moment exactly under such flips, so the oracle need not share
    the GPU run's eigenvector signs.
    """
    st = dict(state)
    dt = p.dtype
    g2 = g.reshape(g.shape[0], -1)
    m, n = g2.shape
    if "L" not in st:
        st.update(L=np.zeros((m, m), dt), R=np.zeros((n, n), dt), exp_avg=np.zeros_like(g2),
                  exp_avg_sq=np.zeros_like(g2), step=0)
    st["L"], st["R"] = oo.kron_factor_update(st["L"], st["R"], g2, shampoo_beta)
    if st["step"] % precondition_frequency == 0:
        if basis_refresh == "power" and "Q_L" in st:
            QL = soap_power_basis(st["L"], st["Q_L"])
            QR = soap_power_basis(st["R"], st["Q_R"])
        else:
            QL = np.linalg.eigh(st["L"].astype(np.float64))[1].astype(dt)
            QR = np.linalg.eigh(st["R"].astype(np.float64))[1].astype(dt)
        if "Q_L" in st:
            CL = st["Q_L"].T @ QL
            CR = st["Q_R"].T @ QR
            st["exp_avg_sq"] = oo.two_sided_product(CL * CL, st["exp_avg_sq"], CR * CR, transpose_a=True)
        st["Q_L"], st["Q_R"] = QL, QR
    QL, QR = st["Q_L"], st["Q_R"]
    b1, b2 = betas
    st["step"] += 1
    t = st["step"]
    st["exp_avg"] = st["exp_avg"] + dt.type(1 - b1) * (g2 - st["exp_avg"])
    g_rot = oo.two_sided_product(QL, g2, QR, transpose_a=True)
    st["exp_avg_sq"] = st["exp_avg_sq"] * dt.type(b2) + dt.type(1 - b2) * g_rot * g_rot
    m_rot = oo.two_sided_product(QL, st["exp_avg"], QR, transpose_a=True)
    denom = np.sqrt(st["exp_avg_sq"]) / dt.type((1 - b2 ** t) ** 0.5) + dt.type(eps)
    upd = oo.two_sided_product(QL, m_rot / denom, QR, transpose_b=True)
    if weight_decay:
        p = p * dt.type(1.0 - lr * weight_decay)
    p = p - dt.type(lr / (1 - b1 ** t)) * upd.reshape(p.shape)
    return p, st


def kfac_damping(A, G, damping):
    """π-split of Tikhonov damping, pytorch_opt/curvature/damping.py:10-26:
    γ_A = π√λ, γ_G = √λ/π, π = √(mean diag A / mean diag G) (1 if not positive)."""
    nu_a = float(np.trace(A)) / A.shape[-1]
    nu_g = float(np.trace(G)) / G.shape[-1]
    ok = np.isfinite(nu_a) and np.isfinite(nu_g) and nu_a > 0 and nu_g > 0
    pi = float(np.sqrt(nu_a / nu_g)) if ok else 1.0
    r = float(np.sqrt(damping))
    return pi * r, r / pi


def kfac_direction(V, A, G, damping):
    """K-FAC natural gradient of one module (pytorch_opt/optim/kfac.py:130-142,
    145-154): (G + γ_G I)⁻¹·V·(A + γ_A I)⁻¹, by two linear solves in float64."""
    V, A, G = (np.asarray(x, np.float64) for x in (V, A, G))
    ga, gg = kfac_damping(A, G, damping)
    left = np.linalg.solve(G + gg * np.eye(G.shape[0]), V)
    return np.linalg.solve((A + ga * np.eye(A.shape[0])).T, left.T).T


def ekfac_direction(V, QA, QG, s_prev, scale_decay, damping):
    """EKFAC direction (pytorch_opt/optim/ekfac.py:44-58) given the previous
    scales s_prev (None on the first call): Vt = Q_Gᵀ·V·Q_A,
    s = decay·s_prev + (1 − decay)·Vt², d = Q_G·(Vt / (s + λ))·Q_Aᵀ.
    Returns (d, s)."""
    V, QA, QG = (np.asarray(x, np.float64) for x in (V, QA, QG))
    Vt = oo.two_sided_product(QG, V, QA, transpose_a=True)
    s = Vt * Vt if s_prev is None else scale_decay * np.asarray(s_prev, np.float64) + (1 - scale_decay) * Vt * Vt
    return oo.two_sided_product(QG, Vt / (s + damping), QA, transpose_b=True), s
