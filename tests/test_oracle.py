"""Pins the numpy oracle against closed forms, the reference's own
known-answer tests (tests/test_ops_reference.py of the reference) and brute
force. Each check is chosen so a plausible slip (dropped term, wrong sign,
transposed operand, wrong index) fails; several tests plant such a slip in
the oracle and assert the check catches it."""

import numpy as np
import pytest

from oracle import ops_oracle as oo

A_, B_, C_ = oo.NS_COEFFS


def _orth(n, rng):
    q, r = np.linalg.qr(rng.standard_normal((n, n)))
    return q * np.sign(np.diag(r))


def _ns_closed_form(U, s, V, steps=5, coeffs=oo.NS_COEFFS, eps=1e-7):
    """NS acts on each singular value independently: s/(‖s‖+eps) through
    φ(x) = a x + b x³ + c x⁵, `steps` times."""
    a, b, c = coeffs
    x = s / (np.sqrt(np.sum(s * s)) + eps)
    for _ in range(steps):
        x = a * x + b * x ** 3 + c * x ** 5
    return (U * x) @ V.T


@pytest.mark.parametrize("shape", [(6, 10), (10, 6), (8, 8), (32, 48)])
def test_ns5_closed_form(shape):
    rng = np.random.default_rng(1)
    m, n = shape
    k = min(m, n)
    U = _orth(m, rng)[:, :k]
    V = _orth(n, rng)[:, :k]
    s = np.exp(rng.uniform(-3, 0, size=k))
    G = (U * s) @ V.T
    want = _ns_closed_form(U, s, V)
    got64 = oo.ns5(G.astype(np.float64))
    assert np.abs(got64 - want).max() < 1e-10
    got32 = oo.ns5(G.astype(np.float32))
    assert np.abs(got32 - want).max() < 2e-5


def test_ns5_closed_form_catches_planted_slips():
    rng = np.random.default_rng(2)
    U, V = _orth(8, rng), _orth(8, rng)
    s = np.exp(rng.uniform(-2, 0, size=8))
    G = (U * s) @ V.T
    want = _ns_closed_form(U, s, V)
    with np.errstate(over="ignore", invalid="ignore"):
        for wrong in [(A_, -B_, C_), (A_, B_, 0.0), (A_, C_, B_)]:
            assert not (np.abs(oo.ns5(G, coeffs=wrong) - want).max() < 1e-3)
    # a transposed product (X·X instead of X·Xᵀ) on a non-symmetric input
    X = G / np.linalg.norm(G)
    bad = X
    for _ in range(5):
        A = bad @ bad
        bad = A_ * bad + (B_ * A + C_ * A @ A) @ bad
    assert np.abs(bad - want).max() > 1e-3


def test_ns5_semi_orthogonal_gives_scalar_multiple():
    # the reference's tests/test_ops_reference.py:72-80
    rng = np.random.default_rng(3)
    for shape in [(8, 8), (12, 6)]:
        Q, _ = np.linalg.qr(rng.standard_normal(shape))
        O = oo.ns5(Q.astype(np.float32), steps=10)
        s = (O * Q).sum() / (Q * Q).sum()
        assert 0.3 < s < 1.6
        assert np.linalg.norm(O - s * Q) / np.linalg.norm(Q) < 1e-3


def test_ns5_band_and_polar_distance():
    # the reference's tests/test_ops_reference.py:62-69
    rng = np.random.default_rng(4)
    G = rng.standard_normal((16, 32)).astype(np.float32)
    O = oo.ns5(G)
    sv = np.linalg.svd(O.astype(np.float64), compute_uv=False)
    assert sv.min() > 0.3 and sv.max() < 1.6
    U, _, Vh = np.linalg.svd(G.astype(np.float64), full_matrices=False)
    polar = U @ Vh
    assert np.linalg.norm(O - polar) / np.linalg.norm(polar) < 0.35


def test_ns5_batched_transpose_and_zero_steps():
    rng = np.random.default_rng(5)
    G = rng.standard_normal((4, 8, 12)).astype(np.float32)
    O = oo.ns5(G)
    for i in range(4):
        np.testing.assert_allclose(O[i], oo.ns5(G[i]), atol=1e-6)
    np.testing.assert_allclose(oo.ns5(G[0].T), O[0].T, atol=1e-6)
    Z = oo.ns5(G[0], steps=0)
    np.testing.assert_allclose(Z, G[0] / (np.linalg.norm(G[0]) + 1e-7), rtol=1e-6)
    with pytest.raises(ValueError, match="ndim"):
        oo.ns5(np.ones(3, dtype=np.float32))


def test_ns5_flops():
    # 5 iterations x (2·4096²·4097 + 2·4096³) = 1.3746e12
    assert oo.ns5_flops(4096, 4096) == 10 * 4096 ** 2 * (4097 + 4096) == 1374557306880
    assert oo.ns5_flops(4096, 11008) == oo.ns5_flops(11008, 4096)


def test_kron_closed_forms():
    # the reference's tests/test_ops_reference.py:92-108
    rng = np.random.default_rng(6)
    G1, G2 = rng.standard_normal((2, 4, 7))
    L, R = np.zeros((4, 4)), np.zeros((7, 7))
    L, R = oo.kron_factor_update(L, R, G1, 1.0)
    L, R = oo.kron_factor_update(L, R, G2, 1.0)
    outer_l = sum(np.outer(G[:, k], G[:, k]) for G in (G1, G2) for k in range(7))
    outer_r = sum(np.outer(G[i, :], G[i, :]) for G in (G1, G2) for i in range(4))
    np.testing.assert_allclose(L, outer_l, atol=1e-12)
    np.testing.assert_allclose(R, outer_r, atol=1e-12)
    b = 0.9
    L, R = oo.kron_factor_update(np.zeros((4, 4)), np.zeros((7, 7)), G1, b)
    L, R = oo.kron_factor_update(L, R, G2, b)
    np.testing.assert_allclose(L, b * (1 - b) * G1 @ G1.T + (1 - b) * G2 @ G2.T, atol=1e-12)
    np.testing.assert_allclose(R, b * (1 - b) * G1.T @ G1 + (1 - b) * G2.T @ G2, atol=1e-12)
    with pytest.raises(ValueError, match="2D"):
        oo.kron_factor_update(L, R, np.ones((2, 3, 4)))


def _spd(n, seed, lo=0.5, hi=4.0):
    rng = np.random.default_rng(seed)
    Q = _orth(n, rng)
    lam = np.linspace(lo, hi, n)
    return (Q * lam) @ Q.T, Q, lam


def test_inverse_root_closed_form():
    # the reference's tests/test_ops_reference.py:16-21
    A, Q, lam = _spd(6, 1)
    for p in (1, 2, 4):
        want = (Q * lam ** (-1.0 / p)) @ Q.T
        got, _ = oo.inverse_root(A, p)
        np.testing.assert_allclose(got, want, atol=1e-10)
        got_n, iters = oo.inverse_root(A, p, method="newton")
        np.testing.assert_allclose(got_n, want, atol=1e-9)
        assert 1 <= iters < 100


def _scalar_coupled_newton(lam, p, max_iter=100, tol=1e-10):
    """The coupled Newton iteration of pytorch_opt/ops/reference.py:17-40
    written per eigenvalue: for A = diag(lam) every matrix in the loop is
    diagonal, so X, Mk and Mi are lists of scalars and max|Mk - I| is the
    largest |m - 1|. Returns (x per eigenvalue, iterations)."""
    import math

    inv_p = 1.0 / p
    z = (1.0 + p) / (2.0 * math.sqrt(math.fsum(v * v for v in lam)))
    x = [z ** inv_p] * len(lam)
    m = [z * v for v in lam]
    good, good_err, iters = x, None, 0
    for _ in range(max_iter):
        iters += 1
        mi = [(1.0 + inv_p) - inv_p * v for v in m]
        x = [a * b for a, b in zip(x, mi)]
        m = [b ** p * v for b, v in zip(mi, m)]
        err = max(abs(v - 1.0) for v in m)
        if good_err is not None and err > 1.2 * good_err:
            return good, iters
        good, good_err = x, err
        if err < tol:
            break
    return x, iters


@pytest.mark.parametrize("p", [1, 2, 3, 4, 6])
def test_coupled_newton_iteration_count_pinned_in_float64(p):
    """The oracle's stop rule and iteration count against the eigenvalue-wise
    recurrence: exact on a diagonal input, and the same count on the rotated
    one (float64, where convergence rather than rounding noise ends the
    loop)."""
    lam = np.logspace(-3, 0, 9)
    xs, n_scalar = _scalar_coupled_newton(list(lam), p)
    X, n_oracle = oo.coupled_newton(np.diag(lam), p)
    assert n_oracle == n_scalar
    np.testing.assert_allclose(np.diag(X), xs, rtol=1e-12)
    np.testing.assert_allclose(xs, lam ** (-1.0 / p), rtol=1e-9)
    Q, _ = np.linalg.qr(np.random.default_rng(p).standard_normal((9, 9)))
    Xr, n_rot = oo.coupled_newton((Q * lam) @ Q.T, p)
    assert n_rot == n_scalar
    np.testing.assert_allclose(Xr, (Q * np.asarray(xs)) @ Q.T, atol=1e-10)
    # a slower start (eigenvalues spread further) takes more iterations
    _, n_wide = _scalar_coupled_newton(list(np.logspace(-6, 0, 9)), p)
    assert n_wide > n_scalar


def _config4_input(n):
    """The ill-conditioned config-4 construction (tests/golden/config4_roots.py)
    at a small size: float32 Q·diag(λ)·Qᵀ, λ = 10^U(−6, 0)."""
    from golden.config4_roots import build_input

    return build_input(n).numpy()


def _k_split(parts):
    """Matrix product whose contraction is summed in `parts` float32 partial sums."""

    def mm(a, b):
        k = a.shape[-1]
        out = None
        for q in range(parts):
            lo, hi = q * k // parts, (q + 1) * k // parts
            t = a[..., :, lo:hi] @ b[..., lo:hi, :]
            out = t if out is None else out + t
        return out

    return mm


def test_coupled_newton_fp32_residual_moves_with_summation_order():
    """At cond ~5e5 the float32 coupled Newton never reaches tol; its returned
    iterate, and so the residual ‖X⁴(A+εI) − I‖_F/√n, is set by product
    rounding. Summing each product's contraction in two or four partial sums
    (a legal reordering) moves the oracle's own residual by far more than
    1e-3, so two float32 implementations are compared one-sided: a kernel's
    residual may not exceed the oracle's by more than 1e-3."""
    A = _config4_input(256)
    resid = {}
    for parts in (1, 2, 4):
        X, it = oo.inverse_root(A, 4, damping=1e-6, method="newton", root_dtype=np.float32, max_iter=40,
                                matmul=_k_split(parts))
        assert it == 40  # the float32 error floor sits far above tol = 1e-10
        resid[parts] = float(oo.root_residual(X, A, 4, 1e-6))
    assert abs(resid[1] - resid[2]) > 3e-3 and abs(resid[1] - resid[4]) > 3e-3, resid
    # the same iteration in float64 meets tol; its root, stored in the input's
    # float32, sits at that storage rounding (~2e-4), far below all three
    X64, it64 = oo.inverse_root(A, 4, damping=1e-6, method="newton", root_dtype=np.float64)
    assert it64 < 40 and oo.root_residual(X64, A, 4, 1e-6) < 1e-3 < min(resid.values()) / 5


def test_config4_golden_residual_reproduces():
    """The committed config-4 golden values come from this oracle on this
    input: re-run the n = 1024 case (about 5 s) and compare."""
    import json
    import os

    from golden import config4_roots as c4

    with open(c4.GOLDEN) as f:
        gold = json.load(f)
    case = gold["cases"]["1024"]
    A = c4.build_input(1024)
    np.testing.assert_allclose(c4.checksum(A), case["input_checksum"], rtol=1e-9)
    X, it = oo.inverse_root(A.numpy(), c4.P, damping=c4.EPS, method="newton", root_dtype=np.float32,
                            max_iter=c4.MAX_ITER, tol=c4.TOL)
    assert it == case["iterations"]
    assert abs(float(oo.root_residual(X, A.numpy(), c4.P, c4.EPS)) - case["residual"]) < 1e-9
    assert os.path.basename(c4.GOLDEN) == "root_config4.json"


def test_newton_matches_eigh_and_damping():
    # the reference's tests/test_ops_reference.py:24-38
    A, _, _ = _spd(8, 3)
    for p in (2, 3, 4, 5):
        got_n, _ = oo.inverse_root(A, p, damping=1e-3, method="newton")
        got_e, _ = oo.inverse_root(A, p, damping=1e-3, method="eigh")
        np.testing.assert_allclose(got_n, got_e, atol=1e-7)
    A5, _, _ = _spd(5, 4)
    d = 0.37
    np.testing.assert_allclose(oo.inverse_root(A5, 2, damping=d)[0], oo.inverse_root(A5 + d * np.eye(5), 2)[0],
                               atol=1e-10)


def test_newton_planted_slip_fails_residual():
    A, _, _ = _spd(8, 7)
    X, _ = oo.inverse_root(A, 4, method="newton")
    assert oo.root_residual(X, A, 4) < 1e-9
    assert oo.root_residual(X.T @ X, A, 4) > 1e-2  # a wrong power
    assert oo.root_residual(X, A + 0.1 * np.eye(8), 4) > 1e-3  # missing damping term


def test_batched_root_and_validation():
    # the reference's tests/test_ops_reference.py:41-58
    rng = np.random.default_rng(5)
    B = rng.standard_normal((3, 5, 5))
    A = (B @ np.swapaxes(B, -1, -2) + 0.1 * np.eye(5)).astype(np.float32)
    got, _ = oo.inverse_root(A, 4)
    assert got.dtype == np.float32 and got.shape == A.shape
    for i in range(3):
        np.testing.assert_allclose(got[i], oo.inverse_root(A[i].astype(np.float64), 4)[0], atol=1e-5)
    with pytest.raises(ValueError, match="positive integer"):
        oo.inverse_root(A, 0)
    with pytest.raises(ValueError, match="method"):
        oo.inverse_root(A, 2, method="qr")


def test_matrix_power_order_matches_numpy():
    rng = np.random.default_rng(8)
    M = rng.standard_normal((6, 6))
    for p in range(1, 9):
        np.testing.assert_allclose(oo.matrix_power(M, p), np.linalg.matrix_power(M, p), rtol=1e-10, atol=1e-10)


def test_gram_update_brute_force():
    rng = np.random.default_rng(9)
    X = rng.standard_normal((2, 5, 3)).astype(np.float64)  # rows flattened over leading dims
    rows = X.reshape(-1, 3)
    aug = np.concatenate([rows, np.ones((10, 1))], axis=1)
    want = sum(np.outer(r, r) for r in aug) / 10
    got = oo.gram_update(None, X, beta=0.0, alpha=0.1, append_ones=True, dtype=np.float64)
    np.testing.assert_allclose(got, want, atol=1e-12)
    F0 = rng.standard_normal((4, 4))
    got = oo.gram_update(F0, X, beta=0.95, alpha=0.05 / 10, append_ones=True, dtype=np.float64)
    np.testing.assert_allclose(got, 0.95 * F0 + 0.05 * want, atol=1e-12)


def test_precond_apply_brute_force():
    rng = np.random.default_rng(10)
    L, G, R = rng.standard_normal((4, 4)), rng.standard_normal((4, 7)), rng.standard_normal((7, 7))
    want = np.einsum("ij,jk,kl->il", L, G, R)
    np.testing.assert_allclose(oo.precond_apply(L, G, R), want, atol=1e-12)


def test_two_sided_product_closed_forms():
    """Orthogonal round trip, permutation/sign closed form, transposes."""
    rng = np.random.default_rng(21)
    m, n = 7, 5
    QL, QR = _orth(m, rng), _orth(n, rng)
    X = rng.standard_normal((m, n))
    rot = oo.two_sided_product(QL, X, QR, transpose_a=True)
    np.testing.assert_allclose(oo.two_sided_product(QL, rot, QR, transpose_b=True), X, atol=1e-12)
    # signed permutations: (PᵀXS)[i, j] = sign·X[perm_L[i], perm_R[j]]
    pl, pr = rng.permutation(m), rng.permutation(n)
    sl, sr = rng.choice([-1.0, 1.0], m), rng.choice([-1.0, 1.0], n)
    PL = np.zeros((m, m)); PL[pl, np.arange(m)] = sl
    PR = np.zeros((n, n)); PR[pr, np.arange(n)] = sr
    want = X[pl][:, pr] * sl[:, None] * sr[None, :]
    np.testing.assert_allclose(oo.two_sided_product(PL, X, PR, transpose_a=True), want, atol=1e-14)
    # each flag transposes exactly its own factor
    A, B = rng.standard_normal((m, m)), rng.standard_normal((n, n))
    for ta in (False, True):
        for tb in (False, True):
            got = oo.two_sided_product(A, X, B, ta, tb)
            np.testing.assert_allclose(got, (A.T if ta else A) @ X @ (B.T if tb else B), atol=1e-12)
    assert not np.allclose(oo.two_sided_product(A, X, B, True, False), oo.two_sided_product(A, X, B, False, False))


def test_adamw_oracle_matches_torch():
    import torch

    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(22)
    p0 = rng.standard_normal((6, 4)).astype(np.float32)
    for wd in (0.0, 0.1):
        pt = torch.nn.Parameter(torch.from_numpy(p0.copy()))
        opt = torch.optim.AdamW([pt], lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=wd)
        p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
        for t in range(1, 6):
            g = rng.standard_normal(p0.shape).astype(np.float32)
            pt.grad = torch.from_numpy(g.copy())
            opt.step()
            p, m, v = oopt.adamw_step(p, g, m, v, t, 1e-2, (0.9, 0.95), 1e-8, wd)
        np.testing.assert_allclose(p, pt.detach().numpy(), atol=1e-6)


def _torch_adam_path(p0, grads, lr, betas, eps):
    import torch

    pt = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.Adam([pt], lr=lr, betas=betas, eps=eps)
    for g in grads:
        pt.grad = torch.from_numpy(g.copy())
        opt.step()
    return pt.detach().numpy()


def test_soap_oracle_is_adam_for_diagonal_factors():
    """Diagonal gradients keep L and R diagonal, the eigenbases are signed
    permutations and SOAP is exactly Adam (the reference's analytic test,
    tests/test_soap.py:8-24)."""
    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(23)
    p0 = rng.standard_normal((5, 5)).astype(np.float32)
    grads = [np.diag(rng.standard_normal(5)).astype(np.float32) for _ in range(7)]
    p, st = p0.copy(), {}
    for g in grads:
        p, st = oopt.soap_matrix_step(p, g, st, lr=1e-2, betas=(0.9, 0.999), precondition_frequency=2)
    np.testing.assert_allclose(p, _torch_adam_path(p0, grads, 1e-2, (0.9, 0.999), 1e-8), atol=1e-6)


def test_soap_oracle_fixed_basis_is_rotated_adam():
    """With the basis fixed after the first refresh, SOAP is Adam run on the
    rotated gradients Q_Lᵀ·G·Q_R, rotated back: p = p0 + Q_L·z·Q_Rᵀ where z
    is Adam's displacement. A transposed rotation fails this."""
    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(24)
    m, n = 6, 4
    p0 = rng.standard_normal((m, n)).astype(np.float64)
    grads = [rng.standard_normal((m, n)) for _ in range(5)]
    p, st = p0.copy(), {}
    p, st = oopt.soap_matrix_step(p, grads[0], st, lr=1e-2, precondition_frequency=1000)
    QL, QR = st["Q_L"], st["Q_R"]
    for g in grads[1:]:
        p, st = oopt.soap_matrix_step(p, g, st, lr=1e-2, precondition_frequency=1000)
    rot = [QL.T @ g @ QR for g in grads]
    z = _torch_adam_path(np.zeros((m, n)), rot, 1e-2, (0.95, 0.95), 1e-8)
    np.testing.assert_allclose(p, p0 + QL @ z @ QR.T, atol=1e-10)
    # the planted slip (un-transposed left rotation) is caught
    bad = [QL @ g @ QR for g in grads]
    z_bad = _torch_adam_path(np.zeros((m, n)), bad, 1e-2, (0.95, 0.95), 1e-8)
    assert not np.allclose(p, p0 + QL @ z_bad @ QR.T, atol=1e-4)


def _spd_with_spectrum(lam, rng):
    V = _orth(len(lam), rng)
    return (V * lam) @ V.T, V


def test_soap_power_basis_closed_form_and_qr_property():
    """From an exact eigenbasis (columns in any order and signs), one step
    returns that basis with the columns in descending eigenvalue order and
    each sign fixed by R's positive diagonal (W = Q·diag(λ) is already
    orthogonal, so R = diag(λ) and Q_new = the sorted columns, signs as
    given). From any basis, Q_newᵀ·Q_new = I and Q_newᵀ·W is upper
    triangular with a positive diagonal, W the sorted F·Q."""
    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(41)
    lam = np.array([5.0, 0.5, 3.0, 1.0, 2.0, 0.25])
    F, V = _spd_with_spectrum(lam, rng)
    signs = np.array([1, -1, -1, 1, 1, -1])
    perm = np.array([3, 0, 5, 1, 4, 2])
    Q = (V * signs)[:, perm]
    got = oopt.soap_power_basis(F, Q)
    want_order = np.argsort(-lam)
    np.testing.assert_allclose(got, (V * signs)[:, want_order], atol=1e-12)
    Q0 = _orth(6, rng)
    Qn = oopt.soap_power_basis(F, Q0)
    np.testing.assert_allclose(Qn.T @ Qn, np.eye(6), atol=1e-12)
    W = F @ Q0
    W = W[:, np.argsort(-np.einsum("ij,ij->j", Q0, W), kind="stable")]
    R = Qn.T @ W
    np.testing.assert_allclose(np.tril(R, -1), 0, atol=1e-12)
    assert np.all(np.diag(R) > 0)


def test_soap_power_basis_converges_to_eigh():
    """Repeated steps on a fixed factor with a separated spectrum converge
    to its eigenbasis (simultaneous iteration): Q_newᵀ·F·Q_new becomes
    diagonal with numpy's eigenvalues in descending order. The planted slip
    (ascending order, so Gram-Schmidt starts from the smallest direction)
    does not converge."""
    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(42)
    n = 24
    lam = 1.6 ** -np.arange(n)
    F, _ = _spd_with_spectrum(lam, rng)
    Q = _orth(n, rng)
    for _ in range(120):
        Q = oopt.soap_power_basis(F, Q)
    D = Q.T @ F @ Q
    off = np.linalg.norm(D - np.diag(np.diag(D))) / np.linalg.norm(D)
    assert off < 1e-9, off
    np.testing.assert_allclose(np.diag(D), np.sort(np.linalg.eigvalsh(F))[::-1], rtol=1e-9)

    def ascending(F, Q):
        W = F @ Q
        Qn, R = np.linalg.qr(W[:, np.argsort(np.einsum("ij,ij->j", Q, W), kind="stable")])
        return Qn * np.where(np.diag(R) < 0, -1.0, 1.0)

    Qb = np.linalg.eigh(F)[1]  # start from the exact basis, ascending as eigh returns it
    Qb = Qb @ _orth(n, rng) * 1e-3 + Qb  # a small perturbation
    Qb = np.linalg.qr(Qb)[0]
    for _ in range(120):
        Qb = ascending(F, Qb)
    Db = Qb.T @ F @ Qb
    assert np.linalg.norm(Db - np.diag(np.diag(Db))) / np.linalg.norm(Db) > 1e-3


def test_kfac_direction_is_the_dense_kronecker_solve():
    """vec(G⁻¹·V·A⁻¹) = (A ⊗ G)⁻¹·vec(V) with column-major vec (the
    reference's orientation test, tests/test_kfac.py:9-20); the swapped
    Kronecker order (a plausible slip) does not match."""
    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(31)
    m, n = 4, 6
    V = rng.standard_normal((m, n))
    Xa, Xg = rng.standard_normal((n, 3 * n)), rng.standard_normal((m, 3 * m))
    A, G = Xa @ Xa.T / n, Xg @ Xg.T / m
    ga, gg = oopt.kfac_damping(A, G, 1e-2)
    Ad, Gd = A + ga * np.eye(n), G + gg * np.eye(m)
    vec = lambda M: M.T.reshape(-1)  # noqa: E731
    want = np.linalg.solve(np.kron(Ad, Gd), vec(V)).reshape(n, m).T
    np.testing.assert_allclose(oopt.kfac_direction(V, A, G, 1e-2), want, atol=1e-12)
    swapped = np.linalg.solve(np.kron(Gd, Ad), vec(V)).reshape(n, m).T  # factors swapped, same vec
    assert not np.allclose(swapped, want, atol=1e-6)
    # π-split: γ_A·γ_G = damping and γ_A/γ_G = mean diag A / mean diag G
    assert np.isclose(ga * gg, 1e-2) and np.isclose(ga / gg, (np.trace(A) / n) / (np.trace(G) / m))


def test_ekfac_direction_with_eigenvalue_scales_is_kfac():
    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(32)
    m, n = 5, 3
    V = rng.standard_normal((m, n))
    Xa, Xg = rng.standard_normal((n, 2 * n)), rng.standard_normal((m, 2 * m))
    A, G = Xa @ Xa.T, Xg @ Xg.T
    evA, QA = np.linalg.eigh(A)
    evG, QG = np.linalg.eigh(G)
    d, s = oopt.ekfac_direction(V, QA, QG, np.outer(evG, evA), 1.0, 0.0)
    np.testing.assert_allclose(d, np.linalg.solve(G, V) @ np.linalg.inv(A), rtol=1e-9, atol=1e-12)
    d0, s0 = oopt.ekfac_direction(V, QA, QG, None, 0.9, 1e-3)
    np.testing.assert_allclose(s0, (QG.T @ V @ QA) ** 2, atol=1e-14)


# ------------------------------------------------------- Muon / Shampoo steps

def _svd_pair(m, n, rng):
    """U (m x k), V (n x k), k = min(m, n), with orthonormal columns."""
    k = min(m, n)
    return _orth(m, rng)[:, :k], _orth(n, rng)[:, :k]


@pytest.mark.parametrize("shape", [(8, 4), (4, 8)])
def test_muon_oracle_step_closed_form(shape):
    """Two Muon steps on gradients sharing singular vectors, g_t = U·diag(a_t)·Vᵀ:
    Nesterov momentum gives u_2 = U·diag((1+μ)·a_2 + μ²·a_1)·Vᵀ, NS5 acts on its
    singular values, and the spectral lr factor is max(1, rows/cols)^½. A
    dropped μ² term, plain (non-Nesterov) momentum or an inverted aspect
    ratio each fail."""
    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(31)
    m, n = shape
    U, V = _svd_pair(m, n, rng)
    k = min(m, n)
    a1, a2 = rng.uniform(0.5, 2.0, k), rng.uniform(0.5, 2.0, k)
    g1, g2 = (U * a1) @ V.T, (U * a2) @ V.T
    mu, lr, wd = 0.9, 0.05, 0.1
    p0 = rng.standard_normal((m, n))
    p1, buf1, _ = oopt.muon_matrix_step(p0, g1, np.zeros((m, n)), lr=lr, momentum=mu, weight_decay=wd)
    p2, buf2, O2 = oopt.muon_matrix_step(p1, g2, buf1, lr=lr, momentum=mu, weight_decay=wd)
    want_O2 = _ns_closed_form(U, (1 + mu) * a2 + mu * mu * a1, V)
    np.testing.assert_allclose(O2, want_O2, atol=2e-6)
    np.testing.assert_allclose(buf2, (U * (mu * a1 + a2)) @ V.T, rtol=0, atol=1e-7)  # μ is cast to fp32
    scale = max(1.0, m / n) ** 0.5
    want_O1 = _ns_closed_form(U, (1 + mu) * a1, V)
    want_p2 = (p0 * (1 - lr * wd) - lr * scale * want_O1) * (1 - lr * wd) - lr * scale * want_O2
    np.testing.assert_allclose(p2, want_p2, atol=2e-6)
    # planted slips move O2 or p2 by far more than the tolerance
    assert np.abs(_ns_closed_form(U, (1 + mu) * a2 + mu * a1, V) - want_O2).max() > 1e-3
    assert np.abs(_ns_closed_form(U, mu * a1 + a2, V) - want_O2).max() > 1e-3
    if m != n:
        wrong = max(1.0, n / m) ** 0.5
        assert np.abs(lr * (wrong - scale) * want_O2).max() > 1e-3


@pytest.mark.parametrize("shape", [(6, 9), (9, 6)])
def test_shampoo_oracle_step_closed_form(shape):
    """First Shampoo step (refresh at step 0) on g = U·diag(s)·Vᵀ with EMA
    factors: L/bias = g·gᵀ and R/bias = gᵀ·g, so the roots are
    U·diag((s²+ε)^-¼)·Uᵀ (plus ε^-¼ on the null space) and P = L_root·g·R_root
    = U·diag(s·(s²+ε)^-½)·Vᵀ; without a graft p moves by lr·P. The AdaGrad
    graft rescales P to ‖g/(√(g²)+δ)‖. A missing bias correction or a root
    of the wrong order fails."""
    from oracle import optim_oracle as oopt

    rng = np.random.default_rng(32)
    m, n = shape
    U, V = _svd_pair(m, n, rng)
    s = rng.uniform(0.5, 2.0, min(m, n))
    g = (U * s) @ V.T
    p0 = rng.standard_normal((m, n))
    eps, lr, beta2 = 1e-6, 0.1, 0.9
    zL, zR = np.zeros((m, m)), np.zeros((n, n))
    out = oopt.shampoo_matrix_step(p0, g, zL, zR, None, None, np.zeros((m, n)), 0, 0, lr=lr, beta2=beta2,
                                   eps=eps, graft="none")
    P = (U * (s / np.sqrt(s * s + eps))) @ V.T
    np.testing.assert_allclose(out[0], p0 - lr * P, atol=1e-6)
    np.testing.assert_allclose(out[1], (1 - beta2) * g @ g.T, atol=1e-12)
    # no bias correction: the roots see (1-β)·g·gᵀ and P grows by (1-β)^-½
    P_nobias = (U * (s / np.sqrt((1 - beta2) * s * s + eps))) @ V.T
    assert np.abs(P_nobias - P).max() > 1e-2
    # inverse square roots instead of 4th roots change every singular value
    assert np.abs((U * (s / (s * s + eps))) @ V.T - P).max() > 1e-2
    out_g = oopt.shampoo_matrix_step(p0, g, zL, zR, None, None, np.zeros((m, n)), 0, 0, lr=lr, beta2=beta2,
                                     eps=eps, graft="adagrad", diag_eps=1e-10)
    target = np.linalg.norm(g / (np.abs(g) + 1e-10))
    np.testing.assert_allclose(out_g[0], p0 - lr * P * (target / np.linalg.norm(P)), atol=1e-6)
