"""SOAP against closed forms, on CPU and, with a GPU, through the HIP
kernels (factor updates, eigenbasis rotations, second-moment transport):

* gradients supported on one permutation pattern keep both factors
  diagonal, their eigenbases are signed permutations, and elementwise Adam
  commutes with those: SOAP is Adam;
* with a single basis refresh (at step 0) SOAP is AdamW run on the rotated
  gradients Q_Lᵀ·G·Q_R and rotated back;
* vectors take the AdamW fallback (vs the numpy oracle);
* teacher-forced steps against the numpy oracle across refreshes, and a
  small regression that converges;
* the opt-in power refresh (basis_refresh="power"): eigh until the second
  refresh, bit for bit; teacher-forced bases and steps against the oracle's
  Householder restatement; convergence to the eigenbasis of a fixed factor;
  shifted CholeskyQR3 on a matrix of condition number 1e10; the eigh
  fallback where a CholeskyQR fails; stacked refreshes of mixed shapes.
"""

import numpy as np
import pytest
import torch
from torch import nn

from oracle import optim_oracle as oopt
from pytorch_opt import SOAP, ops


@pytest.fixture(autouse=True)
def _backend(device):
    if device.type == "cuda":
        assert ops.load_native(), "libpytorch_opt_hip.so failed to load"
        ops.set_backend("native")
    yield
    ops.set_backend("auto")


def _permutation_gradients(rows, cols, steps, seed, device):
    """Gradients whose nonzeros sit on one fixed partial permutation: every
    row and column has at most one entry, so G·Gᵀ and Gᵀ·G are diagonal."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(cols, generator=g)[:rows]
    mask = torch.zeros(rows, cols)
    mask[torch.arange(rows), perm] = 1.0
    return [(mask * torch.randn(rows, cols, generator=g)).to(device) for _ in range(steps)]


def test_permutation_supported_gradients_reduce_to_adam(device):
    p0 = torch.randn(6, 9, generator=torch.Generator().manual_seed(1))
    p_soap = nn.Parameter(p0.clone().to(device))
    p_adam = nn.Parameter(p0.clone().to(device))
    kw = dict(lr=2e-2, betas=(0.9, 0.99), eps=1e-8)
    soap = SOAP([p_soap], precondition_frequency=3, **kw)
    adam = torch.optim.Adam([p_adam], **kw)
    for t, grad in enumerate(_permutation_gradients(6, 9, 8, 2, device)):
        p_soap.grad, p_adam.grad = grad.clone(), grad.clone()
        soap.step()
        adam.step()
        torch.testing.assert_close(p_soap.detach(), p_adam.detach(), rtol=0, atol=2e-6, msg=f"step {t}")


def test_one_refresh_is_adamw_in_the_rotated_basis(device):
    """precondition_frequency beyond the run: the basis from step 0 stays, so
    from then on SOAP(p) = Q_L·AdamW(Q_Lᵀ·p·Q_R on rotated gradients)·Q_Rᵀ
    (the decoupled decay is a scalar, rotation-invariant). AdamW starts from
    SOAP's state after step 0 (rotated parameters and first moment, SOAP's
    second moment, step 1): step 0 itself is not a fair comparison, since
    its basis diagonalises g0, whose rotated off-diagonal entries are
    rounding noise that m/(√v + ε) lifts to O(1)."""
    gen = torch.Generator().manual_seed(3)
    p0 = (0.1 * torch.randn(16, 24, generator=gen)).to(device)
    grads = [torch.randn(16, 24, generator=gen).to(device) for _ in range(6)]
    kw = dict(lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    p = nn.Parameter(p0.clone())
    soap = SOAP([p], precondition_frequency=1000, **kw)
    p.grad = grads[0]
    soap.step()
    st = soap.state[p]
    QL, QR = st["Q_L"], st["Q_R"]
    q = nn.Parameter(QL.T @ p.detach() @ QR)
    adamw = torch.optim.AdamW([q], **kw)
    adamw.state[q] = {"step": torch.tensor(1.0), "exp_avg": QL.T @ st["exp_avg"] @ QR,
                      "exp_avg_sq": st["exp_avg_sq"].clone()}
    for grad in grads[1:]:
        p.grad = grad
        soap.step()
        q.grad = QL.T @ grad @ QR
        adamw.step()
    torch.testing.assert_close(p.detach(), QL @ q.detach() @ QR.T, rtol=0, atol=2e-5)
    assert st["step"] == 6


def test_vectors_take_the_adamw_fallback(device):
    gen = torch.Generator().manual_seed(4)
    v0 = torch.randn(17, generator=gen)
    v = nn.Parameter(v0.clone().to(device))
    soap = SOAP([v], adamw_lr=3e-3, adamw_betas=(0.95, 0.95), adamw_wd=0.01)
    want, m, s = v0.numpy(), np.zeros(17, np.float32), np.zeros(17, np.float32)
    for t in range(1, 5):
        grad = torch.randn(17, generator=gen)
        v.grad = grad.to(device)
        soap.step()
        want, m, s = oopt.adamw_step(want, grad.numpy(), m, s, t, 3e-3, (0.95, 0.95), 1e-8, 0.01)
    np.testing.assert_allclose(v.detach().cpu().numpy(), want, rtol=1e-6, atol=1e-7)
    assert soap.diagnostics["n_adamw_params"] == 1


def test_non_diagonal_gradients_move_away_from_adam(device):
    gen = torch.Generator().manual_seed(5)
    p0 = torch.randn(7, 7, generator=gen)
    p_soap, p_adam = nn.Parameter(p0.clone().to(device)), nn.Parameter(p0.clone().to(device))
    soap = SOAP([p_soap], lr=1e-2, precondition_frequency=1)
    adam = torch.optim.Adam([p_adam], lr=1e-2, betas=(0.95, 0.95), eps=1e-8)
    for _ in range(5):
        grad = torch.randn(7, 7, generator=gen).to(device)
        p_soap.grad, p_adam.grad = grad.clone(), grad.clone()
        soap.step()
        adam.step()
    assert float((p_soap - p_adam).detach().norm()) > 1e-3


def test_trains_a_small_regression(device):
    gen = torch.Generator().manual_seed(6)
    X = torch.randn(320, 10, generator=gen).to(device)
    Y = torch.tanh(0.5 * X @ torch.randn(10, 3, generator=gen).to(device))
    torch.manual_seed(6)
    model = nn.Sequential(nn.Linear(10, 24), nn.Tanh(), nn.Linear(24, 3)).to(device)
    opt = SOAP(model.parameters(), lr=1e-2, precondition_frequency=4)
    first = last = None
    for _ in range(150):
        opt.zero_grad()
        loss = (model(X) - Y).pow(2).mean()
        loss.backward()
        opt.step()
        first = float(loss.detach()) if first is None else first
        last = float(loss.detach())
    assert last < 0.05 * first, (first, last)
    diag = opt.diagnostics
    assert diag["n_adamw_params"] == 2 and diag["stale_steps"] <= 3


def test_teacher_forced_vs_oracle(device):
    """Steps of a 48x80 matrix with a refresh every 2 steps (so the
    second-moment transport runs at steps 2 and 4); each step starts the
    oracle from the state the run reached.

    Step 0 is run but not compared: its refresh sees R = GᵀG of rank 48,
    whose 32 null-space eigenvectors are an arbitrary basis, and the Adam
    step m/(√v + ε) turns the rounding noise of g_rot there (both m and v
    near zero) into O(1) entries, so two correct implementations (two BLAS
    libraries for the reference itself) disagree. From step 1 the factors
    have full rank and the comparison is well posed."""
    torch.manual_seed(3)
    p = nn.Parameter(0.1 * torch.randn(48, 80, device=device))
    kw = dict(lr=1e-2, betas=(0.9, 0.95), shampoo_beta=0.9, precondition_frequency=2, weight_decay=0.05)
    opt = SOAP([p], max_preconditioner_dim=128, **kw)
    for t in range(6):
        g = torch.randn(48, 80, device=device)
        p.grad = g
        st_np = {k: (v.cpu().numpy() if torch.is_tensor(v) else v) for k, v in opt.state[p].items() if k != "stale"}
        want_p, want_st = oopt.soap_matrix_step(p.detach().cpu().numpy(), g.cpu().numpy(), st_np, **kw)
        opt.step()
        if t == 0:
            continue
        np.testing.assert_allclose(p.detach().cpu().numpy(), want_p, atol=2e-5, err_msg=f"step {t}")
        np.testing.assert_allclose(opt.state[p]["exp_avg_sq"].cpu().numpy(), want_st["exp_avg_sq"], rtol=1e-3,
                                   atol=1e-9, err_msg=f"step {t}")
    assert opt.state[p]["step"] == 6


def test_power_refresh_is_eigh_until_its_second_refresh(device):
    """basis_refresh="power" takes eigh for each factor's first basis, so a
    run equals the default's bit for bit through the steps before the
    second refresh, and departs from it there."""
    torch.manual_seed(5)
    p0 = 0.1 * torch.randn(24, 40, device=device)
    grads = [torch.randn(24, 40, device=device) for _ in range(5)]
    runs = {}
    for mode in ("eigh", "power"):
        p = nn.Parameter(p0.clone())
        opt = SOAP([p], precondition_frequency=3, basis_refresh=mode)
        runs[mode] = []
        for g in grads:
            p.grad = g.clone()
            opt.step()
            runs[mode].append(p.detach().clone())
    for t in range(3):
        assert torch.equal(runs["eigh"][t], runs["power"][t]), t
    assert not torch.equal(runs["eigh"][3], runs["power"][3])
    with pytest.raises(ValueError, match="basis_refresh"):
        SOAP([nn.Parameter(p0.clone())], basis_refresh="qr")


def test_power_refresh_teacher_forced_vs_oracle(device):
    """SOAP(basis_refresh="power") on a 36x36 matrix (both factors full
    rank from the first step), refreshing every 2 steps, against the
    oracle's power refresh (Householder QR in float64, independent of the
    CholeskyQR3 here) started from the state each step begins in: the new
    bases after each refresh and the parameters after every step from
    step 1. (Step 0's bases are the eigenvectors of G·Gᵀ and Gᵀ·G, so
    Q_Lᵀ·G·Q_R is diagonal up to rounding, and Adam's first step, the sign
    of each rotated entry, takes the sign of that rounding noise.)"""
    torch.manual_seed(6)
    p = nn.Parameter(0.1 * torch.randn(36, 36, device=device))
    kw = dict(lr=1e-2, betas=(0.9, 0.95), shampoo_beta=0.9, precondition_frequency=2)
    opt = SOAP([p], max_preconditioner_dim=128, basis_refresh="power", **kw)
    for t in range(7):
        g = torch.randn(36, 36, device=device)
        p.grad = g
        st_np = {k: (v.cpu().numpy() if torch.is_tensor(v) else v) for k, v in opt.state[p].items() if k != "stale"}
        want_p, want_st = oopt.soap_matrix_step(p.detach().cpu().numpy(), g.cpu().numpy(), st_np,
                                                basis_refresh="power", **kw)
        opt.step()
        if t % 2 == 0 and t > 0:  # power refreshes (step 0's eigh may pick other signs on a GPU)
            for k in ("Q_L", "Q_R"):
                np.testing.assert_allclose(opt.state[p][k].cpu().numpy(), want_st[k], atol=2e-4, err_msg=f"{k} {t}")
        if t > 0:
            np.testing.assert_allclose(p.detach().cpu().numpy(), want_p, atol=2e-5, err_msg=f"step {t}")


def test_power_refresh_converges_on_a_fixed_factor(device):
    """Refreshed against one fixed factor with eigenvalues 0.8^i, the
    library's bases converge to its eigenbasis: Qᵀ·F·Q diagonal to 1e-5 of
    its norm, the diagonal = the eigenvalues in descending order."""
    n = 48
    g = torch.Generator().manual_seed(7)
    V = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))[0]
    lam = 0.8 ** torch.arange(n, dtype=torch.float64)
    F = ((V * lam) @ V.T).float().to(device)
    Q = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))[0].float().to(device)
    opt = SOAP([nn.Parameter(torch.zeros(n, n, device=device))], basis_refresh="power")
    for _ in range(150):
        Q = opt._power_bases([F], [Q])[0]
    D = Q.double().T @ F.double() @ Q.double()
    d = torch.diagonal(D)
    assert float((D - torch.diag(d)).norm() / D.norm()) < 1e-5
    np.testing.assert_allclose(d.cpu().numpy(), lam.numpy(), atol=1e-6)


def test_cholqr3_on_an_ill_conditioned_matrix(device):
    """Shifted CholeskyQR3 in float64 on W of condition number 1e10 (past
    what plain CholeskyQR handles, cond² > 1/u): QᵀQ = I and W = Q·R with R
    upper triangular and a positive diagonal, R = QᵀW; its Q equals
    numpy's Householder factor with R's signs made positive on the leading
    (well-conditioned) columns."""
    rng = np.random.default_rng(8)
    m, k = 64, 40
    U = np.linalg.qr(rng.standard_normal((m, k)))[0]
    Vt = np.linalg.qr(rng.standard_normal((k, k)))[0]
    W = (U * np.logspace(0, -10, k)) @ Vt
    Q, ok = SOAP._cholqr3(torch.from_numpy(W).to(device)[None])
    assert bool(ok[0])
    Q = Q[0].cpu().numpy()
    np.testing.assert_allclose(Q.T @ Q, np.eye(k), atol=1e-12)
    R = Q.T @ W
    np.testing.assert_allclose(np.tril(R, -1), 0, atol=1e-12)
    assert np.all(np.diag(R) > 0)
    np.testing.assert_allclose(Q @ R, W, atol=1e-14)
    Qh, Rh = np.linalg.qr(W)
    Qh = Qh * np.where(np.diag(Rh) < 0, -1.0, 1.0)
    np.testing.assert_allclose(Q[:, :10], Qh[:, :10], atol=1e-9)


def test_power_refresh_falls_back_to_eigh(device, monkeypatch):
    """Where the CholeskyQR reports failure, that matrix's refresh is eigh:
    with every CholeskyQR failing, basis_refresh="power" runs exactly the
    default's steps (two parameters of different shapes, so two stacks)."""
    torch.manual_seed(9)
    shapes = [(12, 20), (16, 16)]
    p0 = [0.1 * torch.randn(s, device=device) for s in shapes]
    grads = [[torch.randn(s, device=device) for s in shapes] for _ in range(5)]

    def failing(W):
        return W, torch.zeros(W.shape[0], dtype=torch.bool, device=W.device)

    runs = {}
    for mode in ("eigh", "power"):
        ps = [nn.Parameter(x.clone()) for x in p0]
        opt = SOAP(ps, precondition_frequency=2, basis_refresh=mode)
        if mode == "power":
            monkeypatch.setattr(SOAP, "_cholqr3", staticmethod(failing))
        for gs in grads:
            for p, g in zip(ps, gs):
                p.grad = g.clone()
            opt.step()
        runs[mode] = [p.detach().clone() for p in ps]
    for a, b in zip(runs["eigh"], runs["power"]):
        assert torch.equal(a, b)


def test_power_refresh_mixed_shapes_match_single_parameter_runs(device):
    """Same-shape factors are stacked into one refresh; each parameter's
    trajectory equals a run of that parameter alone, up to the rounding of
    stacked against single GEMMs and eighs."""
    torch.manual_seed(10)
    shapes = [(12, 20), (12, 20), (20, 12)]
    p0 = [0.1 * torch.randn(s, device=device) for s in shapes]
    grads = [[torch.randn(s, device=device) for s in shapes] for _ in range(6)]
    ps = [nn.Parameter(x.clone()) for x in p0]
    opt = SOAP(ps, precondition_frequency=2, basis_refresh="power")
    for gs in grads:
        for p, g in zip(ps, gs):
            p.grad = g.clone()
        opt.step()
    for i in range(len(shapes)):
        q = nn.Parameter(p0[i].clone())
        solo = SOAP([q], precondition_frequency=2, basis_refresh="power")
        for gs in grads:
            q.grad = gs[i].clone()
            solo.step()
        torch.testing.assert_close(ps[i].detach(), q.detach(), rtol=0, atol=2e-5, msg=f"parameter {i}")


def test_oversized_matrix_raises(device):
    with pytest.raises(ValueError, match="max_preconditioner_dim"):
        SOAP([nn.Parameter(torch.randn(2048, 8, device=device))])
