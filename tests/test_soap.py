"""SOAP: the reference's tests/test_soap.py identities (Adam when the factors
stay diagonal, 1-D parameters are Adam, rotations change the path,
convergence) on CPU and, on a GPU box, through the HIP kernels; plus
teacher-forced steps against the numpy oracle across basis refreshes."""

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


def test_equals_adam_when_factors_diagonal(device):
    torch.manual_seed(0)
    p_soap = nn.Parameter(torch.randn(5, 5, device=device))
    p_adam = nn.Parameter(p_soap.detach().clone())
    lr, betas, eps = 1e-2, (0.9, 0.999), 1e-8
    soap = SOAP([p_soap], lr=lr, betas=betas, eps=eps, precondition_frequency=2)
    adam = torch.optim.Adam([p_adam], lr=lr, betas=betas, eps=eps)
    for t in range(7):
        g = torch.diag(torch.randn(5, device=device))
        p_soap.grad = g.clone()
        p_adam.grad = g.clone()
        soap.step()
        adam.step()
        assert torch.allclose(p_soap.detach(), p_adam.detach(), atol=1e-6), t


def test_1d_params_are_exactly_adam(device):
    torch.manual_seed(1)
    p_soap = nn.Parameter(torch.randn(9, device=device))
    p_adam = nn.Parameter(p_soap.detach().clone())
    soap = SOAP([p_soap], adamw_lr=3e-3, adamw_betas=(0.95, 0.95))
    adam = torch.optim.Adam([p_adam], lr=3e-3, betas=(0.95, 0.95), eps=1e-8)
    for _ in range(5):
        g = torch.randn(9, device=device)
        p_soap.grad = g.clone()
        p_adam.grad = g.clone()
        soap.step()
        adam.step()
    assert torch.allclose(p_soap.detach(), p_adam.detach(), atol=1e-6)


def test_rotation_actually_used(device):
    torch.manual_seed(2)
    p_soap = nn.Parameter(torch.randn(4, 4, device=device))
    p_adam = nn.Parameter(p_soap.detach().clone())
    soap = SOAP([p_soap], lr=1e-2, precondition_frequency=1)
    adam = torch.optim.Adam([p_adam], lr=1e-2, betas=(0.95, 0.95), eps=1e-8)
    for _ in range(6):
        g = torch.randn(4, 4, device=device)
        p_soap.grad = g.clone()
        p_adam.grad = g.clone()
        soap.step()
        adam.step()
    assert not torch.allclose(p_soap.detach(), p_adam.detach(), atol=1e-4)


def test_converges_small_regression(device):
    torch.manual_seed(0)
    X = torch.randn(256, 8, device=device)
    W_true = torch.randn(8, 4, device=device)
    y = torch.tanh(X @ W_true)
    model = nn.Sequential(nn.Linear(8, 16), nn.Tanh(), nn.Linear(16, 4)).to(device)
    opt = SOAP(model.parameters(), lr=1e-2, precondition_frequency=5)
    losses = []
    for _ in range(200):
        opt.zero_grad()
        loss = 0.5 * (model(X) - y).pow(2).mean()
        loss.backward()
        opt.step()
        losses.append(float(loss.detach()))
    assert losses[-1] < 0.15 * losses[0], (losses[0], losses[-1])
    assert opt.diagnostics["n_adamw_params"] == 2 and opt.diagnostics["stale_steps"] <= 4


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


def test_oversized_matrix_raises(device):
    with pytest.raises(ValueError, match="max_preconditioner_dim"):
        SOAP([nn.Parameter(torch.randn(2048, 8, device=device))])
