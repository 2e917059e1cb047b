"""KronTracker factors routed through ops.gram_update_: the reference's
hand-computed factors, EMA vs running mean, Conv2d 1x1 == Linear and the
autocast precision tests (tests/test_kron_tracker.py:9-53,142-147 of the
reference), on CPU and, on a GPU box, through the HIP Gram kernel."""

import pytest
import torch
from torch import nn

from pytorch_opt import KronTracker, ops


@pytest.fixture(autouse=True)
def _backend(device):
    if device.type == "cuda":
        assert ops.load_native(), "libpytorch_opt_hip.so failed to load"
        ops.set_backend("native")
    yield
    ops.set_backend("auto")


def mse_half(pred, target):
    return 0.5 * (pred - target).pow(2).sum() / pred.shape[0]


def test_linear_factors_hand_computed(device):
    torch.manual_seed(1)
    lin = nn.Linear(3, 2).to(device)
    X = torch.randn(4, 3, device=device)
    y = torch.randn(4, 2, device=device)
    tr = KronTracker(lin)
    with tr.track():
        out = lin(X)
        mse_half(out, y).backward()
    a_aug = torch.cat([X, X.new_ones(4, 1)], dim=1)
    ghat = out.detach() - y  # B · dL/dout for mse_half
    assert torch.allclose(tr.factors[""]["A"], a_aug.T @ a_aug / 4, atol=1e-6)
    assert torch.allclose(tr.factors[""]["G"], ghat.T @ ghat / 4, atol=1e-6)


def _one_pass(lin, X, y, tr):
    with tr.track():
        return torch.autograd.grad(mse_half(lin(X), y), list(lin.parameters()))


def test_ema_vs_running_mean(device):
    torch.manual_seed(2)
    lin = nn.Linear(3, 2, bias=False).to(device)
    X1, y1 = torch.randn(4, 3, device=device), torch.randn(4, 2, device=device)
    X2, y2 = torch.randn(4, 3, device=device), torch.randn(4, 2, device=device)
    ema = KronTracker(lin, ema_decay=0.9)
    _one_pass(lin, X1, y1, ema)
    _one_pass(lin, X2, y2, ema)
    assert torch.allclose(ema.factors[""]["A"], 0.9 * X1.T @ X1 / 4 + 0.1 * X2.T @ X2 / 4, atol=1e-6)
    ema.remove()
    rm = KronTracker(lin, ema_decay=None)
    _one_pass(lin, X1, y1, rm)
    _one_pass(lin, X2, y2, rm)
    assert torch.allclose(rm.factors[""]["A"], 0.5 * (X1.T @ X1 / 4 + X2.T @ X2 / 4), atol=1e-6)


def test_conv_1x1_output_equals_linear(device):
    torch.manual_seed(3)
    conv = nn.Conv2d(2, 5, kernel_size=4).to(device)
    lin = nn.Linear(32, 5).to(device)
    with torch.no_grad():
        lin.weight.copy_(conv.weight.reshape(5, -1))
        lin.bias.copy_(conv.bias)
    X = torch.randn(3, 2, 4, 4, device=device)
    y = torch.randn(3, 5, device=device)
    tc, tl = KronTracker(conv), KronTracker(lin)
    with tc.track():
        torch.autograd.grad(mse_half(conv(X).reshape(3, 5), y), list(conv.parameters()))
    with tl.track():
        torch.autograd.grad(mse_half(lin(X.reshape(3, -1)), y), list(lin.parameters()))
    assert torch.allclose(tc.factors[""]["A"], tl.factors[""]["A"], atol=1e-5)
    assert torch.allclose(tc.factors[""]["G"], tl.factors[""]["G"], atol=1e-5)


def test_grad_scale_divides_out(device):
    torch.manual_seed(4)
    lin = nn.Linear(6, 3).to(device)
    X, y = torch.randn(8, 6, device=device), torch.randn(8, 3, device=device)
    t1, t2 = KronTracker(lin), KronTracker(lin)
    t2.set_grad_scale(64.0)
    with t1.track():
        torch.autograd.grad(mse_half(lin(X), y), list(lin.parameters()))
    t1.remove()
    with t2.track():
        torch.autograd.grad(64.0 * mse_half(lin(X), y), list(lin.parameters()))
    assert torch.allclose(t1.factors[""]["G"], t2.factors[""]["G"], rtol=1e-5, atol=1e-7)
    with pytest.raises(ValueError, match="positive and finite"):
        t2.set_grad_scale(0.0)


def test_bf16_activations_keep_fp32_factors(device):
    torch.manual_seed(5)
    lin = nn.Linear(16, 8).to(device)
    X = torch.randn(32, 16, device=device)
    tr = KronTracker(lin)
    with tr.track():
        with torch.autocast(device_type=device.type, dtype=torch.bfloat16):
            out = lin(X.bfloat16() if device.type == "cuda" else X)
            loss = out.float().pow(2).mean()
        loss.backward()
    A = tr.factors[""]["A"]
    assert A.dtype == torch.float32
    Xa = torch.cat([X, X.new_ones(32, 1)], 1)
    Xa = Xa.bfloat16().float() if device.type == "cuda" else Xa
    assert torch.allclose(A, Xa.T @ Xa / 32, atol=1e-5)
