"""KronTracker (factor statistics through ops.gram_update_) against brute
force, on CPU and, with a GPU, through the HIP Gram kernel:

* A and G of a Linear layer equal sums of per-row outer products;
* the blend schedule over three batches (EMA weights β², β(1−β), 1−β; the
  running mean 1/3 each);
* a module called twice in one forward contributes both calls, each
  activation paired with its own output gradient;
* a padded, strided 3x3 convolution's factors equal those of its explicit
  unfolded patches;
* the loss scale divides out of G, capture gates the forward binding, and
  bf16 activations keep float32 factors.
"""

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from pytorch_opt import KronTracker, ops


@pytest.fixture(autouse=True)
def _backend(device):
    if device.type == "cuda":
        assert ops.load_native(), "libpytorch_opt_hip.so failed to load"
        ops.set_backend("native")
    yield
    ops.set_backend("auto")


def _outer_sum(rows):
    return sum(torch.outer(r, r) for r in rows)


def test_linear_factors_are_outer_product_sums(device):
    gen = torch.Generator().manual_seed(11)
    lin = nn.Linear(5, 3).double().to(device)
    X = torch.randn(7, 5, generator=gen, dtype=torch.float64).to(device)
    tr = KronTracker(lin)
    with tr.track():
        out = lin(X)
        out.retain_grad()
        (out.pow(3).sum() / 7).backward()  # a mean-reduced loss
    n = 7
    a_rows = torch.cat([X, torch.ones(n, 1, dtype=X.dtype, device=device)], 1)
    g_rows = n * out.grad  # per-example output gradients
    torch.testing.assert_close(tr.factors[""]["A"], _outer_sum(a_rows) / n, rtol=1e-12, atol=1e-14)
    torch.testing.assert_close(tr.factors[""]["G"], _outer_sum(g_rows) / n, rtol=1e-12, atol=1e-14)
    assert tr.updates("") == 1


@pytest.mark.parametrize("decay", [0.8, None])
def test_three_batch_blend(device, decay):
    gen = torch.Generator().manual_seed(47)
    lin = nn.Linear(4, 2, bias=False).to(device)
    tr = KronTracker(lin, ema_decay=decay)
    batches = [torch.randn(6, 4, generator=gen).to(device) for _ in range(3)]
    for X in batches:
        with tr.track():
            torch.autograd.grad(lin(X).square().mean(), [lin.weight])
    grams = [X.T @ X / 6 for X in batches]
    w = [decay * decay, decay * (1 - decay), 1 - decay] if decay is not None else [1 / 3] * 3
    torch.testing.assert_close(tr.factors[""]["A"], sum(wi * Gi for wi, Gi in zip(w, grams)), rtol=1e-5, atol=1e-6)
    assert tr.updates("") == 3


def test_reused_module_pairs_each_call(device):
    """x -> lin -> tanh -> lin: two calls per forward, each bound to its own
    input, so A is the running mean of the two calls' activation Grams."""
    gen = torch.Generator().manual_seed(13)
    lin = nn.Linear(6, 6, bias=False).double().to(device)
    X = torch.randn(9, 6, generator=gen, dtype=torch.float64).to(device)
    tr = KronTracker(lin, ema_decay=None)
    with tr.track():
        h = torch.tanh(lin(X))
        lin(h).sum().backward()
    want = 0.5 * (X.T @ X / 9 + h.detach().T @ h.detach() / 9)
    torch.testing.assert_close(tr.factors[""]["A"], want, rtol=1e-12, atol=1e-14)
    assert tr.updates("") == 2


def test_conv_factors_are_unfolded_patch_grams(device):
    gen = torch.Generator().manual_seed(14)
    conv = nn.Conv2d(3, 4, kernel_size=3, stride=2, padding=1).double().to(device)
    X = torch.randn(2, 3, 7, 7, generator=gen, dtype=torch.float64).to(device)
    tr = KronTracker(conv)
    with tr.track():
        out = conv(X)
        out.retain_grad()
        (out.square().sum() / 2).backward()
    B, L = 2, out.shape[-1] * out.shape[-2]
    patches = F.unfold(X, 3, padding=1, stride=2).transpose(1, 2).reshape(B * L, -1)
    a_rows = torch.cat([patches, torch.ones(B * L, 1, dtype=X.dtype, device=device)], 1)
    g_rows = B * out.grad.flatten(2).transpose(1, 2).reshape(B * L, -1)
    torch.testing.assert_close(tr.factors[""]["A"], a_rows.T @ a_rows / (B * L), rtol=1e-12, atol=1e-13)
    torch.testing.assert_close(tr.factors[""]["G"], g_rows.T @ g_rows / (B * L), rtol=1e-12, atol=1e-13)


def test_loss_scale_divides_out(device):
    gen = torch.Generator().manual_seed(15)
    lin = nn.Linear(8, 5).to(device)
    X = torch.randn(16, 8, generator=gen).to(device)
    plain, scaled = KronTracker(lin), KronTracker(lin)
    scaled.set_grad_scale(8.0)
    scaled.enabled = False
    with plain.track():
        torch.autograd.grad(lin(X).pow(2).mean(), list(lin.parameters()))
    plain.enabled = False
    with scaled.track():
        torch.autograd.grad(8.0 * lin(X).pow(2).mean(), list(lin.parameters()))
    torch.testing.assert_close(scaled.factors[""]["G"], plain.factors[""]["G"], rtol=1e-5, atol=1e-8)
    for bad in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="positive and finite"):
            scaled.set_grad_scale(bad)


def test_capture_off_binds_nothing(device):
    lin = nn.Linear(3, 3).to(device)
    tr = KronTracker(lin)
    tr.capture = False
    with tr.track():
        lin(torch.ones(2, 3, device=device)).sum().backward()
    assert tr.factors == {} and tr.updates("") == 0
    tr.remove()
    tr.capture = True
    with tr.track():  # hooks removed: still nothing
        lin(torch.ones(2, 3, device=device)).sum().backward()
    assert tr.factors == {}


def test_bf16_activations_keep_fp32_factors(device):
    """bf16 activations (an autocast region upstream) reach the hook as bf16
    rows; the factor stays float32 and equals the Gram of those values."""
    gen = torch.Generator().manual_seed(16)
    lin = nn.Linear(32, 8).to(device)
    Xb = torch.randn(64, 32, generator=gen).to(device).bfloat16()
    tr = KronTracker(lin)
    with tr.track():
        with torch.autocast(device_type=device.type, dtype=torch.bfloat16):
            loss = lin(Xb).float().square().mean()
        loss.backward()
    A = tr.factors[""]["A"]
    assert A.dtype == torch.float32
    Xa = torch.cat([Xb.float(), torch.ones(64, 1, device=device)], 1)
    torch.testing.assert_close(A, Xa.T @ Xa / 64, rtol=1e-5, atol=1e-5)
