"""Fused elementwise steps of Muon (momentum / NS5 input, decay + update +
Σ update²) and of Shampoo's AdaGrad graft with its update, through the C
ABI, against the torch op sequences they replace (the package's pure-torch
reference run on the same GPU tensors) and float64 closed forms.

The elementwise results follow torch's op-by-op rounding; the norms and
Σ update² are fixed-order float64 sums where torch sums in float32, so the
graft ratio (and what it scales) agrees to a few float32 ulps."""

import numpy as np
import pytest
import torch

from pytorch_opt import ops
from pytorch_opt.ops import reference as ops_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.float64, torch.bfloat16]


def _rand(n, seed, dtype, scale=1.0, offset=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    base = scale * torch.randn(n + offset, generator=g, device=DEV, dtype=torch.float64)
    return base.to(dtype)[offset:]


def _ulps(dtype):
    return {torch.float32: 2.0 ** -23, torch.float64: 2.0 ** -52, torch.bfloat16: 2.0 ** -7}[dtype]


def _close(a, b, ulps, dtype, scale=None):
    """|a - b| <= ulps·eps(dtype)·max(|a|, |b|, scale) elementwise, scale the
    magnitude of the operands a result was formed from (cancellation can
    leave a result far smaller than them)."""
    a64, b64 = a.double(), b.double()
    mag = torch.maximum(a64.abs(), b64.abs())
    if scale is not None:
        mag = torch.maximum(mag, scale.double())
    tol = ulps * _ulps(dtype) * mag + 1e-300
    bad = (a64 - b64).abs() > tol
    assert not bool(bad.any()), (int(bad.sum()), float((a64 - b64).abs().max()))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("nesterov", [True, False])
@pytest.mark.parametrize("n,offset", [(1, 0), (13, 0), (65536 * 3 + 5, 0), (4099, 1)])
def test_muon_momentum_matches_torch_ops(native_backend, dtype, nesterov, n, offset):
    """buf·μ + g then g + μ·buf (or buf), three steps in a row; the unaligned
    view (offset 1) takes the element-wise path. buf is bit for bit torch's
    mul_ / add_; the Nesterov input matches torch's add(alpha=μ) to an ulp."""
    buf = torch.zeros(n, dtype=dtype, device=DEV)
    buf_r = buf.clone()
    for t in range(3):
        g = _rand(n, 10 + t, dtype, offset=offset)
        u = _rand(n, 20 + t, dtype)  # stale contents must be overwritten
        u_r = torch.empty_like(u)
        ops.muon_momentum_(buf, g, u, 0.95, nesterov)
        ops_ref.muon_momentum_(buf_r, g, u_r, 0.95, nesterov)
        assert torch.equal(buf, buf_r), t
        _close(u, u_r, 1.0, dtype)
    # a matrix slot of a stacked batch, from a conv-shaped parameter
    p_shape = (8, 4, 3, 3)
    g = _rand(288, 30, dtype).reshape(p_shape)
    buf, buf_r = torch.ones(p_shape, dtype=dtype, device=DEV), torch.ones(p_shape, dtype=dtype, device=DEV)
    U = torch.zeros(3, 8, 36, dtype=dtype, device=DEV)
    ops.muon_momentum_(buf, g, U[1], 0.9, nesterov)
    want = ops_ref.muon_momentum_(buf_r, g, torch.empty(8, 36, dtype=dtype, device=DEV), 0.9, nesterov)
    _close(U[1], want, 1.0, dtype)
    assert not U[0].any() and not U[2].any()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("decay", [1.0, 1.0 - 0.02 * 0.1])
@pytest.mark.parametrize("n,offset", [(7, 0), (1 << 20, 0), (100003, 1)])
def test_muon_update_matches_torch_ops(native_backend, dtype, decay, n, offset):
    """p·decay + (−lr)·O with the fused multiply-add of torch's add_(alpha);
    Σ O² against a float64 sum."""
    p = _rand(n, 40, dtype, offset=offset)
    O = _rand(n, 41, dtype, scale=0.02)
    p_r = p.clone()
    sq = ops.muon_update_(p, O, decay, -0.02 * 1.4)
    sq_r = ops_ref.muon_update_(p_r, O, decay, -0.02 * 1.4)
    _close(p, p_r, 1.0, dtype)
    want = float((O.double() ** 2).sum())
    assert sq.dtype == torch.float64 and abs(float(sq) - want) <= 1e-12 * want
    assert abs(float(sq_r) - want) <= 1e-2 * want  # torch's own sum, for scale


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("momentum", [0.0, 0.9])
@pytest.mark.parametrize("decay", [1.0, 0.999])
@pytest.mark.parametrize("n,offset", [(5, 0), (2048 * 2048, 0), (70001, 1)])
def test_shampoo_graft_matches_torch_ops(native_backend, dtype, momentum, decay, n, offset):
    """Three steps of acc += g², ratio = ‖g/(√acc + ε)‖ / (‖P‖ + 1e-30),
    (momentum), decay, p += −lr·P·ratio, against the reference's torch ops
    on the GPU. acc matches torch's addcmul_ to an ulp; the ratio is within
    a few ulps of torch's (float64 sums here, float32 in torch) and of the
    float64 closed form; p and the momentum buffer follow it."""
    p = _rand(n, 50, dtype, offset=offset)
    acc = torch.zeros(n, dtype=dtype, device=DEV)
    buf = torch.zeros(n, dtype=dtype, device=DEV) if momentum else None
    p_r, acc_r = p.clone(), acc.clone()
    buf_r = buf.clone() if buf is not None else None
    # ulps of the ratio against torch's (float32 sums there) and of what it scales
    ulps = {torch.float32: 64.0, torch.bfloat16: 2.0, torch.float64: 1e4}[dtype]
    # p and buf evolve separately from their torch copies: a difference made
    # at one step stays at that step's magnitude, so the scales accumulate
    pscale = torch.zeros(n, dtype=torch.float64, device=DEV)
    bscale = torch.zeros(n, dtype=torch.float64, device=DEV)
    for t in range(3):
        g = _rand(n, 60 + t, dtype, scale=1e-2)
        P = _rand(n, 70 + t, dtype, scale=3.0)
        acc_before, p_before = acc.clone(), p.clone()
        buf_before = buf.clone() if buf is not None else None
        ratio = ops.shampoo_graft_(p, g, acc, P, buf, 1e-10, momentum, decay, -0.05)
        ratio_r = ops_ref.shampoo_graft_(p_r, g, acc_r, P, buf_r, 1e-10, momentum, decay, -0.05)
        _close(acc, acc_r, 1.0, dtype)
        _close(ratio.reshape(1), ratio_r.reshape(1), ulps, dtype)
        a64 = acc_before.double() + g.double() ** 2
        want = float((g.double() / (a64.sqrt() + 1e-10)).norm() / P.double().norm())
        bar = 1e-12 if dtype == torch.float64 else 8 * _ulps(dtype)
        assert abs(float(ratio) - want) <= bar * want, (t, float(ratio), want)
        # the step lr·P·ratio carries the ratio's few-ulp difference
        step = 0.05 * P.abs().double() * float(ratio_r)
        if buf is not None:
            bscale += momentum * buf_before.abs().double() + step / 0.05
            _close(buf, buf_r, ulps, dtype, scale=bscale)
            step = 0.05 * buf_r.abs().double() + 0.05 * bscale
        pscale += p_before.abs().double() + step
        _close(p, p_r, ulps, dtype, scale=pscale)


def test_fused_steps_reject_mismatched_tensors(native_backend):
    """Shapes or dtypes that do not line up take the reference's torch ops
    (which raise on a size mismatch) rather than a kernel over wrong sizes."""
    buf = torch.zeros(10, device=DEV)
    with pytest.raises(RuntimeError):
        ops.muon_momentum_(buf, torch.zeros(11, device=DEV), torch.zeros(10, device=DEV), 0.9, True)
    p = torch.zeros(10, device=DEV)
    with pytest.raises(RuntimeError):
        ops.muon_update_(p, torch.zeros(12, device=DEV), 1.0, -0.1)
    # momentum given without a buffer: the reference path raises too
    with pytest.raises((RuntimeError, AttributeError)):
        ops.shampoo_graft_(p, torch.ones(10, device=DEV), torch.zeros(10, device=DEV), torch.ones(10, device=DEV),
                           None, 1e-10, 0.9, 1.0, -0.1)


def test_shampoo_step_uses_fused_graft_and_matches_unfused(native_backend):
    """A Shampoo step with the AdaGrad graft and momentum equals, to float32
    rounding of the norms, the same step assembled from the reference's torch
    ops (direction from the same roots)."""
    from pytorch_opt import Shampoo

    torch.manual_seed(3)
    W = torch.nn.Parameter(torch.randn(64, 96, device=DEV))
    opt = Shampoo([W], lr=0.05, momentum=0.9, weight_decay=0.01, graft="adagrad", precondition_frequency=1,
                  eps=1e-3)
    for _ in range(2):
        W.grad = torch.randn(64, 96, device=DEV)
        st = opt.state[W]
        p_before = W.detach().clone()
        acc = st["graft_acc"].clone() if "graft_acc" in st else torch.zeros(64, 96, device=DEV)
        buf = st["momentum_buffer"].clone() if "momentum_buffer" in st else torch.zeros(64, 96, device=DEV)
        opt.step()
        P = ops_ref.precond_apply_two_sided(st["L_root"], W.grad, st["R_root"])
        want = p_before.clone()
        ops_ref.shampoo_graft_(want, W.grad, acc, P, buf, opt.param_groups[0]["diag_eps"], 0.9, 1 - 0.05 * 0.01,
                               -0.05)
        np.testing.assert_allclose(W.detach().cpu().numpy(), want.cpu().numpy(), rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(st["graft_acc"].cpu().numpy(), acc.cpu().numpy(), rtol=2.4e-7, atol=0)
