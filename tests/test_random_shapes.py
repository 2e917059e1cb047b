"""Seeded random shapes through every op, HIP path vs the CPU oracle.

Sizes up to ~520 per side (the oracle finishes in seconds) with ragged
extents, batch dims, transposed (non-contiguous) inputs, every dtype an op
accepts and each flag, so the launchers' tile choice, the masked edge
tiles, the padded workspaces and the layout transforms are exercised on
shapes no fixed-size test names. Tolerances are the op contracts': bf16
NS5 relative Frobenius 2e-2, fp32 products 1e-5 to 2e-4 (independent fp32
roundings of the same sums), fp64 1e-9 or tighter.
"""

import random

import numpy as np
import pytest
import torch

from oracle import ops_oracle as oo
from pytorch_opt import ops

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _np(t):
    t = t.detach()
    return (t.float() if t.dtype == torch.bfloat16 else t).cpu().numpy()


def _relfro(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))


@pytest.mark.parametrize("seed", [0, 1, 2, 36, 37])
def test_ns5_random_shapes(native_backend, seed):
    rng = random.Random(seed)
    for _ in range(12):
        dtype = rng.choice([torch.float32, torch.bfloat16, torch.float64])
        batch, m, n = rng.choice([(), (2,), (3,)]), rng.randint(1, 520), rng.randint(1, 520)
        steps = rng.choice([0, 1, 5])
        g = torch.Generator().manual_seed(rng.randint(0, 10**6))
        G = torch.randn(*batch, m, n, generator=g, dtype=torch.float64)
        if rng.random() < 0.3:
            G = G * 1e-3
        Gd = G.to(dtype).to(DEV)
        if rng.random() < 0.3:  # a transposed view: non-contiguous input
            Gd = Gd.transpose(-1, -2).contiguous().transpose(-1, -2)
        case = (dtype, batch, m, n, steps)
        got = ops.newton_schulz_orthogonalize(Gd, steps=steps)
        assert got.dtype == dtype and got.shape == Gd.shape, case
        work = np.float64 if dtype == torch.float64 else np.float32
        want = oo.ns5(_np(Gd).astype(work), steps=steps)
        tol = {torch.float64: 1e-9, torch.float32: 2e-4, torch.bfloat16: 2e-2}[dtype]
        if dtype == torch.bfloat16 and min(m, n) < 128:
            tol = 5e-3  # the fp32 chain, rounded once
        err = _relfro(_np(got), want)
        assert err < tol, (case, err)


@pytest.mark.parametrize("seed", [0, 1])
def test_kron_and_gram_random_shapes(native_backend, seed):
    rng = random.Random(100 + seed)
    for _ in range(8):
        dtype = rng.choice([torch.float32, torch.float64])
        m, n, beta = rng.randint(1, 400), rng.randint(1, 400), rng.choice([1.0, 0.95])
        g = torch.Generator().manual_seed(rng.randint(0, 10**6))
        G = torch.randn(m, n, generator=g, dtype=dtype)
        L0, R0 = torch.randn(m, m, generator=g, dtype=dtype), torch.randn(n, n, generator=g, dtype=dtype)
        L0, R0 = L0 + L0.T, R0 + R0.T
        L, R = L0.to(DEV), R0.to(DEV)
        ops.kron_factor_update_(L, R, G.to(DEV), beta2=beta)
        wl, wr = oo.kron_factor_update(L0.double().numpy(), R0.double().numpy(), G.double().numpy(), beta)
        tol = 1e-5 if dtype == torch.float32 else 1e-12
        case = (dtype, m, n, beta)
        assert _relfro(_np(L), wl) < tol and _relfro(_np(R), wr) < tol, case
    for _ in range(8):
        dtype = rng.choice([torch.float32, torch.bfloat16])
        rows, d, ones = rng.randint(1, 700), rng.randint(1, 400), rng.random() < 0.4
        beta, alpha = rng.choice([0.0, 0.95]), rng.choice([1.0, 0.01])
        g = torch.Generator().manual_seed(rng.randint(0, 10**6))
        X = torch.randn(rows, d, generator=g).to(dtype)
        k = d + int(ones)
        F0 = torch.randn(k, k, generator=g)
        F0 = F0 + F0.T
        F = F0.to(DEV)
        ops.gram_update_(F, X.to(DEV), beta=beta, alpha=alpha, append_ones=ones)
        want = oo.gram_update(F0.double().numpy(), _np(X).astype(np.float64), beta, alpha, ones, dtype=np.float64)
        assert _relfro(_np(F), want) < 2e-6, (dtype, rows, d, ones, beta, alpha)


@pytest.mark.parametrize("seed", [0, 1])
def test_two_sided_random_shapes(native_backend, seed):
    rng = random.Random(200 + seed)
    for _ in range(10):
        dtype = rng.choice([torch.float32, torch.float64, torch.bfloat16])
        m, n = rng.randint(1, 300), rng.randint(1, 300)
        ta, tb, lead = rng.random() < 0.5, rng.random() < 0.5, rng.choice([(), (2,), (3,)])
        g = torch.Generator().manual_seed(rng.randint(0, 10**6))
        A = torch.randn(*lead, m, m, generator=g).to(dtype)
        B = torch.randn(n, n, generator=g).to(dtype)  # shared across the batch (stride 0)
        X = torch.randn(*lead, m, n, generator=g).to(dtype)
        case = (dtype, m, n, ta, tb, lead)
        tol = {torch.float64: 1e-12, torch.float32: 2e-6, torch.bfloat16: 2e-2}[dtype]
        got = ops.two_sided_product(A.to(DEV), X.to(DEV), B.to(DEV), transpose_a=ta, transpose_b=tb)
        want = oo.two_sided_product(_np(A).astype(np.float64), _np(X).astype(np.float64),
                                    _np(B).astype(np.float64), ta, tb)
        assert got.dtype == dtype and _relfro(_np(got), want) < tol, case
        got = ops.precond_apply_two_sided(A.to(DEV), X.to(DEV), B.to(DEV))
        want = oo.precond_apply(_np(A).astype(np.float64), _np(X).astype(np.float64), _np(B).astype(np.float64))
        assert _relfro(_np(got), want) < tol, case


@pytest.mark.parametrize("seed", [0, 1])
def test_inverse_root_random_shapes(native_backend, seed):
    """Well-conditioned SPD stacks (eigenvalues in [1e-2, 1]) where the
    coupled Newton converges in both precisions: fp64 vs the oracle's own
    iterate, fp32 by residual."""
    rng = random.Random(300 + seed)
    for _ in range(6):
        n, p, batch = rng.randint(1, 160), rng.choice([1, 2, 3, 4]), rng.choice([(), (3,)])
        g = torch.Generator().manual_seed(rng.randint(0, 10**6))
        Q, _ = torch.linalg.qr(torch.randn(*batch, n, n, generator=g, dtype=torch.float64))
        lam = 10 ** (-2 * torch.rand(*batch, n, generator=g, dtype=torch.float64))
        A = (Q * lam.unsqueeze(-2)) @ Q.transpose(-1, -2)
        case = (n, p, batch)
        got = ops.inverse_matrix_root(A.to(DEV), p, damping=1e-3, method="newton", root_dtype=torch.float64)
        want, _ = oo.inverse_root(A.numpy(), p, damping=1e-3, method="newton", root_dtype=np.float64)
        assert _relfro(_np(got), want) < 1e-9, case
        got32 = ops.inverse_matrix_root(A.float().to(DEV), p, damping=1e-3, method="newton",
                                        root_dtype=torch.float32)
        res = oo.root_residual(_np(got32), A.numpy(), p, damping=1e-3)
        assert float(np.max(res)) < 1e-3, case
