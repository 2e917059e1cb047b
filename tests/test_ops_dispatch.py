"""The backend switch contract of the reference's pytorch_opt/ops/__init__.py
(the behaviour its tests/test_ops_dispatch.py and the load/skip logic of
tests/test_ops_native_parity.py check): states and refusals of the switch,
the pure-torch maths when no library is loaded (against closed forms),
load failures that warn and degrade, CPU tensors under a loaded backend,
and argument errors raised as both ValueError and RuntimeError."""

import warnings

import pytest
import torch

from pytorch_opt import ops
from pytorch_opt.ops import reference as ops_ref


@pytest.fixture(autouse=True)
def _restore():
    saved = ops._NATIVE
    yield
    ops._NATIVE = saved
    ops.set_backend("auto")


def test_switch_states_and_refusals():
    """The switch starts at "auto"; "reference" and "auto" can always be
    chosen, "native" only once a library is loaded, anything else never; a
    refused switch leaves the selection as it was."""
    assert ops.get_backend() == "auto"
    ops._NATIVE = None
    ops.set_backend("reference")
    refusals = [("native", RuntimeError, "native backend not loaded"), ("cuda", ValueError, "backend must be one of"),
                ("Reference", ValueError, "backend must be one of")]
    for name, exc, message in refusals:
        with pytest.raises(exc, match=message):
            ops.set_backend(name)
        assert ops.get_backend() == "reference"
    ops.set_backend("auto")
    assert ops.get_backend() == "auto"


def _known_spectrum(n, seed, device):
    """Q·diag(λ)·Qᵀ with Q from QR of a seeded Gaussian and λ in [0.2, 3]."""
    g = torch.Generator().manual_seed(seed)
    Q, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    lam = 0.2 + 2.8 * torch.rand(n, generator=g, dtype=torch.float64)
    return Q, lam


def test_unloaded_auto_computes_closed_forms(device):
    """With no library loaded, "auto" runs the pure-torch maths on any device:
    the inverse 4th root of Q·diag(λ)·Qᵀ is Q·diag(λ^-1/4)·Qᵀ, and NS5 of a
    matrix with orthonormal singular vectors keeps them, mapping each
    normalised singular value through five quintic steps."""
    ops._NATIVE = None
    Q, lam = _known_spectrum(6, 31, device)
    A = ((Q * lam) @ Q.T).float().to(device)
    want = (Q * lam ** -0.25) @ Q.T
    assert float((ops.inverse_matrix_root(A, 4).double().cpu() - want).abs().max()) < 1e-5
    s = torch.tensor([1.7, 0.9, 0.4], dtype=torch.float64)
    U, V = Q[:, :3], _known_spectrum(5, 32, device)[0][:, :3]
    x = s / s.norm()
    for _ in range(5):
        x = 3.4445 * x - 4.7750 * x ** 3 + 2.0315 * x ** 5
    out = ops.newton_schulz_orthogonalize(((U * s) @ V.T).float().to(device))
    assert float((out.double().cpu() - (U * x) @ V.T).abs().max()) < 1e-5


def test_load_failure_warns_and_degrades(monkeypatch, tmp_path):
    ops._NATIVE = None
    monkeypatch.setenv("PYTORCH_OPT_HIP_LIB", str(tmp_path / "missing.so"))
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        assert ops.load_native() is False
    assert any(issubclass(x.category, RuntimeWarning) and "native backend unavailable" in str(x.message) for x in w)
    assert not ops.native_available()
    G = torch.randn(3, 4)
    assert torch.equal(ops.newton_schulz_orthogonalize(G), ops_ref.newton_schulz_orthogonalize(G))


def test_load_native_succeeds_with_built_library():
    ops._NATIVE = None
    assert ops.load_native() is True
    assert ops.native_available()
    assert ops.load_native() is True  # idempotent


def test_auto_prefers_native_cpu_tensor():
    # the reference's test_auto_backend_prefers_native: CPU tensor, native loaded
    assert ops.load_native()
    assert ops.get_backend() == "auto"
    g = torch.Generator().manual_seed(11)
    B = torch.randn(5, 5, generator=g)
    A = B @ B.mT + 0.1 * torch.eye(5)
    assert torch.allclose(ops.inverse_matrix_root(A, 4), ops_ref.inverse_matrix_root(A, 4), atol=1e-6)


def test_argument_errors_are_value_and_runtime_errors():
    assert ops.load_native()
    ops.set_backend("native")
    A = torch.eye(3)
    for exc in (ValueError, RuntimeError):
        with pytest.raises(exc, match="positive integer"):
            ops.inverse_matrix_root(A, 0)
        with pytest.raises(exc, match="method"):
            ops.inverse_matrix_root(A, 2, method="qr")
        with pytest.raises(exc, match="ndim"):
            ops.newton_schulz_orthogonalize(torch.ones(3))
        with pytest.raises(exc, match="2D"):
            ops.kron_factor_update_(torch.zeros(2, 2), torch.zeros(2, 2), torch.ones(2, 2, 2))
