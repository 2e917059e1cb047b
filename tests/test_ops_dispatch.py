"""The backend switch contract of the reference's pytorch_opt/ops/__init__.py
(tests/test_ops_dispatch.py and the load/skip behaviour of
tests/test_ops_native_parity.py in the reference)."""

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


def test_default_backend():
    assert ops.get_backend() == "auto"


def test_auto_without_native_matches_reference(device):
    ops._NATIVE = None
    A = torch.randn(5, 5, device=device)
    A = A @ A.T + 0.1 * torch.eye(5, device=device)
    assert torch.allclose(ops.inverse_matrix_root(A, 4), ops_ref.inverse_matrix_root(A, 4))
    G = torch.randn(4, 6, device=device)
    assert torch.allclose(ops.newton_schulz_orthogonalize(G), ops_ref.newton_schulz_orthogonalize(G))


def test_reference_backend_explicit():
    ops.set_backend("reference")
    assert ops.get_backend() == "reference"


def test_unknown_backend_rejected():
    with pytest.raises(ValueError, match="backend"):
        ops.set_backend("bogus")


def test_native_requires_load():
    ops._NATIVE = None
    with pytest.raises(RuntimeError, match="native backend not loaded"):
        ops.set_backend("native")


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
