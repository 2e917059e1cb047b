"""The C-ABI library loads and exports every symbol include/pytorch_opt_hip.h
declares; host-only entry points behave (no GPU work is issued here)."""

import ctypes
import os
import re

import pytest

from pytorch_opt.ops import _hip, native_build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pytorch_opt_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pto_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    path = native_build.library_path()
    assert os.path.exists(path), f"build the library first: {path}"
    return ctypes.CDLL(path)


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 16
    for name in names:
        assert hasattr(lib, name), name


def test_adapter_signatures_cover_header():
    assert set(_declared()) == set(_hip.SIGNATURES)


def test_version_and_workspace_queries(lib):
    be = _hip.HipBackend(native_build.library_path())
    L = be._lib
    assert L.pto_version() >= 10000
    ws_small = L.pto_ns5_workspace_bytes(2, 1, 512, 256)
    ws_big = L.pto_ns5_workspace_bytes(2, 32, 4096, 11008)
    assert 0 < ws_small < ws_big
    # bf16 NS5 workspace: A, B (m²) + two X buffers (m·n) per matrix
    assert ws_big >= 32 * 2 * (2 * 4096 * 4096 + 2 * 4096 * 11008)
    # fp32 keeps X and a pair of stored Xᵀ
    assert L.pto_ns5_workspace_bytes(0, 32, 4096, 11008) >= 32 * 4 * (2 * 4096 * 4096 + 3 * 4096 * 11008)
    assert L.pto_ns5_workspace_bytes(9, 1, 8, 8) == 0  # unknown dtype
    assert L.pto_kron_workspace_bytes(0, 4096, 4096) >= 4096 * 4096 * 4
    assert L.pto_inverse_root_workspace_bytes(1, 1, 1024, 100) > 10 * 1024 * 1024 * 8
    assert L.pto_gram_workspace_bytes(2, 16384, 4096, 1) >= 4097 * 16384 * 2
    assert L.pto_precond_apply_workspace_bytes(0, 8, 8) > 0


def test_host_side_argument_errors(lib):
    be = _hip.HipBackend(native_build.library_path())
    L = be._lib
    # pointers below are never dereferenced: every call fails its host checks
    a, b, w = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000), ctypes.c_void_p(0x3000)
    rc = L.pto_ns5(a, b, 7, 1, 4, 4, 5, 1.0, 1.0, 1.0, 1e-7, w, 0, None)
    assert rc != 0 and b"dtype" in L.pto_last_error()
    rc = L.pto_ns5(None, None, 0, -1, 4, 4, 5, 1.0, 1.0, 1.0, 1e-7, None, 0, None)
    assert rc != 0 and b"negative" in L.pto_last_error()
    rc = L.pto_kron_factor_update(a, b, a, 0, 4, 4, 0.9, w, 0, None)
    assert rc != 0 and b"alias" in L.pto_last_error()
    rc = L.pto_gram_update(a, 2, b, 2, 4, 4, 0, 0.0, 1.0, w, 0, None)
    assert rc != 0 and b"unsupported" in L.pto_last_error()


def test_host_side_null_pointers(lib):
    """A null operand, output or workspace of a non-empty call is an error,
    not a launch; empty calls accept nulls."""
    L = _hip.HipBackend(native_build.library_path())._lib
    a, b, w = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000), ctypes.c_void_p(0x3000)
    calls = [
        lambda: L.pto_ns5(None, b, 0, 1, 4, 4, 5, 1.0, 1.0, 1.0, 1e-7, w, 1 << 20, None),
        lambda: L.pto_ns5(a, b, 0, 1, 4, 4, 5, 1.0, 1.0, 1.0, 1e-7, None, 1 << 20, None),
        lambda: L.pto_kron_factor_update(None, a, b, 0, 4, 4, 0.9, w, 1 << 20, None),
        lambda: L.pto_gram_update(None, 0, a, 0, 4, 4, 0, 0.0, 1.0, w, 1 << 20, None),
        lambda: L.pto_inverse_root(None, b, 0, 0, 1, 4, 4, 0.0, 10, 1e-6, w, 1 << 20, None, None),
        lambda: L.pto_precond_apply(a, None, a, b, 0, 4, 4, w, 1 << 20, None),
        lambda: L.pto_two_sided_product(a, a, None, b, 0, 4, 4, 1, 0, w, 1 << 20, None),
        lambda: L.pto_two_sided_product_batched(a, a, a, None, 0, 2, 4, 4, 16, 16, 16, 0, 0, w, 1 << 20, None),
    ]
    for i, call in enumerate(calls):
        assert call() != 0 and b"null" in L.pto_last_error(), i
    assert L.pto_ns5(None, None, 0, 0, 4, 4, 5, 1.0, 1.0, 1.0, 1e-7, None, 0, None) == 0
    assert L.pto_kron_factor_update(None, None, a, 0, 0, 4, 0.9, None, 0, None) == 0
    # workspace too small is caught before any launch
    rc = L.pto_ns5(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000), 0, 1, 64, 64, 5, 1.0, 1.0, 1.0, 1e-7, None, 0,
                   None)
    assert rc != 0 and b"workspace" in L.pto_last_error()
