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
    rc = L.pto_ns5(None, None, 7, 1, 4, 4, 5, 1.0, 1.0, 1.0, 1e-7, None, 0, None)
    assert rc != 0 and b"dtype" in L.pto_last_error()
    rc = L.pto_ns5(None, None, 0, -1, 4, 4, 5, 1.0, 1.0, 1.0, 1e-7, None, 0, None)
    assert rc != 0 and b"negative" in L.pto_last_error()
    buf = ctypes.c_void_p(0x1000)
    rc = L.pto_kron_factor_update(buf, ctypes.c_void_p(0x2000), buf, 0, 4, 4, 0.9, None, 0, None)
    assert rc != 0 and b"alias" in L.pto_last_error()
    rc = L.pto_gram_update(None, 2, None, 2, 4, 4, 0, 0.0, 1.0, None, 0, None)
    assert rc != 0 and b"unsupported" in L.pto_last_error()
    # workspace too small is caught before any launch
    rc = L.pto_ns5(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000), 0, 1, 64, 64, 5, 1.0, 1.0, 1.0, 1e-7, None, 0,
                   None)
    assert rc != 0 and b"workspace" in L.pto_last_error()
