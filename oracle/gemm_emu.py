"""Python side of oracle/gemm_emu.c — TEST INFRASTRUCTURE ONLY.

``sym_matmul(P, Q)`` is P·Q for symmetric Q with the summation order and
mirrored storage of the library's fp32 root products (blocked fused
multiply-add chains of 16, added into the running sum; the value for
(min(i,j), max(i,j)) stored at both positions), for use as the ``matmul``
hook of ops_oracle.coupled_newton / inverse_root. The shared library is
built by ``make -C oracle`` (done by __graft_entry__.build()).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def library():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libgemm_emu.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built: make -C oracle")
        lib = ctypes.CDLL(path)
        lib.emu_sym_product_f32.restype = ctypes.c_int
        lib.emu_sym_product_f32.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_int]
        _LIB = lib
    return _LIB


def sym_matmul(P, Q, blocked=True):
    """P·Q (float32, [..., n, n], Q symmetric) in the root kernels' order
    (blocked=False: one plain sequential FMA chain over k instead)."""
    P = np.ascontiguousarray(P, dtype=np.float32)
    Q = np.ascontiguousarray(np.broadcast_to(Q, P.shape), dtype=np.float32)
    n = P.shape[-1]
    out = np.empty(P.shape, dtype=np.float32)
    lib = library()
    for idx in np.ndindex(*P.shape[:-2]):
        p, q, o = P[idx], Q[idx], out[idx]
        rc = lib.emu_sym_product_f32(p.ctypes.data, q.ctypes.data, o.ctypes.data, n, int(bool(blocked)))
        if rc != 0:
            raise ValueError(f"gemm_emu: n = {n} must be a positive multiple of 16")
    return out
