"""The fp32 coupled-Newton root kernels pinned two-sided: on the config-4
inputs (A = Q·diag(λ)·Qᵀ, cond ~1e6, p = 4, ε = 1e-6) the kernels return,
bit for bit, the root the oracle's coupled Newton (the reference's
iteration, pytorch_opt/ops/reference.py:17-40) computes when its products
sum in the kernels' order (oracle/gemm_emu.c), after the same number of
iterations, both for a run that uses all 100 iterations (tol 1e-10, below
the fp32 floor) and for one that stops at tol 1e-6.

The fixture tests/golden/root_config4_emulated.json is written by
tests/golden/config4_emulated.py. On the CPU: the fixture reproduces at
n = 256, and a plain sequential product order (a planted difference)
does not. On the GPU: the kernels' roots against the fixture (SHA-256 of
the float32 root, iterations, and the residual within 1e-3, the contract's
bar), beside the one-sided check against the plain oracle's residual."""

import hashlib
import json
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import config4_emulated as gen  # noqa: E402
from config4_roots import build_input, checksum  # noqa: E402

from oracle import ops_oracle as oo  # noqa: E402

with open(os.path.join(HERE, "golden", "root_config4_emulated.json")) as _f:
    GOLDEN = json.load(_f)
with open(os.path.join(HERE, "golden", "root_config4.json")) as _f:
    PLAIN = json.load(_f)["cases"]

_emu_built = os.path.exists(os.path.join(os.path.dirname(HERE), "oracle", "libgemm_emu.so"))


def _ids(c):
    return f"n{c['n']}-tol{c['tol']:g}"


@pytest.mark.skipif(not _emu_built, reason="oracle/libgemm_emu.so not built (make -C oracle)")
@pytest.mark.parametrize("case", [c for c in GOLDEN["cases"] if c["n"] == 256], ids=_ids)
def test_fixture_reproduces_and_order_matters(case):
    X, iters, resid, errs = gen.emulated_case(case["n"], case["tol"])
    assert iters == case["iterations"] and gen.root_digest(X) == case["sha256"]
    assert errs == pytest.approx(case["err"], rel=1e-8, abs=0)
    # the plain sequential chain over k rounds differently: another root
    Xp, _, _, _ = gen.emulated_case(case["n"], case["tol"], blocked=False)
    assert gen.root_digest(Xp) != case["sha256"]


def test_fixture_trajectories():
    """Every recorded run falls to the fp32 floor 2^-22 and stays there; the
    tol 1e-6 runs stop at the first err below 1e-6, the tol 1e-10 ones use
    all 100 iterations; equal prefixes for the two tolerances of a size."""
    floor = 2.0 ** -22
    by_n = {}
    for c in GOLDEN["cases"]:
        e = c["err"]
        assert len(e) == c["iterations"]
        if c["tol"] == 1e-6:
            assert e[-1] < 1e-6 and all(x >= 1e-6 for x in e[:-1])
        else:
            assert c["iterations"] == 100 and e[-1] == pytest.approx(floor, rel=1e-6)
        by_n.setdefault(c["n"], []).append(e)
    for n, (a, b) in by_n.items():
        k = min(len(a), len(b))
        assert a[:k] == b[:k], n


@pytest.mark.gpu
@pytest.mark.parametrize("case", GOLDEN["cases"], ids=_ids)
def test_kernel_root_equals_emulated_oracle(hip, case):
    n = case["n"]
    A = build_input(n)
    assert checksum(A) == pytest.approx(case["input_checksum"], rel=1e-12)
    X, iters = hip.inverse_matrix_root_iters(A.to("cuda"), GOLDEN["p"], GOLDEN["damping"], "newton", False,
                                             GOLDEN["max_iter"], case["tol"])
    Xn = X.cpu().numpy()
    resid = float(oo.root_residual(Xn, A.numpy(), GOLDEN["p"], GOLDEN["damping"]))
    assert iters == case["iterations"]
    assert abs(resid - case["residual"]) <= 1e-3
    assert hashlib.sha256(np.ascontiguousarray(Xn).tobytes()).hexdigest() == case["sha256"], (
        "the root kernels no longer sum their products in the emulated order")
    plain = PLAIN.get(str(n))
    if plain is not None:  # one-sided against numpy's own float32 products
        assert resid <= plain["residual"] + 1e-3
