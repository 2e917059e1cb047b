"""Golden vectors pinning the fp32 coupled-Newton root kernels two-sided.

The oracle's coupled Newton (oracle/ops_oracle.py, the reference's
pytorch_opt/ops/reference.py:17-40) is run with its ``matmul`` hook set to
oracle/gemm_emu.c, a restatement of the order in which the library's fp32
root products sum (blocked fused multiply-add chains of 16 in the 16x16x4
MFMA's k order, added into the running sum; each symmetric product's upper
value stored at both positions). On the config-4 inputs
(tests/golden/config4_roots.py: A = Q·diag(λ)·Qᵀ, λ = 10^U(−6, 0), p = 4,
ε = 1e-6, fp32 root) this records, per size and tolerance: the iterations,
the residual ‖X⁴(A + εI) − I‖_F/√n, the per-iteration err = max|Mk − I|, and
a SHA-256 of the returned float32 root. With tol 1e-10 every run uses all
100 iterations (err stays at the fp32 floor 2^-22 from about iteration 19);
tol 1e-6 stops in the convergence phase.

    make -C oracle && python tests/golden/config4_emulated.py   (CPU, ~30 s)
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "root_config4_emulated.json")
SIZES = (256, 1024)
TOLS = (1e-10, 1e-6)
P, EPS, MAX_ITER = 4, 1e-6, 100


def root_digest(X) -> str:
    import numpy as np

    return hashlib.sha256(np.ascontiguousarray(X, dtype=np.float32).tobytes()).hexdigest()


def _paths():
    root = os.path.dirname(os.path.dirname(HERE))
    for path in (root, HERE):
        if path not in sys.path:
            sys.path.insert(0, path)


def emulated_case(n, tol, blocked=True):
    """(X, iterations, residual, errs) of the oracle with the emulated products."""
    import numpy as np

    _paths()
    from config4_roots import build_input
    from oracle import gemm_emu, ops_oracle as oo

    A = build_input(n).numpy()
    errs = []
    X, iters = oo.inverse_root(A, P, damping=EPS, method="newton", root_dtype=np.float32, max_iter=MAX_ITER, tol=tol,
                               matmul=lambda a, b: gemm_emu.sym_matmul(a, b, blocked), errors=errs)
    return X, int(iters), float(oo.root_residual(X, A, P, EPS)), errs


def main():
    out = {"p": P, "damping": EPS, "max_iter": MAX_ITER, "root_dtype": "float32", "method": "newton",
           "products": "oracle/gemm_emu.c (blocked fp32 chains, upper value mirrored)", "cases": []}
    for n in SIZES:
        for tol in TOLS:
            X, iters, resid, errs = emulated_case(n, tol)
            _paths()
            from config4_roots import build_input, checksum

            case = {"n": n, "tol": tol, "iterations": iters, "residual": resid, "sha256": root_digest(X),
                    "input_checksum": checksum(build_input(n)), "err": [float(f"{e:.9e}") for e in errs]}
            out["cases"].append(case)
            print(n, tol, iters, resid, case["sha256"][:16], flush=True)
    with open(GOLDEN, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
