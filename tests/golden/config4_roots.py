"""Inverse 4th roots of ill-conditioned SPD matrices (coupled Newton, fp32).

Input builder shared by the golden-vector script below and the GPU test:
A = Q·diag(λ)·Qᵀ with Q from the QR of a seeded float64 Gaussian matrix
(torch.Generator seed 4) and λ = 10^U(−6, 0) (seed 5), cast to float32.
The root is (A + 1e-6·I)^(−1/4) by method "newton" in float32 with
max_iter 100 and tol 1e-10, judged by ‖X⁴(A + εI) − I‖_F / √n in float64.

Run as a script (CPU only, about two minutes) to rewrite
``root_config4.json`` from the oracle:

    python tests/golden/config4_roots.py
"""

from __future__ import annotations

import json
import os
import sys
import time

SIZES = (1024, 2048, 4096)
P, EPS, MAX_ITER, TOL = 4, 1e-6, 100, 1e-10
HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "root_config4.json")


def build_input(n):
    """float32 torch tensor [n, n] on the CPU."""
    import torch

    g = torch.Generator().manual_seed(4)
    Q, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    g5 = torch.Generator().manual_seed(5)
    lam = 10 ** (-6 * torch.rand(n, generator=g5, dtype=torch.float64))
    return ((Q * lam) @ Q.T).float()


def checksum(A):
    """Two float64 moments that identify the input (entry sum, squared sum)."""
    import torch

    Ad = A.double()
    return [float(Ad.sum()), float((Ad * Ad).sum())]


def main():
    import numpy as np

    root = os.path.dirname(os.path.dirname(HERE))
    if root not in sys.path:
        sys.path.insert(0, root)
    from oracle import ops_oracle as oo

    out = {"p": P, "damping": EPS, "max_iter": MAX_ITER, "tol": TOL, "root_dtype": "float32",
           "method": "newton", "cases": {}}
    for n in SIZES:
        A = build_input(n)
        t0 = time.perf_counter()
        X, iters = oo.inverse_root(A.numpy(), P, damping=EPS, method="newton", root_dtype=np.float32,
                                   max_iter=MAX_ITER, tol=TOL)
        secs = time.perf_counter() - t0
        resid = float(oo.root_residual(X, A.numpy(), P, EPS))
        out["cases"][str(n)] = {"residual": resid, "iterations": int(iters), "input_checksum": checksum(A),
                                "oracle_seconds": round(secs, 1)}
        print(n, out["cases"][str(n)], flush=True)
    with open(GOLDEN, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
