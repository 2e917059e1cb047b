"""K-FAC's split of Tikhonov damping between the two Kronecker factors
(the reference's pytorch_opt/curvature/damping.py:10-26)."""

from __future__ import annotations

import math

import torch


def kfac_factored_damping(A: torch.Tensor, G: torch.Tensor, damping: float):
    """γ_A = π·√damping, γ_G = √damping / π with π = √(mean diag A / mean diag G);
    π = 1 when either mean is non-positive or not finite."""
    nu_a = float(A.diagonal(dim1=-2, dim2=-1).sum()) / A.shape[-1]
    nu_g = float(G.diagonal(dim1=-2, dim2=-1).sum()) / G.shape[-1]
    ok = math.isfinite(nu_a) and math.isfinite(nu_g) and nu_a > 0 and nu_g > 0
    pi = math.sqrt(nu_a / nu_g) if ok else 1.0
    root = math.sqrt(damping)
    return pi * root, root / pi
