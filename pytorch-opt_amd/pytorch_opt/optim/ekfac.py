"""EKFAC (George et al.): K-FAC's Kronecker eigenbasis with a rescaled diagonal.

Same behaviour as the reference's pytorch_opt/optim/ekfac.py: every
``inv_every`` steps the float64 eigenbases Q_A, Q_G of the factors (and their
eigenvalues, for the condition diagnostics) are refreshed (:27-42); each
step the rotated gradient Vt = Q_Gᵀ·V·Q_A updates per-entry second moments
s (initialised to Vt², then an EMA with ``scale_decay``) and the direction
is Q_G·(Vt / (s + damping))·Q_Aᵀ (:44-58). With s fixed to the outer
product of the factor eigenvalues and no damping this is K-FAC.

The two rotations are ops.two_sided_product calls (MFMA kernels on a GPU);
the refresh eighs of same-shape factors share one batched call.
"""

from __future__ import annotations

import torch

from .. import ops
from .kfac import KFAC, batched_eigh


class EKFAC(KFAC):
    def __init__(self, model, *args, scale_decay: float = 0.95, **kwargs):
        if kwargs.get("inverse_method", "eigh") != "eigh":
            raise ValueError("EKFAC preconditions in the factors' eigenbases: inverse_method must be 'eigh'")
        self._scales: dict[str, torch.Tensor] = {}
        self._scale_decay = scale_decay
        super().__init__(model, *args, **kwargs)

    def _refresh_inverses(self):
        lam = self.param_groups[0]["damping"]
        names = list(self.tracker.factors)
        facs = [self.tracker.factors[n] for n in names]
        eig = batched_eigh([F for f in facs for F in (f["A"], f["G"])])
        conds = []
        for i, (name, f) in enumerate(zip(names, facs)):
            (evA, QA), (evG, QG) = eig[2 * i], eig[2 * i + 1]
            dt = f["A"].dtype
            cA = float((evA.max() + lam) / max(float(evA.min()) + lam, 1e-300))
            cG = float((evG.max() + lam) / max(float(evG.min()) + lam, 1e-300))
            self._inv[name] = {"QA": QA.to(dt), "QG": QG.to(dt), "evA": evA.to(dt), "evG": evG.to(dt),
                               "cond_A": cA, "cond_G": cG}
            conds.append((cA, cG))
        return conds

    def _precondition(self, name: str, V: torch.Tensor) -> torch.Tensor:
        inv = self._inv.get(name)
        if inv is None:
            raise RuntimeError(f"Missing EKFAC inverse for {name!r}")
        dtype = V.dtype
        V = V.to(inv["QG"].dtype)
        lam = self.param_groups[0]["damping"]
        Vt = ops.two_sided_product(inv["QG"], V, inv["QA"], transpose_a=True)
        s = self._scales.get(name)
        if s is None:
            s = Vt.pow(2).detach().clone()
            self._scales[name] = s
        else:
            s.mul_(self._scale_decay).add_(Vt.pow(2), alpha=1 - self._scale_decay)
        return ops.two_sided_product(inv["QG"], Vt / (s + lam), inv["QA"], transpose_b=True).to(dtype)

    def state_dict(self):
        sd = super().state_dict()
        sd["ekfac"] = {"scales": dict(self._scales), "scale_decay": self._scale_decay}
        return sd

    def load_state_dict(self, sd):
        sd = dict(sd)
        extra = sd.pop("ekfac", None)
        super().load_state_dict(sd)
        if extra is not None:
            self._scale_decay = extra.get("scale_decay", self._scale_decay)
            restored = self._restore_curvature({n: {"scale": v} for n, v in extra["scales"].items()})
            self._scales = {n: d["scale"] for n, d in restored.items()}
