"""EKFAC (George et al.): K-FAC's Kronecker eigenbasis with a rescaled
diagonal.

Behaviour of the reference's pytorch_opt/optim/ekfac.py: every
``inv_every`` steps the float64 eigenbases Q_A, Q_G of the factors are
refreshed (:27-42); each step the rotated gradient Vt = Q_Gᵀ·V·Q_A updates
per-entry second moments s (Vt² the first time, then an EMA with
``scale_decay``, kept across refreshes) and the direction is
Q_G·(Vt / (s + damping))·Q_Aᵀ (:44-58). With s fixed to the outer product of
the factors' eigenvalues and no damping this is K-FAC's direction.

Here both rotations are ops.two_sided_product calls (MFMA kernels on a GPU),
the refresh eighs of same-shape factors share one batched call, and the
scales live in each module's curvature entry; checkpoints carry them in the
reference's ``"ekfac": {"scales", "scale_decay"}`` entry (:60-72).
"""

from __future__ import annotations

import torch

from .. import ops
from .kfac import KFAC, batched_eigh


def _cond(ev: torch.Tensor, lam: float) -> float:
    return float(ev.max() + lam) / max(float(ev.min()) + lam, 1e-300)


class EKFAC(KFAC):
    def __init__(self, model, *args, scale_decay: float = 0.95, **kwargs):
        if kwargs.get("inverse_method", "eigh") != "eigh":
            raise ValueError("EKFAC preconditions in the factors' eigenbases: inverse_method must be 'eigh'")
        self.scale_decay = scale_decay
        super().__init__(model, *args, **kwargs)

    def _refresh_inverses(self):
        lam = self.param_groups[0]["damping"]
        names = list(self.tracker.factors)
        flat = [self.tracker.factors[n][k] for n in names for k in ("A", "G")]
        eig = batched_eigh(flat)
        conds = []
        for k, name in enumerate(names):
            (evA, QA), (evG, QG) = eig[2 * k], eig[2 * k + 1]
            dt = flat[2 * k].dtype
            entry = {"QA": QA.to(dt), "QG": QG.to(dt), "evA": evA.to(dt), "evG": evG.to(dt),
                     "cond_A": _cond(evA, lam), "cond_G": _cond(evG, lam)}
            previous = self._inv.get(name, {})
            if "scale" in previous:  # the second moments outlive the basis
                entry["scale"] = previous["scale"]
            self._inv[name] = entry
            conds.append((entry["cond_A"], entry["cond_G"]))
        return conds

    def _precondition(self, name: str, V: torch.Tensor) -> torch.Tensor:
        inv = self._inv.get(name)
        if inv is None or "QG" not in inv:  # (a restored scale alone is no basis)
            raise RuntimeError(f"Missing EKFAC inverse for {name!r}")
        QG, QA = inv["QG"], inv["QA"]
        Vt = ops.two_sided_product(QG, V.to(QG.dtype), QA, transpose_a=True)
        moment = Vt.square()
        scale = inv.get("scale")
        if scale is None:
            scale = inv["scale"] = moment
        else:
            scale.mul_(self.scale_decay).add_(moment, alpha=1.0 - self.scale_decay)
        lam = self.param_groups[0]["damping"]
        return ops.two_sided_product(QG, Vt / (scale + lam), QA, transpose_b=True).to(V.dtype)

    def state_dict(self):
        sd = super().state_dict()
        scales = {}
        for name, entry in sd["kfac"]["inv"].items():  # shallow copies of the live entries
            if "scale" in entry:
                scales[name] = entry.pop("scale")
        sd["ekfac"] = {"scales": scales, "scale_decay": self.scale_decay}
        return sd

    def load_state_dict(self, state_dict):
        sd = dict(state_dict)
        extra = sd.pop("ekfac", None)
        # an earlier version of this module kept scale_decay in the K-FAC entry
        # and each scale inside its curvature entry, which the K-FAC loader restores
        self.scale_decay = sd.get("kfac", {}).get("scale_decay", self.scale_decay)
        super().load_state_dict(sd)
        if extra is not None:
            self.scale_decay = extra.get("scale_decay", self.scale_decay)
            restored = self._on_module_device({n: {"scale": v} for n, v in extra.get("scales", {}).items()})
            for name, entry in restored.items():
                self._inv.setdefault(name, {})["scale"] = entry["scale"]
