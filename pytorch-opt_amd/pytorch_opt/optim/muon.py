"""Muon: Nesterov momentum orthogonalised by Newton–Schulz.

Same behaviour as the reference's pytorch_opt/optim/muon.py: constructor
and legacy ``use_muon`` handling (:22-44), state layout (:47-49), the
spectral / RMS-matching learning-rate scale (:52-58) and the step (:60-102):
per routed parameter buf = μ·buf + g, u = g + μ·buf (Nesterov) or buf,
O = NS5(u reshaped to (rows, -1)), p ← p·(1 − lr·wd) − lr·scale·O;
everything else takes the shared AdamW fallback.
"""

from __future__ import annotations

import torch
from torch.optim import Optimizer

from .. import ops
from ._common import (DiagnosticsMixin, StepTimer, adamw_update, matrix_path, validate_checkpoint_groups,
                      validate_groups)

_LR_ADJUST = ("spectral", "match_rms_adam", "none")


class Muon(Optimizer, DiagnosticsMixin):
    def __init__(self, params, lr: float = 0.02, momentum: float = 0.95, nesterov: bool = True,
                 ns_steps: int = 5, weight_decay: float = 0.0, lr_adjust: str = "spectral",
                 adamw_lr: float = 3e-4, adamw_betas: tuple = (0.9, 0.95), adamw_eps: float = 1e-8,
                 adamw_wd: float = 0.0):
        if lr_adjust not in _LR_ADJUST:
            raise ValueError(f"lr_adjust must be one of {_LR_ADJUST}, got {lr_adjust!r}")
        defaults = dict(lr=lr, momentum=momentum, nesterov=nesterov, ns_steps=ns_steps,
                        weight_decay=weight_decay, lr_adjust=lr_adjust, adamw_lr=adamw_lr,
                        adamw_betas=adamw_betas, adamw_eps=adamw_eps, adamw_wd=adamw_wd,
                        use_muon=None, use_preconditioner=None)
        super().__init__(params, defaults)
        for group in self.param_groups:
            legacy = group["use_muon"]
            if legacy is None:
                continue
            explicit = group["use_preconditioner"]
            if explicit is not None and explicit != legacy:
                raise ValueError("use_muon conflicts with use_preconditioner")
            if explicit is None and not legacy:
                # a legacy use_muon=False group keeps its adamw_* settings
                group["lr"] = group["adamw_lr"]
                group["weight_decay"] = group["adamw_wd"]
            group["use_preconditioner"] = legacy
        validate_groups(self.param_groups)

    @classmethod
    def state_layout(cls) -> dict:
        return {k: "shardable" for k in ("momentum_buffer", "exp_avg", "exp_avg_sq", "step")}

    @staticmethod
    def _scale(shape, lr_adjust: str) -> float:
        rows, cols = shape[-2], shape[-1]
        if lr_adjust == "spectral":
            return max(1.0, rows / cols) ** 0.5
        if lr_adjust == "match_rms_adam":
            return 0.2 * max(rows, cols) ** 0.5
        return 1.0

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        n_muon = n_adamw = 0
        sq_sum = 0.0
        count = 0
        with StepTimer() as timer:
            for group in self.param_groups:
                for p in group["params"]:
                    g = p.grad
                    if g is None:
                        continue
                    st = self.state[p]
                    if matrix_path(p, group):
                        n_muon += 1
                        buf = st.get("momentum_buffer")
                        if buf is None:
                            buf = st["momentum_buffer"] = torch.zeros_like(p)
                        mu = group["momentum"]
                        buf.mul_(mu).add_(g)
                        u = g.add(buf, alpha=mu) if group["nesterov"] else buf
                        u2 = u if u.ndim == 2 else u.reshape(u.shape[0], -1)
                        O = ops.newton_schulz_orthogonalize(u2, steps=group["ns_steps"])
                        lr_eff = group["lr"] * self._scale(O.shape, group["lr_adjust"])
                        if group["weight_decay"]:
                            p.mul_(1.0 - group["lr"] * group["weight_decay"])
                        upd = O.reshape(p.shape)
                        p.add_(upd, alpha=-lr_eff)
                    else:
                        n_adamw += 1
                        upd, lr_eff = adamw_update(p, g, st, group)
                    sq_sum += float(upd.pow(2).sum()) * lr_eff * lr_eff
                    count += upd.numel()
        self._diag = {"update_rms": (sq_sum / max(count, 1)) ** 0.5, "n_muon_params": n_muon,
                      "n_adamw_params": n_adamw, "step_ms": timer.ms}
        return loss

    def load_state_dict(self, state_dict):
        validate_checkpoint_groups(self.param_groups, state_dict["param_groups"])
        return super().load_state_dict(state_dict)
