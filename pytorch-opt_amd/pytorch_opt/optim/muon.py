"""Muon: Nesterov momentum orthogonalised by Newton–Schulz.

Same behaviour as the reference's pytorch_opt/optim/muon.py: constructor
and legacy ``use_muon`` handling (:22-44), state layout (:47-49), the
spectral / RMS-matching learning-rate scale (:52-58) and the step (:60-102):
per routed parameter buf = μ·buf + g, u = g + μ·buf (Nesterov) or buf,
O = NS5(u reshaped to (rows, -1)), p ← p·(1 − lr·wd) − lr·scale·O;
everything else takes the shared AdamW fallback.

Unlike the reference, which orthogonalises one parameter per call, the
routed parameters of a group are bucketed by (2-D shape, dtype, device)
and each bucket is orthogonalised by one batched NS5 launch (up to
``ns_batch_bytes`` of stacked input per launch). NS5 treats every matrix
of a batch independently, so the parameters end where the per-parameter
loop would put them; the batched launch fills the GPU where one 2048²
matrix cannot. The momentum step writes each parameter's NS5 input
straight into its slot of the stacked batch (``ops.muon_momentum_``, one
pass) and the update applies decay, step and the Σ update² term in one
pass (``ops.muon_update_``); the reference's torch ops for both run the
same arithmetic in five and three passes. The ``update_rms`` diagnostic is
summed in the reference's parameter order from per-parameter sums read
back with one host synchronisation per step instead of one per parameter.
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

    # Stacked NS5 input per batched launch, in bytes; 0 orthogonalises each
    # parameter on its own, as the reference does.
    ns_batch_bytes = 4 << 30

    def _orthogonalize_bucket(self, group, shape2, items, contrib):
        """Momentum into the stacked NS5 input, NS5, then each parameter's update."""
        limit = self.ns_batch_bytes
        mu, nesterov = group["momentum"], group["nesterov"]
        decay = 1.0 - group["lr"] * group["weight_decay"] if group["weight_decay"] else 1.0
        start = 0
        while start < len(items):
            end = start + 1
            per = items[start][0].numel() * items[start][0].element_size()
            while end < len(items) and (end - start + 1) * per <= limit:
                end += 1
            chunk = items[start:end]
            p0 = chunk[0][0]
            U = torch.empty((len(chunk),) + shape2, dtype=p0.dtype, device=p0.device)
            for i, (p, g, buf, _) in enumerate(chunk):
                ops.muon_momentum_(buf, g, U[i], mu, nesterov)
            if len(chunk) == 1:
                outs = [ops.newton_schulz_orthogonalize(U[0], steps=group["ns_steps"])]
            else:
                outs = ops.newton_schulz_orthogonalize(U, steps=group["ns_steps"]).unbind(0)
            for (p, _, _, slot), O in zip(chunk, outs):
                lr_eff = group["lr"] * self._scale(O.shape, group["lr_adjust"])
                contrib[slot] = (ops.muon_update_(p, O, decay, -lr_eff), lr_eff, p.numel())
            start = end

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        n_muon = n_adamw = 0
        contrib = []  # per parameter, in order: (sum of upd², lr_eff, numel)
        with StepTimer() as timer:
            for group in self.param_groups:
                buckets = {}
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
                        # the NS5 input is u reshaped to (rows, -1)
                        shape2 = tuple(p.shape) if p.ndim == 2 else (p.shape[0], p.numel() // max(p.shape[0], 1))
                        buckets.setdefault((shape2, p.dtype, p.device), []).append((p, g, buf, len(contrib)))
                        contrib.append(None)
                    else:
                        n_adamw += 1
                        sq, lr_eff = adamw_update(p, g, st, group, want_update_sq=True)
                        contrib.append((sq, lr_eff, p.numel()))
                for (shape2, _, _), items in buckets.items():
                    self._orthogonalize_bucket(group, shape2, items, contrib)
            sq_sum, count = 0.0, 0
            if contrib:
                by_kind = {}
                for i, (s, _, _) in enumerate(contrib):
                    by_kind.setdefault((s.device, s.dtype), []).append(i)
                host = [0.0] * len(contrib)
                for idx in by_kind.values():
                    vals = torch.stack([contrib[i][0] for i in idx]).cpu().tolist()
                    for i, v in zip(idx, vals):
                        host[i] = v
                for v, (_, lr_eff, n) in zip(host, contrib):
                    sq_sum += v * lr_eff * lr_eff
                    count += n
        self._diag = {"update_rms": (sq_sum / max(count, 1)) ** 0.5, "n_muon_params": n_muon,
                      "n_adamw_params": n_adamw, "step_ms": timer.ms}
        return loss

    def load_state_dict(self, state_dict):
        validate_checkpoint_groups(self.param_groups, state_dict["param_groups"])
        return super().load_state_dict(state_dict)
