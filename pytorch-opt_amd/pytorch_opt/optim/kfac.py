"""K-FAC natural-gradient optimizer (Martens & Grosse).

Same behaviour as the reference's pytorch_opt/optim/kfac.py: it takes the
model, installs factor hooks on its untied nn.Linear / groups=1 nn.Conv2d
modules (or on the modules an explicit ``params`` split selects), and the
other trainable parameters take the AdamW fallback (:28-105). Curvature comes
from the training backward every ``stats_every`` steps ("empirical") or from
``update_curvature(outputs)`` with sampled labels ("sampled") (:107-143).
Every ``inv_every`` steps the damped factor inverses are refreshed with π-split
damping, (F + γI)⁻¹ from a float64 eigh (:145-176); a module's weight gradient
V (out × in, bias column appended) becomes (G + γ_G I)⁻¹·V·(A + γ_A I)⁻¹,
then optional global norm clipping, momentum, weight decay and the step
(:180-263); the state dict carries the curvature (:267-306).

Here the factor statistics are ops.gram_update_ calls (through KronTracker),
the preconditioning is ops.precond_apply_two_sided — both MFMA kernels on a
GPU — and the refresh eighs of same-shape factors run as one batched call.
``inverse_method="newton"`` (an addition; the default "eigh" is the
reference's) computes the damped inverses instead with the coupled Newton
iteration of ops.inverse_matrix_root at p = 1 — the MFMA root kernels — on
the same batches, in the factors' precision, with the condition numbers of
the diagnostics estimated by power iteration.
"""

from __future__ import annotations

import torch
from torch import nn
from torch.optim import Optimizer

from .. import ops
from ..curvature.damping import kfac_factored_damping
from ..curvature.kron import KronTracker
from ._common import DiagnosticsMixin, StepTimer, adamw_update, validate_checkpoint_groups, validate_groups

_FISHER_MODES = ("empirical", "sampled")
_INVERSE_METHODS = ("eigh", "newton")


def _top_eigenvalues(M: torch.Tensor, iters: int) -> torch.Tensor:
    """Largest eigenvalue of each symmetric PSD matrix of a batch, by power
    iteration from a fixed start (a lower estimate after few steps)."""
    g = torch.Generator(device=M.device).manual_seed(0)
    v = torch.randn(M.shape[0], M.shape[-1], 1, generator=g, device=M.device, dtype=M.dtype)
    for _ in range(iters):
        v = M @ v
        v = v / v.norm(dim=1, keepdim=True).clamp_min(torch.finfo(M.dtype).tiny)
    return (v.mT @ (M @ v)).reshape(-1)


def damped_inverses_newton(mats, gammas, batch_bytes: int = 4 << 30, power_iters: int = 30):
    """(F_i + γ_i·I)⁻¹ for each factor by the coupled Newton iteration of
    ops.inverse_matrix_root with p = 1 (the MFMA root kernels on a GPU),
    same-shape factors in one ops.inverse_matrix_root_each call (each with
    its own stop rule), in the factor's precision
    (float64 factors in float64, others in float32). Also returns the
    condition number of each F_i + γ_i·I estimated as λ_max(F + γI)·λ_max
    of the inverse, both by power iteration. Returns [(inverse, cond)]."""
    out = [None] * len(mats)
    buckets = {}
    for i, F in enumerate(mats):
        buckets.setdefault((tuple(F.shape), F.device, F.dtype), []).append(i)
    for (shape, dev, dt), idx in buckets.items():
        n = shape[-1]
        rdt = torch.float64 if dt == torch.float64 else torch.float32
        # the stack and the root's workspace hold about eight n x n matrices
        # of the root precision per entry
        step = max(1, batch_bytes // (8 * n * n * (torch.finfo(rdt).bits // 8)))
        eye = torch.eye(n, device=dev, dtype=rdt)
        for s in range(0, len(idx), step):
            chunk = idx[s:s + step]
            M = torch.stack([mats[i].to(rdt) + gammas[i] * eye for i in chunk])
            inv = ops.inverse_matrix_root_each(M, 1, damping=0.0, method="newton", root_dtype=rdt,
                                               tol=1e-10 if rdt == torch.float64 else 1e-5)
            cond = (_top_eigenvalues(M, power_iters) * _top_eigenvalues(inv, power_iters)).tolist()
            for j, i in enumerate(chunk):
                out[i] = (inv[j].to(dt), cond[j])
    return out


def batched_eigh(mats, batch_bytes: int = 4 << 30):
    """float64 eigh of each matrix; same-shape matrices share one batched call.
    Returns [(eigenvalues, eigenvectors)] in float64, in input order."""
    out = [None] * len(mats)
    buckets = {}
    for i, M in enumerate(mats):
        buckets.setdefault((tuple(M.shape), M.device), []).append(i)
    for idx in buckets.values():
        step = max(1, batch_bytes // (mats[idx[0]].numel() * 8))
        for s in range(0, len(idx), step):
            chunk = idx[s:s + step]
            ev, V = torch.linalg.eigh(torch.stack([mats[i].double() for i in chunk]))
            for j, i in enumerate(chunk):
                out[i] = (ev[j], V[j])
    return out


class KFAC(Optimizer, DiagnosticsMixin):
    def __init__(self, model: nn.Module, lr: float = 0.01, damping: float = 1e-3,
                 ema_decay: float | None = 0.95, momentum: float = 0.9, stats_every: int = 1, inv_every: int = 10,
                 fisher_mode: str = "empirical", weight_decay: float = 0.0, max_grad_norm: float | None = None, *,
                 params=None, adamw_lr: float = 3e-4, adamw_betas: tuple = (0.9, 0.95), adamw_eps: float = 1e-8,
                 adamw_wd: float = 0.0, inverse_method: str = "eigh"):
        if fisher_mode not in _FISHER_MODES:
            raise ValueError(f"fisher_mode must be one of {_FISHER_MODES}, got {fisher_mode!r}")
        if stats_every < 1 or inv_every < 1:
            raise ValueError("stats_every and inv_every must be positive")
        if inverse_method not in _INVERSE_METHODS:
            raise ValueError(f"inverse_method must be one of {_INVERSE_METHODS}, got {inverse_method!r}")
        self.inverse_method = inverse_method
        self.model = model
        self.fisher_mode = fisher_mode
        owners = {}
        for module in model.modules():
            for p in module.parameters(recurse=False):
                owners[id(p)] = owners.get(id(p), 0) + 1
        supported = {name: m for name, m in model.named_modules()
                     if isinstance(m, (nn.Linear, nn.Conv2d)) and (not isinstance(m, nn.Conv2d) or m.groups == 1)
                     and m.weight.requires_grad and owners[id(m.weight)] == 1}
        if params is None:
            primary = [p for m in supported.values() for p in m.parameters(recurse=False)
                       if p.requires_grad and owners[id(p)] == 1]
            chosen = {id(p) for p in primary}
            params = [{"params": primary, "use_preconditioner": True}]
            for decay in (False, True):  # the fallback keeps the usual no-decay split
                rest = [p for p in model.parameters() if p.requires_grad and id(p) not in chosen
                        and (p.ndim >= 2 and not getattr(p, "_no_weight_decay", False)) == decay]
                if rest:
                    params.append(dict(params=rest, use_preconditioner=False, lr=adamw_lr,
                                       weight_decay=adamw_wd if decay else 0.0))
        else:
            params = list(params)
            if any(not isinstance(g, dict) or not isinstance(g.get("use_preconditioner"), bool) for g in params):
                raise ValueError("KFAC params must be groups with explicit use_preconditioner")
        # curvature settings live in the first preconditioned group
        params = sorted(params, key=lambda g: not g["use_preconditioner"])
        defaults = dict(lr=lr, damping=damping, momentum=momentum, stats_every=stats_every, inv_every=inv_every,
                        weight_decay=weight_decay, max_grad_norm=max_grad_norm, adamw_lr=adamw_lr,
                        adamw_betas=adamw_betas, adamw_eps=adamw_eps, adamw_wd=adamw_wd)
        super().__init__(params, defaults)
        validate_groups(self.param_groups, matrices=False)
        trainable = {id(p) for p in model.parameters() if p.requires_grad}
        assigned = {id(p) for g in self.param_groups for p in g["params"]}
        if assigned != trainable:
            raise ValueError("KFAC groups must cover every trainable model parameter exactly once")
        selected = {id(p) for g in self.param_groups if g["use_preconditioner"] for p in g["params"]}
        self._name_to_module = {n: m for n, m in supported.items() if id(m.weight) in selected}
        bias_modules = {n for n, m in self._name_to_module.items()
                        if m.bias is not None and id(m.bias) in selected and owners[id(m.bias)] == 1}
        covered = {id(m.weight) for m in self._name_to_module.values()}
        covered.update(id(self._name_to_module[n].bias) for n in bias_modules)
        if covered != selected:
            raise ValueError("KFAC selection must contain supported, untied module weights and optional biases")
        self.tracker = KronTracker(model, ema_decay=ema_decay, module_names=self._name_to_module,
                                   bias_modules=bias_modules)
        self._steps = 0
        self._inv: dict[str, dict] = {}
        self._last_counts = {}
        self._inv_stale = 0
        self._sync_tracking()

    def _sync_tracking(self) -> None:
        collect = self._steps % self.param_groups[0]["stats_every"] == 0
        self.tracker.capture = collect
        self.tracker.enabled = self.fisher_mode == "empirical" and collect

    def set_grad_scale(self, scale: float) -> None:
        """Set before backward: 1 / accumulation steps, or AMP scale / steps.
        Corrects the curvature only; unscale parameter gradients as usual."""
        self.tracker.set_grad_scale(scale)

    @classmethod
    def state_layout(cls) -> dict:
        layout = {k: "replicable" for k in ("A", "G", "iA", "iG", "steps", "inv_stale")}
        layout.update({k: "shardable" for k in ("momentum_buffer", "step", "exp_avg", "exp_avg_sq")})
        return layout

    # ------------------------------------------------------------- curvature
    def update_curvature(self, outputs: torch.Tensor, kind: str = "categorical",
                         generator: torch.Generator | None = None) -> None:
        if self.fisher_mode != "sampled":
            raise RuntimeError("update_curvature() is only used with fisher_mode='sampled'; "
                               "empirical mode accumulates from the training backward")
        if self._steps % self.param_groups[0]["stats_every"] != 0:
            return
        self.tracker.sampled_backward(outputs, kind=kind, generator=generator)

    @staticmethod
    def _damped_inverse_from(ev, V, gamma, dtype):
        """(F + γI)⁻¹ = V·diag(1/(λ + γ))·Vᵀ and cond(F + γI), from F's float64 eigh."""
        inv = ((V * (1.0 / (ev + gamma))) @ V.T).to(dtype)
        cond = float((ev.max() + gamma) / max(float(ev.min()) + gamma, 1e-300))
        return inv, cond

    @classmethod
    def _damped_inverse(cls, F: torch.Tensor, gamma: float):
        ev, V = torch.linalg.eigh(F.double())
        return cls._damped_inverse_from(ev, V, gamma, F.dtype)

    def _precondition(self, name: str, V: torch.Tensor) -> torch.Tensor:
        """(G + γ_G I)⁻¹·V·(A + γ_A I)⁻¹ for one module (EKFAC overrides)."""
        inv = self._inv.get(name)
        if inv is None:
            raise RuntimeError(f"Missing K-FAC inverse for {name!r}")
        with torch.autocast(device_type=V.device.type, enabled=False):
            return ops.precond_apply_two_sided(inv["iG"], V.to(inv["iG"].dtype), inv["iA"]).to(V.dtype)

    def _refresh_inverses(self) -> list[tuple[float, float]]:
        g = self.param_groups[0]
        names = list(self.tracker.factors)
        facs = [self.tracker.factors[n] for n in names]
        gammas = [kfac_factored_damping(f["A"], f["G"], g["damping"]) for f in facs]
        if self.inverse_method == "newton":
            res = damped_inverses_newton([F for f in facs for F in (f["A"], f["G"])],
                                         [gm for pair in gammas for gm in pair])
        else:
            eig = batched_eigh([F for f in facs for F in (f["A"], f["G"])])
        conds = []
        for i, (name, f) in enumerate(zip(names, facs)):
            gamma_A, gamma_G = gammas[i]
            if self.inverse_method == "newton":
                (iA, cA), (iG, cG) = res[2 * i], res[2 * i + 1]
            else:
                iA, cA = self._damped_inverse_from(*eig[2 * i], gamma_A, f["A"].dtype)
                iG, cG = self._damped_inverse_from(*eig[2 * i + 1], gamma_G, f["G"].dtype)
            self._inv[name] = {"iA": iA, "iG": iG, "cond_A": cA, "cond_G": cG}
            conds.append((cA, cG))
        return conds

    # ------------------------------------------------------------------ step
    def _check_curvature(self, g0) -> None:
        """Every selected layer with a gradient must have fresh curvature on a
        statistics step: a fused or functional call can bypass the hooks."""
        for name, module in self._name_to_module.items():
            if module.weight.grad is None and not (self.tracker.includes_bias(module) and module.bias.grad is not None):
                continue
            fresh = self.tracker._counts.get(name, 0) > self._last_counts.get(name, 0)
            if name not in self.tracker.factors or (self._steps % g0["stats_every"] == 0 and not fresh):
                raise RuntimeError(
                    f"No K-FAC curvature collected for {name!r}. Check update_curvature "
                    "and module hooks; fused/functional projections bypass hooks. "
                    "For Mamba-2, use_mem_eff_path=False exposes out_proj.")

    def _precondition_many(self, items):
        """{name: preconditioned V} for [(name, V)]. K-FAC's same-shape
        modules share one batched two-sided product (the same per-module
        arithmetic, one launch per product); subclasses that override
        _precondition (EKFAC) are called per module."""
        if type(self)._precondition is not KFAC._precondition:
            return {name: self._precondition(name, V) for name, V in items}
        out, buckets = {}, {}
        for name, V in items:
            inv = self._inv.get(name)
            if inv is None:
                raise RuntimeError(f"Missing K-FAC inverse for {name!r}")
            key = (tuple(inv["iG"].shape), tuple(V.shape), tuple(inv["iA"].shape), inv["iG"].dtype, V.dtype, V.device)
            buckets.setdefault(key, []).append((name, V))
        for group in buckets.values():
            if len(group) == 1:
                name, V = group[0]
                out[name] = self._precondition(name, V)
                continue
            iG = torch.stack([self._inv[n]["iG"] for n, _ in group])
            iA = torch.stack([self._inv[n]["iA"] for n, _ in group])
            Vs = torch.stack([V.to(iG.dtype) for _, V in group])
            with torch.autocast(device_type=Vs.device.type, enabled=False):
                P = ops.precond_apply_two_sided(iG, Vs, iA)
            for j, (name, V) in enumerate(group):
                out[name] = P[j].to(V.dtype)
        return out

    def _natural_gradients(self):
        nat = []  # (parameter, its natural-gradient direction)
        todo = []
        for name, m in self._name_to_module.items():
            w = m.weight
            has_bias = self.tracker.includes_bias(m)
            if w.grad is None and not (has_bias and m.bias.grad is not None):
                continue
            gW = (w.grad if w.grad is not None else torch.zeros_like(w)).reshape(w.shape[0], -1)
            if has_bias:
                gb = m.bias.grad if m.bias.grad is not None else torch.zeros_like(m.bias)
                V = torch.cat([gW, gb.unsqueeze(1)], dim=1)
            else:
                V = gW
            todo.append((name, m, has_bias, V))
        pre = self._precondition_many([(name, V) for name, _, _, V in todo])
        for name, m, has_bias, _ in todo:
            V, w = pre[name], m.weight
            if w.grad is not None:
                nat.append((w, (V[:, :-1] if has_bias else V).reshape(w.shape)))
            if has_bias and m.bias.grad is not None:
                nat.append((m.bias, V[:, -1]))
        return nat

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        g0 = self.param_groups[0]
        self._check_curvature(g0)
        groups = {id(p): group for group in self.param_groups for p in group["params"]}
        curvature_ms = 0.0
        conds = []
        with StepTimer() as t_all:
            if self.tracker.factors and self._steps % g0["inv_every"] == 0:
                with StepTimer() as t_c:
                    conds = self._refresh_inverses()
                curvature_ms = t_c.ms
                self._inv_stale = 0
            elif self._inv:
                self._inv_stale += 1
            nat = self._natural_gradients()
            nat_norm = torch.sqrt(sum(d.pow(2).sum() for _, d in nat)) if nat else torch.tensor(0.0)
            scale = 1.0
            if g0["max_grad_norm"] is not None and float(nat_norm) > g0["max_grad_norm"]:
                scale = g0["max_grad_norm"] / (float(nat_norm) + 1e-12)
            for p, d in nat:
                group = groups[id(p)]
                st = self.state[p]
                if group["momentum"]:
                    if "momentum_buffer" not in st:
                        st["momentum_buffer"] = torch.zeros_like(p)
                    st["momentum_buffer"].mul_(group["momentum"]).add_(d, alpha=scale)
                    upd = st["momentum_buffer"]
                else:
                    upd = d * scale
                if group["weight_decay"]:
                    p.mul_(1.0 - group["lr"] * group["weight_decay"])
                p.add_(upd, alpha=-group["lr"])
            n_adamw = 0
            for group in self.param_groups:
                if group["use_preconditioner"]:
                    continue
                for p in group["params"]:
                    if p.grad is not None:
                        adamw_update(p, p.grad, self.state[p], group)
                        n_adamw += 1
            self._last_counts = dict(self.tracker._counts)
            self._steps += 1
            self._sync_tracking()
        self._diag = {
            "n_adamw_params": n_adamw,
            "damping": g0["damping"],
            "mean_cond_A": sum(c[0] for c in conds) / len(conds) if conds else None,
            "mean_cond_G": sum(c[1] for c in conds) / len(conds) if conds else None,
            "inv_stale_steps": self._inv_stale,
            "nat_grad_norm": float(nat_norm),
            "step_ms": t_all.ms,
            "curvature_ms": curvature_ms,
        }
        return loss

    # ------------------------------------------------------------ state dict
    def state_dict(self):
        sd = super().state_dict()
        sd["kfac"] = {
            "steps": self._steps,
            "inv_stale": self._inv_stale,
            "factors": {n: dict(f) for n, f in self.tracker.factors.items()},
            "inv": {n: dict(d) for n, d in self._inv.items()},
            "counts": dict(self.tracker._counts),
            "last_counts": dict(self._last_counts),
            "modules": list(self._name_to_module),
            "bias_modules": sorted(self.tracker.bias_modules),
            "fisher_mode": self.fisher_mode,
            "ema_decay": self.tracker.ema_decay,
            "grad_scale": self.tracker.grad_scale,
        }
        return sd

    def load_state_dict(self, sd):
        sd = dict(sd)
        extra = sd.pop("kfac", None)
        if extra is None:
            raise ValueError("Checkpoint is missing K-FAC curvature state")
        if "modules" in extra and (extra["modules"] != list(self._name_to_module)
                                   or extra["bias_modules"] != sorted(self.tracker.bias_modules)):
            raise ValueError("Checkpoint K-FAC module selection differs from this optimizer")
        validate_checkpoint_groups(self.param_groups, sd["param_groups"])
        super().load_state_dict(sd)
        self._steps = int(extra["steps"])
        self._inv_stale = int(extra["inv_stale"])
        self.fisher_mode = extra.get("fisher_mode", self.fisher_mode)
        self.tracker.ema_decay = extra.get("ema_decay", self.tracker.ema_decay)
        self.tracker.set_grad_scale(extra.get("grad_scale", 1.0))
        self.tracker.factors = self._restore_curvature(extra["factors"])
        self._inv = self._restore_curvature(extra["inv"])
        self.tracker._counts = dict(extra["counts"])
        self._last_counts = dict(extra.get("last_counts", extra["counts"]))
        self._sync_tracking()

    def _restore_curvature(self, values):
        """Curvature tensors back on each module's device, in float64 for a
        float64 weight and float32 otherwise."""
        restored = {}
        for name, tensors in values.items():
            weight = self._name_to_module[name].weight
            dtype = torch.float64 if weight.dtype == torch.float64 else torch.float32
            restored[name] = {k: v.to(device=weight.device, dtype=dtype).clone() if torch.is_tensor(v) else v
                              for k, v in tensors.items()}
        return restored
