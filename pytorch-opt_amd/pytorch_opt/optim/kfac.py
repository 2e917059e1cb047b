"""K-FAC natural-gradient optimizer (Martens & Grosse) on the MFMA kernels.

Behaviour of the reference's pytorch_opt/optim/kfac.py: the optimizer takes
the model; K-FAC preconditions the weights (and optionally biases) of its
nn.Linear / ungrouped nn.Conv2d modules whose weight is trainable and held
by one module only, every other trainable parameter takes the AdamW
fallback, or an explicit ``params`` split (groups flagged
use_preconditioner) decides (:28-105). Factor statistics come from the
training backward every ``stats_every`` steps; every ``inv_every`` steps
the damped inverses (F + γI)⁻¹ are refreshed with π-split damping
(:133-158); a module's gradient V (out × in, bias column appended) becomes
(G + γ_G I)⁻¹·V·(A + γ_A I)⁻¹, then global norm clipping, momentum, weight
decay and the update (:162-256). Curvature comes from the training backward
(``fisher_mode="empirical"``) or only from update_curvature(outputs),
an extra backward on labels sampled from the model (``"sampled"``, the
true Fisher, :27,124-131).

MI355X design:
  * statistics: KronTracker -> ops.gram_update_, one symmetric MFMA launch
    per factor per backward with the /n and the EMA fused;
  * inverses: float64 eigh batched over same-shape factors (the reference's
    method, default), or ``inverse_method="newton"``: the coupled Newton
    iteration at p = 1 on the MFMA root kernels, same-shape factors in one
    ops.inverse_matrix_root_each call (each with its own stop rule), in the
    factors' precision;
  * directions: modules with equal factor shapes are preconditioned in one
    batched two-sided MFMA product (one launch per product).
"""

from __future__ import annotations

from collections import Counter

import torch
from torch import nn
from torch.optim import Optimizer

from .. import ops
from ..curvature.damping import kfac_factored_damping
from ..curvature.kron import KronTracker
from ._common import DiagnosticsMixin, StepTimer, adamw_update, validate_checkpoint_groups, validate_groups

_FISHER_MODES = ("empirical", "sampled")
_INVERSE_METHODS = ("eigh", "newton")


# --------------------------------------------------------------- inverses

def _power_top(M: torch.Tensor, iters: int) -> torch.Tensor:
    """Largest eigenvalue of each symmetric PSD matrix of the batch M by
    power iteration from a fixed start (an estimate from below)."""
    g = torch.Generator(device=M.device).manual_seed(0)
    v = torch.randn(M.shape[0], M.shape[-1], 1, generator=g, device=M.device, dtype=M.dtype)
    for _ in range(iters):
        v = M @ v
        v = v / torch.linalg.vector_norm(v, dim=1, keepdim=True).clamp_min(torch.finfo(M.dtype).tiny)
    return (v.mT @ (M @ v)).reshape(-1)


def _by_shape(mats):
    """{(shape, device, dtype): [indices]} in first-seen order."""
    out = {}
    for i, M in enumerate(mats):
        out.setdefault((tuple(M.shape), M.device, M.dtype), []).append(i)
    return out


def _chunks(idx, per_entry_bytes: int, budget: int):
    step = max(1, budget // max(per_entry_bytes, 1))
    return (idx[s:s + step] for s in range(0, len(idx), step))


def batched_eigh(mats, batch_bytes: int = 4 << 30):
    """float64 eigendecomposition (eigenvalues, eigenvectors) of every matrix,
    same-shape matrices in one batched torch.linalg.eigh call."""
    out = [None] * len(mats)
    for (shape, _, _), idx in _by_shape(mats).items():
        for chunk in _chunks(idx, 8 * shape[-1] * shape[-1], batch_bytes):
            ev, V = torch.linalg.eigh(torch.stack([mats[i].double() for i in chunk]))
            for j, i in enumerate(chunk):
                out[i] = (ev[j], V[j])
    return out


def damped_inverses_newton(mats, gammas, batch_bytes: int = 4 << 30, power_iters: int = 30):
    """[(F_i + γ_i·I)⁻¹, estimated cond(F_i + γ_i·I))] by the coupled Newton
    iteration of ops.inverse_matrix_root at p = 1 (the MFMA root kernels on
    a GPU); same-shape factors share one ops.inverse_matrix_root_each call,
    each with its own stop rule. float64 factors iterate in float64 (tol
    1e-10), others in float32 (tol 1e-5). The condition number is
    λ_max(F + γI)·λ_max((F + γI)⁻¹), both by power iteration."""
    out = [None] * len(mats)
    for (shape, dev, dt), idx in _by_shape(mats).items():
        n = shape[-1]
        rdt = torch.float64 if dt == torch.float64 else torch.float32
        # the stack and the root's workspace: about eight n x n matrices per entry
        for chunk in _chunks(idx, 8 * n * n * torch.finfo(rdt).bits // 8, batch_bytes):
            eye = torch.eye(n, device=dev, dtype=rdt)
            M = torch.stack([mats[i].to(rdt) + gammas[i] * eye for i in chunk])
            inv = ops.inverse_matrix_root_each(M, 1, damping=0.0, method="newton", root_dtype=rdt,
                                               tol=1e-10 if rdt == torch.float64 else 1e-5)
            cond = (_power_top(M, power_iters) * _power_top(inv, power_iters)).tolist()
            for j, i in enumerate(chunk):
                out[i] = (inv[j].to(dt), cond[j])
    return out


def _inverse_from_eigh(ev, V, gamma, dtype):
    """(F + γI)⁻¹ = V·diag(1/(λ + γ))·Vᵀ and cond(F + γI) from F's float64 eigh."""
    inv = ((V / (ev + gamma)) @ V.mT).to(dtype)
    lo = max(float(ev.min()) + gamma, 1e-300)
    return inv, float(ev.max() + gamma) / lo


# --------------------------------------------------------------- selection

def _registrations(model) -> Counter:
    return Counter(id(p) for m in model.modules() for p in m.parameters(recurse=False))


def _preconditionable(model, regs) -> dict:
    """{name: module} of the modules K-FAC can precondition."""
    def ok(m):
        if isinstance(m, nn.Conv2d) and m.groups != 1:
            return False
        return isinstance(m, (nn.Linear, nn.Conv2d)) and m.weight.requires_grad and regs[id(m.weight)] == 1
    return {name: m for name, m in model.named_modules() if ok(m)}


def _automatic_groups(model, modules, regs, adamw_lr, adamw_wd):
    """The preconditioned group (the modules' untied trainable parameters)
    and AdamW groups for the rest: without decay (vectors, parameters marked
    _no_weight_decay), then with adamw_wd."""
    pre = [p for m in modules.values() for p in m.parameters(recurse=False) if p.requires_grad and regs[id(p)] == 1]
    taken = {id(p) for p in pre}
    rest = [p for p in model.parameters() if p.requires_grad and id(p) not in taken]
    decays = lambda p: p.ndim >= 2 and not getattr(p, "_no_weight_decay", False)  # noqa: E731
    groups = [{"params": pre, "use_preconditioner": True}]
    for decay in (False, True):
        members = [p for p in rest if decays(p) == decay]
        if members:
            groups.append({"params": members, "use_preconditioner": False, "lr": adamw_lr,
                           "weight_decay": adamw_wd if decay else 0.0})
    return groups


class KFAC(Optimizer, DiagnosticsMixin):
    def __init__(self, model: nn.Module, lr: float = 0.01, damping: float = 1e-3,
                 ema_decay: float | None = 0.95, momentum: float = 0.9, stats_every: int = 1, inv_every: int = 10,
                 fisher_mode: str = "empirical", weight_decay: float = 0.0, max_grad_norm: float | None = None, *,
                 params=None, adamw_lr: float = 3e-4, adamw_betas: tuple = (0.9, 0.95), adamw_eps: float = 1e-8,
                 adamw_wd: float = 0.0, inverse_method: str = "eigh"):
        if fisher_mode not in _FISHER_MODES:
            raise ValueError(f"fisher_mode must be one of {_FISHER_MODES}, got {fisher_mode!r}")
        if min(stats_every, inv_every) < 1:
            raise ValueError("stats_every and inv_every must be positive")
        if inverse_method not in _INVERSE_METHODS:
            raise ValueError(f"inverse_method must be one of {_INVERSE_METHODS}, got {inverse_method!r}")
        regs = _registrations(model)
        candidates = _preconditionable(model, regs)
        if params is None:
            groups = _automatic_groups(model, candidates, regs, adamw_lr, adamw_wd)
        else:
            groups = list(params)
            if not all(isinstance(g, dict) and isinstance(g.get("use_preconditioner"), bool) for g in groups):
                raise ValueError("KFAC params must be groups with explicit use_preconditioner")
        # the first group is a preconditioned one: it carries the curvature settings
        groups.sort(key=lambda g: 0 if g["use_preconditioner"] else 1)
        defaults = dict(lr=lr, damping=damping, momentum=momentum, stats_every=stats_every, inv_every=inv_every,
                        weight_decay=weight_decay, max_grad_norm=max_grad_norm, adamw_lr=adamw_lr,
                        adamw_betas=adamw_betas, adamw_eps=adamw_eps, adamw_wd=adamw_wd)
        super().__init__(groups, defaults)
        validate_groups(self.param_groups, matrices=False)
        self.model = model
        self.fisher_mode = fisher_mode
        self.inverse_method = inverse_method
        self._modules, bias_names = self._bind_selection(model, candidates, regs)
        self.tracker = KronTracker(model, ema_decay=ema_decay, module_names=self._modules, bias_modules=bias_names)
        self._steps = 0          # optimizer steps taken
        self._inv_stale = 0      # steps since the last inverse refresh
        self._inv: dict[str, dict] = {}
        self._last_counts: dict[str, int] = {}  # tracker update counts at the last step
        self._arm_tracker()

    def _bind_selection(self, model, candidates, regs):
        """Modules whose weight the preconditioned groups hold, and those of
        them whose (untied) bias is held too; every trainable parameter must be
        in exactly one group, and the preconditioned ones must be exactly
        those weights and biases."""
        trainable = {id(p) for p in model.parameters() if p.requires_grad}
        everything = [id(p) for g in self.param_groups for p in g["params"]]
        if set(everything) != trainable:
            raise ValueError("KFAC groups must cover every trainable model parameter exactly once")
        chosen = {id(p) for g in self.param_groups if g["use_preconditioner"] for p in g["params"]}
        modules = {n: m for n, m in candidates.items() if id(m.weight) in chosen}
        with_bias = {n for n, m in modules.items()
                     if m.bias is not None and id(m.bias) in chosen and regs[id(m.bias)] == 1}
        explained = {id(m.weight) for m in modules.values()} | {id(modules[n].bias) for n in with_bias}
        if explained != chosen:
            raise ValueError("KFAC selection must contain supported, untied module weights and optional biases")
        return modules, with_bias

    def _stats_step(self) -> bool:
        return self._steps % self.param_groups[0]["stats_every"] == 0

    def _arm_tracker(self) -> None:
        """Forward calls are bound on steps that are multiples of stats_every;
        the training backward feeds the factors on those steps only for the
        empirical Fisher (the sampled one feeds them from update_curvature)."""
        on = self._stats_step()
        self.tracker.capture = on
        self.tracker.enabled = on and self.fisher_mode == "empirical"

    def update_curvature(self, outputs: torch.Tensor, kind: str = "categorical",
                         generator: torch.Generator | None = None) -> None:
        """fisher_mode="sampled": accumulate the factors from one extra
        backward of `outputs` (the model's outputs of this step's forward)
        on labels drawn from the model's predictive distribution
        (KronTracker.sampled_backward); nothing outside statistics steps."""
        if self.fisher_mode != "sampled":
            raise RuntimeError("update_curvature() is only used with fisher_mode='sampled'; "
                               "empirical mode accumulates from the training backward")
        if self._stats_step():
            self.tracker.sampled_backward(outputs, kind=kind, generator=generator)

    def set_grad_scale(self, scale: float) -> None:
        """The scale of the next backward's loss (AMP scale / accumulation
        steps); it is divided out of the curvature only."""
        self.tracker.set_grad_scale(scale)

    @classmethod
    def state_layout(cls) -> dict:
        tags = dict.fromkeys(("A", "G", "iA", "iG", "steps", "inv_stale"), "replicable")
        tags.update(dict.fromkeys(("momentum_buffer", "step", "exp_avg", "exp_avg_sq"), "shardable"))
        return tags

    # ------------------------------------------------------------- curvature
    def _refresh_inverses(self) -> list[tuple[float, float]]:
        """Damped inverses of every module's factors; returns (cond_A, cond_G)."""
        damping = self.param_groups[0]["damping"]
        names = list(self.tracker.factors)
        pairs = [(self.tracker.factors[n]["A"], self.tracker.factors[n]["G"]) for n in names]
        gammas = [kfac_factored_damping(A, G, damping) for A, G in pairs]
        flat = [F for pair in pairs for F in pair]
        flat_gammas = [gm for pair in gammas for gm in pair]
        if self.inverse_method == "newton":
            done = damped_inverses_newton(flat, flat_gammas)
        else:
            done = [_inverse_from_eigh(ev, V, gm, F.dtype)
                    for (ev, V), gm, F in zip(batched_eigh(flat), flat_gammas, flat)]
        conds = []
        for k, name in enumerate(names):
            (iA, cA), (iG, cG) = done[2 * k], done[2 * k + 1]
            self._inv[name] = {"iA": iA, "iG": iG, "cond_A": cA, "cond_G": cG}
            conds.append((cA, cG))
        return conds

    def _precondition(self, name: str, V: torch.Tensor) -> torch.Tensor:
        """(G + γ_G I)⁻¹·V·(A + γ_A I)⁻¹ for one module (EKFAC overrides this)."""
        inv = self._inv.get(name)
        if inv is None:
            raise RuntimeError(f"Missing K-FAC inverse for {name!r}")
        with torch.autocast(device_type=V.device.type, enabled=False):
            return ops.precond_apply_two_sided(inv["iG"], V.to(inv["iG"].dtype), inv["iA"]).to(V.dtype)

    def _precondition_many(self, items) -> dict:
        """{name: direction} for [(name, V)]: modules with equal factor and
        gradient shapes share one batched two-sided product (per-module
        arithmetic unchanged); a subclass with its own _precondition is
        called per module."""
        if type(self)._precondition is not KFAC._precondition:
            return {name: self._precondition(name, V) for name, V in items}
        for name, _ in items:
            if name not in self._inv:
                raise RuntimeError(f"Missing K-FAC inverse for {name!r}")
        bins = {}
        for name, V in items:
            inv = self._inv[name]
            bins.setdefault((inv["iG"].shape, V.shape, inv["iA"].shape, inv["iG"].dtype, V.dtype, V.device),
                            []).append((name, V))
        out = {}
        for members in bins.values():
            if len(members) == 1:
                (name, V), = members
                out[name] = self._precondition(name, V)
                continue
            iG = torch.stack([self._inv[n]["iG"] for n, _ in members])
            iA = torch.stack([self._inv[n]["iA"] for n, _ in members])
            with torch.autocast(device_type=iG.device.type, enabled=False):
                P = ops.precond_apply_two_sided(iG, torch.stack([V.to(iG.dtype) for _, V in members]), iA)
            out.update((name, P[j].to(V.dtype)) for j, (name, V) in enumerate(members))
        return out

    # ------------------------------------------------------------------ step
    def _gradient_matrices(self):
        """[(name, module, has_bias, V)] for the modules with a gradient, V the
        weight gradient as (out, -1) with the bias gradient appended."""
        out = []
        for name, m in self._modules.items():
            has_bias = self.tracker.includes_bias(m)
            gw, gb = m.weight.grad, (m.bias.grad if has_bias else None)
            if gw is None and gb is None:
                continue
            V = (gw if gw is not None else torch.zeros_like(m.weight)).reshape(m.weight.shape[0], -1)
            if has_bias:
                V = torch.cat([V, (gb if gb is not None else torch.zeros_like(m.bias)).unsqueeze(1)], dim=1)
            out.append((name, m, has_bias, V))
        return out

    def _require_fresh_curvature(self, todo) -> None:
        """On a statistics step every module with a gradient must have been
        seen by the hooks (fused or functional calls bypass them)."""
        stats_step = self._stats_step()
        for name, _, _, _ in todo:
            fresh = self.tracker.updates(name) > self._last_counts.get(name, 0)
            if name not in self.tracker.factors or (stats_step and not fresh):
                raise RuntimeError(
                    f"No K-FAC curvature collected for {name!r}. Check update_curvature and the module hooks: "
                    "fused or functional projections bypass them.")

    def _apply_direction(self, p, d, scale) -> None:
        group = self._group_of[id(p)]
        st = self.state[p]
        if group["momentum"]:
            buf = st.get("momentum_buffer")
            if buf is None:
                buf = st["momentum_buffer"] = torch.zeros_like(p)
            d = buf.mul_(group["momentum"]).add_(d, alpha=scale)
        elif scale != 1.0:
            d = d * scale
        if group["weight_decay"]:
            p.mul_(1.0 - group["lr"] * group["weight_decay"])
        p.add_(d, alpha=-group["lr"])

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        g0 = self.param_groups[0]
        todo = self._gradient_matrices()
        self._require_fresh_curvature(todo)
        self._group_of = {id(p): g for g in self.param_groups for p in g["params"]}
        conds, curvature_ms = [], 0.0
        with StepTimer() as timer:
            if self.tracker.factors and self._steps % g0["inv_every"] == 0:
                with StepTimer() as tc:
                    conds = self._refresh_inverses()
                curvature_ms = tc.ms
                self._inv_stale = 0
            elif self._inv:
                self._inv_stale += 1
            pre = self._precondition_many([(name, V) for name, _, _, V in todo])
            directions = []
            for name, m, has_bias, _ in todo:
                D = pre[name]
                if m.weight.grad is not None:
                    directions.append((m.weight, (D[:, :-1] if has_bias else D).reshape(m.weight.shape)))
                if has_bias and m.bias.grad is not None:
                    directions.append((m.bias, D[:, -1]))
            nat_norm = float(torch.sqrt(sum(d.pow(2).sum() for _, d in directions))) if directions else 0.0
            clip = g0["max_grad_norm"]
            scale = clip / (nat_norm + 1e-12) if clip is not None and nat_norm > clip else 1.0
            for p, d in directions:
                self._apply_direction(p, d, scale)
            n_adamw = 0
            for group in (g for g in self.param_groups if not g["use_preconditioner"]):
                for p in (q for q in group["params"] if q.grad is not None):
                    adamw_update(p, p.grad, self.state[p], group)
                    n_adamw += 1
            self._last_counts = self.tracker.update_counts()
            self._steps += 1
            self._arm_tracker()
        mean = lambda k: sum(c[k] for c in conds) / len(conds) if conds else None  # noqa: E731
        self._diag = {"n_adamw_params": n_adamw, "damping": g0["damping"], "mean_cond_A": mean(0),
                      "mean_cond_G": mean(1), "inv_stale_steps": self._inv_stale, "nat_grad_norm": nat_norm,
                      "step_ms": timer.ms, "curvature_ms": curvature_ms}
        return loss

    # ------------------------------------------------------------ checkpoint
    # The "kfac" entry carries the reference's keys (pytorch_opt/optim/kfac.py:
    # 260-298), so checkpoints move between the two implementations.
    def _extra_state(self) -> dict:
        return {"steps": self._steps, "inv_stale": self._inv_stale,
                "factors": {n: dict(f) for n, f in self.tracker.factors.items()},
                "inv": {n: dict(f) for n, f in self._inv.items()},
                "counts": self.tracker.update_counts(), "last_counts": dict(self._last_counts),
                "modules": list(self._modules), "bias_modules": sorted(self.tracker.bias_modules),
                "fisher_mode": self.fisher_mode, "ema_decay": self.tracker.ema_decay,
                "grad_scale": self.tracker.grad_scale}

    def state_dict(self):
        sd = super().state_dict()
        sd["kfac"] = self._extra_state()
        return sd

    def load_state_dict(self, state_dict):
        """Restores a checkpoint of either implementation. The module lists
        are compared as sets (the reference writes them in named_modules
        order); optional keys fall back as the reference's loader does."""
        sd = dict(state_dict)
        extra = sd.pop("kfac", None)
        if extra is None:
            raise ValueError("Checkpoint is missing K-FAC curvature state")
        if "modules" in extra and (set(extra["modules"]) != set(self._modules)
                                   or sorted(extra.get("bias_modules", ())) != sorted(self.tracker.bias_modules)):
            raise ValueError("Checkpoint K-FAC module selection differs from this optimizer")
        mode = extra.get("fisher_mode", self.fisher_mode)
        if mode not in _FISHER_MODES:
            raise ValueError(f"fisher_mode must be one of {_FISHER_MODES}, got {mode!r}")
        validate_checkpoint_groups(self.param_groups, sd["param_groups"])
        super().load_state_dict(sd)
        self._steps, self._inv_stale = int(extra["steps"]), int(extra["inv_stale"])
        self.fisher_mode = mode
        self.tracker.ema_decay = extra.get("ema_decay", self.tracker.ema_decay)
        self.tracker.set_grad_scale(extra.get("grad_scale", 1.0))
        self.tracker.factors = self._on_module_device(extra["factors"])
        self._inv = self._on_module_device(extra["inv"])
        self.tracker.restore_counts(extra["counts"])
        # "seen_counts": the key an earlier version of this module wrote
        self._last_counts = dict(extra.get("last_counts", extra.get("seen_counts", extra["counts"])))
        self._arm_tracker()

    def _on_module_device(self, tree: dict) -> dict:
        """Copies of a {name: {key: value}} tree with every tensor on its
        module's device, float64 for float64 weights, float32 otherwise."""
        out = {}
        for name, entries in tree.items():
            w = self._modules[name].weight
            dt = torch.float64 if w.dtype == torch.float64 else torch.float32
            out[name] = {k: (v.to(device=w.device, dtype=dt).clone() if torch.is_tensor(v) else v)
                         for k, v in entries.items()}
        return out
