"""Explicit parameter groups shared by the matrix optimizers and AdamW.

matrix_param_groups has the behaviour of the reference's
pytorch_opt/optim/routing.py:6-53: the named nn.Linear / ungrouped
nn.Conv2d weights go to the matrix preconditioner, every other trainable
parameter to AdamW, each exactly once; vectors, biases and parameters
flagged ``_no_weight_decay`` never decay; a weight that several modules
share (tied) cannot be selected. The same groups serve an AdamW control
run. The error messages are the reference's.
"""

from collections import Counter

from torch import nn


def _holders(model) -> Counter:
    """Number of modules that register each parameter directly."""
    return Counter(id(p) for mod in model.modules() for p in mod.parameters(recurse=False))


def _matrix_module(mod) -> bool:
    return mod.groups == 1 if isinstance(mod, nn.Conv2d) else isinstance(mod, nn.Linear)


def _selection_error(name, mod, holders):
    """Why module `name` cannot be selected, or None."""
    if mod is None:
        return f"Unknown module {name!r}"
    if not _matrix_module(mod):
        return f"{name!r} must be Linear or ungrouped Conv2d"
    if not mod.weight.requires_grad:
        return f"Selected weight {name!r} is frozen"
    if holders[id(mod.weight)] > 1:
        return f"Selected weight {name!r} is shared; assign it to AdamW"
    return None


def _selected_weights(model, names) -> set:
    if len(set(names)) < len(names):
        raise ValueError("module_names contains duplicates")
    by_name, holders = dict(model.named_modules()), _holders(model)
    for name in names:
        err = _selection_error(name, by_name.get(name), holders)
        if err is not None:
            raise ValueError(err)
    return {id(by_name[name].weight) for name in names}


def matrix_param_groups(model, module_names, *, lr, adamw_lr=3e-4, weight_decay=0.0, adamw_wd=0.0):
    """Optimizer groups: selected weights (use_preconditioner=True, lr,
    weight_decay) and AdamW parameters (use_preconditioner=False, adamw_lr,
    adamw_wd), split further by whether they decay; each group lists its
    parameters' names in param_names, in model order."""
    selected = _selected_weights(model, list(module_names))

    def route(name, p):
        primary = id(p) in selected
        exempt = p.ndim < 2 or name.endswith("bias") or getattr(p, "_no_weight_decay", False)
        return primary, 0.0 if exempt else (weight_decay if primary else adamw_wd)

    groups = {}
    for name, p in model.named_parameters():
        if not p.requires_grad:
            continue
        key = route(name, p)
        group = groups.get(key)
        if group is None:
            primary, decay = key
            group = groups[key] = {"params": [], "param_names": [], "use_preconditioner": primary,
                                   "lr": lr if primary else adamw_lr, "weight_decay": decay}
        group["params"].append(p)
        group["param_names"].append(name)
    return list(groups.values())
