"""Explicit parameter groups shared by the matrix optimizers and AdamW.

Same behaviour as the reference's pytorch_opt/optim/routing.py:6-53: the
named Linear / ungrouped Conv2d weights are selected for the matrix
preconditioner; every other trainable parameter goes to AdamW exactly once;
vectors, biases and parameters flagged ``_no_weight_decay`` never decay;
shared (tied) weights cannot be selected.
"""

from torch import nn


def matrix_param_groups(model, module_names, *, lr, adamw_lr=3e-4, weight_decay=0.0, adamw_wd=0.0):
    names = list(module_names)
    if len(set(names)) != len(names):
        raise ValueError("module_names contains duplicates")
    modules = dict(model.named_modules())
    uses = {}
    for mod in model.modules():
        for prm in mod.parameters(recurse=False):
            uses[id(prm)] = uses.get(id(prm), 0) + 1
    chosen = set()
    for name in names:
        mod = modules.get(name)
        if mod is None:
            raise ValueError(f"Unknown module {name!r}")
        ok = isinstance(mod, nn.Linear) or (isinstance(mod, nn.Conv2d) and mod.groups == 1)
        if not ok:
            raise ValueError(f"{name!r} must be Linear or ungrouped Conv2d")
        if not mod.weight.requires_grad:
            raise ValueError(f"Selected weight {name!r} is frozen")
        if uses[id(mod.weight)] != 1:
            raise ValueError(f"Selected weight {name!r} is shared; assign it to AdamW")
        chosen.add(id(mod.weight))

    groups = {}
    for pname, prm in model.named_parameters():
        if not prm.requires_grad:
            continue
        primary = id(prm) in chosen
        decay = weight_decay if primary else adamw_wd
        if prm.ndim < 2 or pname.endswith("bias") or getattr(prm, "_no_weight_decay", False):
            decay = 0.0
        key = (primary, decay)
        if key not in groups:
            groups[key] = dict(params=[], param_names=[], use_preconditioner=primary,
                               lr=lr if primary else adamw_lr, weight_decay=decay)
        groups[key]["params"].append(prm)
        groups[key]["param_names"].append(pname)
    return list(groups.values())
