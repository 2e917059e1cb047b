"""Loader for the prebuilt gfx950 library (replaces the reference's JIT build,
pytorch_opt/ops/native_build.py:10-21).

The library is compiled ahead of time (``make -C pytorch-opt_amd/csrc`` or
``__graft_entry__.build()``) to ``libpytorch_opt_hip.so`` next to this file;
``PYTORCH_OPT_HIP_LIB`` may point at another copy.
"""

from __future__ import annotations

import os

LIB_NAME = "libpytorch_opt_hip.so"


def library_path() -> str:
    return os.environ.get("PYTORCH_OPT_HIP_LIB") or os.path.join(os.path.dirname(__file__), LIB_NAME)


def load(verbose: bool = False):
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)

    from ._hip import HipBackend

    path = library_path()
    if not os.path.exists(path):
        raise FileNotFoundError(f"native library not built: {path}")
    backend = HipBackend(path)
    if verbose:
        print(f"pytorch-opt: loaded {path} (version {backend.version})")
    return backend
