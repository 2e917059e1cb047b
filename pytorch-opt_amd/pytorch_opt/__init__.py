"""pytorch_opt — MI355X-native backend for the matrix-optimizer numerics.

Drop-in for the reference package's ``pytorch_opt.ops`` hot path and the
optimizers that drive it (Muon, Shampoo, the shared AdamW fallback and
routing, and the K-FAC factor tracker), plus SOAP, K-FAC and EKFAC, whose
rotations and preconditioner products run on the same kernels.
``pytorch_opt.ops.load_native()`` loads the gfx950 HIP library.
"""

from . import ops
from .curvature import KronTracker
from .optim import EKFAC, KFAC, SOAP, Muon, Shampoo, matrix_param_groups

__version__ = "0.1.0"

__all__ = ["ops", "Muon", "Shampoo", "SOAP", "KFAC", "EKFAC", "matrix_param_groups", "KronTracker", "__version__"]
