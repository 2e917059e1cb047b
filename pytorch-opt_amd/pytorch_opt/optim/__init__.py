from .muon import Muon
from .routing import matrix_param_groups
from .shampoo import Shampoo

__all__ = ["Muon", "Shampoo", "matrix_param_groups"]
