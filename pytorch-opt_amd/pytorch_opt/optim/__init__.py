from .muon import Muon
from .routing import matrix_param_groups
from .shampoo import Shampoo
from .soap import SOAP

__all__ = ["Muon", "Shampoo", "SOAP", "matrix_param_groups"]
