from .ekfac import EKFAC
from .kfac import KFAC
from .muon import Muon
from .routing import matrix_param_groups
from .shampoo import Shampoo
from .soap import SOAP

__all__ = ["Muon", "Shampoo", "SOAP", "KFAC", "EKFAC", "matrix_param_groups"]
