from .kron import KronTracker

__all__ = ["KronTracker"]
