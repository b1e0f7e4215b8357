"""Layer declaration API: one facade per primitive, each resolving an ordered strategy
tuple whose HIP bindings precede the Core (stock-op) chains."""

from .resolve import RESOLVED, resolve

__all__ = ["RESOLVED", "resolve"]
