"""Loading `libomnia_hip.so` and calling its C ABI from torch."""

from .loader import LibraryMissing, available, call, last_error, library

__all__ = ["LibraryMissing", "available", "call", "last_error", "library"]
