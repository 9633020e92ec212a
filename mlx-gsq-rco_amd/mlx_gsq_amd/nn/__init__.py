"""Packed-weight modules."""
from .linear import GSQLinear

__all__ = ["GSQLinear"]
