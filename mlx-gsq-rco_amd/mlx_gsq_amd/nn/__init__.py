"""Packed-weight modules."""
from .embedding import GSQEmbedding
from .linear import GSQLinear

__all__ = ["GSQEmbedding", "GSQLinear"]
