"""Packed-weight modules."""
from .embedding import GSQEmbedding
from .linear import GSQFusedLinear, GSQLinear

__all__ = ["GSQEmbedding", "GSQFusedLinear", "GSQLinear"]
