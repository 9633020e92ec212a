"""Packed-weight modules."""
from .embedding import GSQEmbedding
from .linear import GSQFusedLinear, GSQGroupedLinear, GSQLinear

__all__ = ["GSQEmbedding", "GSQFusedLinear", "GSQGroupedLinear", "GSQLinear"]
