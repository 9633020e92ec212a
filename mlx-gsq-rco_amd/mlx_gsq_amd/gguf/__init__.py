"""GGML type ids and block sizes (validation constants of the packed path)."""
from .parser import GGMLQuantizationType, QUANT_BLOCK_SIZES

__all__ = ["GGMLQuantizationType", "QUANT_BLOCK_SIZES"]
