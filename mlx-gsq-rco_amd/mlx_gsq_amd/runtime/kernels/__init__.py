"""Device operators: fused QMV, tiled QMM and the dequantization registry."""
from .qmm import QMM_MIN_ROWS, quantized_matmul
from .qmv import quantized_matvec
from .registry import SUPPORTED_QUANT_TYPES, decode, decode_weight

__all__ = ["QMM_MIN_ROWS", "quantized_matmul", "quantized_matvec", "SUPPORTED_QUANT_TYPES", "decode", "decode_weight"]
