"""Device operators: fused QMV, tiled QMM, the packed embedding gather and the dequantization
registry."""
from .embedding import iq2_s_embedding
from .qmm import QMM_MIN_ROWS, quantized_matmul
from .qmv import quantized_matvec
from .registry import SUPPORTED_QUANT_TYPES, decode, decode_weight

__all__ = ["QMM_MIN_ROWS", "iq2_s_embedding", "quantized_matmul", "quantized_matvec", "SUPPORTED_QUANT_TYPES",
           "decode", "decode_weight"]
