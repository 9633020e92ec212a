"""GGUF inspection, lossless packed-weight conversion, and the GGML type constants the packed
path validates with."""
from .converter import convert_gguf_to_mlx, convert_gguf_to_safetensors, verify_conversion
from .parser import GGMLQuantizationType, QUANT_BLOCK_SIZES
from .reader import GGUFError, GGUFModelAnalyzer, GGUFReader, GGUFValueType, TensorInfo

__all__ = [
    "GGMLQuantizationType", "GGUFError", "GGUFModelAnalyzer", "GGUFReader", "GGUFValueType",
    "QUANT_BLOCK_SIZES", "TensorInfo", "convert_gguf_to_mlx", "convert_gguf_to_safetensors",
    "verify_conversion",
]
