"""GGUF header reading, lossless conversion into the packed container, and the GGML type
constants the packed path validates with."""
from .container import FORMAT
from .converter import build_manifest, convert_gguf_to_mlx, convert_gguf_to_safetensors, verify_conversion
from .parser import GGMLQuantizationType, QUANT_BLOCK_SIZES
from .reader import GGUFError, GGUFReader, GGUFValueType, TensorInfo

__all__ = [
    "FORMAT", "GGMLQuantizationType", "GGUFError", "GGUFReader", "GGUFValueType", "QUANT_BLOCK_SIZES",
    "TensorInfo", "build_manifest", "convert_gguf_to_mlx", "convert_gguf_to_safetensors", "verify_conversion",
]
