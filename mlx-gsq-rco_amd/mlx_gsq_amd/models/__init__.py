"""Model decode step around the packed projections."""
from .qwen35 import GraphDecoder, Qwen35Args, Qwen35Cache, Qwen35Model, build_qwen35

__all__ = ["GraphDecoder", "Qwen35Args", "Qwen35Cache", "Qwen35Model", "build_qwen35"]
