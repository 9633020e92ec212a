"""MI355X-native quantized-linear path over untouched GGUF superblocks.

Operators mirror the reference's seam (mlx_gsq/runtime/kernels/qmv.py, qmm.py,
registry.py, mlx_gsq/nn/linear.py, mlx_gsq/runtime/store.py) on torch tensors; the work
runs in hand-written gfx950 kernels in libgsq.so (C ABI: include/gsq.h).
"""
from .formats import BLOCK_BYTES, QTYPES, TYPE_IDS

__all__ = ["BLOCK_BYTES", "QTYPES", "TYPE_IDS"]
__version__ = "0.1.0"
