"""Packed IQ2_S embedding row lookup on torch tensors.

Drop-in counterpart of mlx_gsq/runtime/kernels/embedding.py:30-36 ``iq2_s_embedding``: same
name, keyword arguments, checks and exceptions (dimensions % 256 and the packed size raise
``ValueError``), default output dtype bfloat16. Each output row is the exact float32 decode of
the packed row rounded once to the output dtype, computed by libgsq.so's gather kernel on the
ids' device and current stream.
"""
from __future__ import annotations

import torch

from ... import _lib
from ...formats import TYPE_IDS

IQ2_S_BLOCK_BYTES = 82


def iq2_s_embedding(ids, packed, *, vocab_size: int, dimensions: int, dtype=None):
    if dimensions % 256:
        raise ValueError("embedding dimensions must be divisible by 256")
    expected = vocab_size * (dimensions // 256) * IQ2_S_BLOCK_BYTES
    if packed.numel() != expected:
        raise ValueError("packed embedding size mismatch")
    dtype = dtype or torch.bfloat16
    if dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"unsupported embedding dtype {dtype}")
    if packed.dtype != torch.uint8:
        raise TypeError("packed input must be uint8")
    if ids.dtype not in _lib.ID_CODES:
        raise TypeError(f"ids must be int32 or int64, got {ids.dtype}")
    if ids.device.type != "cuda" or packed.device != ids.device:
        raise ValueError("ids and packed must be on the same GPU device")
    flat = ids.reshape(-1).contiguous()
    out = torch.empty((flat.numel(), dimensions), dtype=dtype, device=ids.device)
    if flat.numel():
        _lib.ensure_tables("IQ2_S", ids.device)
        with torch.cuda.device(ids.device):
            _lib.check(_lib.lib().gsq_embedding(TYPE_IDS["IQ2_S"], packed.contiguous().data_ptr(), flat.data_ptr(),
                                                _lib.ID_CODES[flat.dtype], flat.numel(), vocab_size, dimensions,
                                                out.data_ptr(), _lib.DTYPE_CODES[dtype], _lib.stream_handle(ids.device)),
                       "iq2_s_embedding")
    return out.reshape(*ids.shape, dimensions)
