"""Dequantization registry: packed superblocks -> flat float32 on the GPU.

Drop-in counterpart of mlx_gsq/runtime/kernels/registry.py:8-46: the same
``SUPPORTED_QUANT_TYPES``, ``decode(packed, qtype)`` and
``decode_weight(weight, *, block_count=None)``, with the same exceptions. The device
decoder is bit-exact with the CPU dequantizer (libgsq.so ``gsq_dequant``).
"""
from __future__ import annotations

import torch

from ... import _lib
from ...formats import BLOCK_BYTES, TYPE_IDS

SUPPORTED_QUANT_TYPES = (
    "IQ1_M", "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS",
    "IQ3_S", "IQ4_XS", "Q2_K", "Q4_K", "Q6_K",
)


def decode(packed, qtype: str):
    """Flat uint8 payload of whole superblocks -> flat float32 tensor (nblocks * 256)."""
    if qtype not in SUPPORTED_QUANT_TYPES:
        raise NotImplementedError(f"validated decoder not yet available for {qtype}")
    if packed.dtype != torch.uint8:
        raise TypeError("packed input must be uint8")
    bb = BLOCK_BYTES[qtype]
    if packed.numel() % bb:
        raise ValueError(f"{qtype} payload is not block aligned")
    if packed.device.type != "cuda":
        raise ValueError("packed must be on a GPU device")
    packed = packed.reshape(-1).contiguous()
    nblocks = packed.numel() // bb
    out = torch.empty(nblocks * 256, dtype=torch.float32, device=packed.device)
    if nblocks:
        _lib.ensure_tables(qtype, packed.device)
        with torch.cuda.device(packed.device):
            _lib.check(_lib.lib().gsq_dequant(TYPE_IDS[qtype], packed.data_ptr(), nblocks, out.data_ptr(),
                                              _lib.stream_handle(packed.device)), "decode")
    return out


def decode_weight(weight, *, block_count: int | None = None):
    """Route a PackedWeight to its decoder using its metadata (registry.py:35-46)."""
    from ...gguf.parser import QUANT_BLOCK_SIZES

    qtype = weight.quantization_type
    if qtype not in SUPPORTED_QUANT_TYPES:
        raise TypeError(f"{weight.name} is not a supported quantized weight: {qtype}")
    data = weight.data
    if block_count is not None:
        block_bytes = QUANT_BLOCK_SIZES[weight.quantization_type_id][1]
        data = data[: block_count * block_bytes]
    return decode(data, qtype)
