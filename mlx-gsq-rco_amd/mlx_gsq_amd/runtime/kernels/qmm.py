"""Tiled quantized matrix-matrix product on packed GGUF weights (prefill path).

Drop-in counterpart of mlx_gsq/runtime/kernels/qmm.py:559-594 ``quantized_matmul``:
same name, keyword arguments (``kt`` is accepted for compatibility; the gfx950 kernel
chooses its own K tiling), validation and exceptions. Each wave decodes its own weight rows
straight from the packed superblocks (DMA'd into LDS) into fp16 MFMA operands in registers,
once per product, and multiplies them with fp16 activation tiles staged in LDS, accumulating in
fp32 (libgsq.so; M <= 16 runs a small-batch kernel that decodes every weight once as well).
"""
from __future__ import annotations

import torch

from ... import _lib
from ...formats import QTYPES, TYPE_IDS
from ...gguf.parser import GGMLQuantizationType, QUANT_BLOCK_SIZES

# Same routing threshold as the reference (qmm.py:26): quantized_matvec sends inputs with
# at least this many rows here.
QMM_MIN_ROWS = 8


def quantized_matmul(x, packed, *, qtype: str, out_features: int, in_features: int, kt: int = 256,
                     out_dtype=None):
    if qtype not in QTYPES:
        raise NotImplementedError(f"no tiled QMM kernel for {qtype}")
    if kt not in (128, 256):
        raise ValueError(f"unsupported kt {kt}")
    type_id = int(GGMLQuantizationType[qtype])
    block_elements, block_bytes = QUANT_BLOCK_SIZES[type_id]
    if block_elements != 256 or in_features % 256:
        raise ValueError(f"invalid {qtype} matrix width")
    expected = out_features * (in_features // 256) * block_bytes
    if packed.numel() != expected:
        raise ValueError(f"packed size {packed.numel()} != expected {expected}")
    if x.shape[-1] != in_features:
        raise ValueError("input feature size mismatch")
    if packed.dtype != torch.uint8:
        raise TypeError("packed input must be uint8")
    if x.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"unsupported activation dtype {x.dtype}")
    if x.device.type != "cuda" or packed.device != x.device:
        raise ValueError("x and packed must be on the same GPU device")
    original = x.shape[:-1]
    rows = x.numel() // in_features
    flat = x.reshape(rows, in_features).contiguous()
    packed = packed.contiguous()
    odt = out_dtype or x.dtype
    y = torch.empty((rows, out_features), dtype=odt, device=x.device)
    if rows:
        _lib.ensure_tables(qtype, x.device)
        with torch.cuda.device(x.device):
            _lib.check(_lib.lib().gsq_qmm(TYPE_IDS[qtype], packed.data_ptr(), flat.data_ptr(),
                                          _lib.DTYPE_CODES[flat.dtype], y.data_ptr(), _lib.DTYPE_CODES[odt],
                                          rows, out_features, in_features, _lib.stream_handle(x.device)),
                       "quantized_matmul")
    return y.reshape(*original, out_features)
