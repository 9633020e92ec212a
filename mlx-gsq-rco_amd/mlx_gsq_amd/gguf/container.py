"""The packed Safetensors container ("mlx-gsq-packed-v1"): header layout, written and read.

This is the file format PackedModelStore loads, shared with the reference so that files are
interchangeable (its writer: mlx_gsq/gguf/converter.py:22-57, its reader:
mlx_gsq/runtime/store.py:33-58). A Safetensors file is

    u64 little-endian header length | JSON header (UTF-8) | data section

and here every tensor is a 1-D ``U8`` array of ``num_bytes`` holding the tensor's GGUF payload
exactly as stored (no dequantization), the payloads back to back in GGUF directory order. The
header's ``__metadata__`` (string values only, as Safetensors requires) names the format and
carries ``tensor_quantization``, a compact JSON map from tensor name to its GGUF description
(qtype, qtype_id, gguf_shape, logical_shape = gguf_shape reversed, num_elements,
block_elements, block_bytes). The JSON is padded with spaces to a multiple of 8 bytes, so the
data section starts 8-byte aligned.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

from .parser import QUANT_BLOCK_SIZES

FORMAT = "mlx-gsq-packed-v1"
_LEN = struct.Struct("<Q")
# a header larger than this is not a container of this format (Safetensors caps it at 100 MB)
MAX_HEADER_BYTES = 100 * 1024 * 1024


def quantization_record(t) -> dict:
    """The ``tensor_quantization`` entry of one GGUF tensor (a reader ``TensorInfo``)."""
    per_block, block_bytes = QUANT_BLOCK_SIZES[int(t.quantization_type)]
    return {"qtype": t.quantization_type.name, "qtype_id": int(t.quantization_type),
            "gguf_shape": list(t.shape), "logical_shape": list(t.shape[::-1]),
            "num_elements": t.num_elements, "block_elements": per_block, "block_bytes": block_bytes}


def build_header(tensors, architecture: str) -> bytes:
    """Length prefix + padded JSON header for ``tensors`` stored back to back."""
    doc = {"__metadata__": {
        "format": FORMAT,
        "source_format": "GGUF",
        "architecture": architecture,
        "note": "each tensor is the untouched GGUF packed payload as U8; decode with the packed kernels",
        "tensor_quantization": json.dumps({t.name: quantization_record(t) for t in tensors}, separators=(",", ":")),
    }}
    end = 0
    for t in tensors:
        if t.name in doc:
            raise ValueError(f"tensor name {t.name!r} cannot be stored in a Safetensors header")
        doc[t.name] = {"dtype": "U8", "shape": [t.num_bytes], "data_offsets": [end, end + t.num_bytes]}
        end += t.num_bytes
    body = json.dumps(doc, ensure_ascii=False, separators=(",", ":")).encode("utf-8")
    body += b" " * (-len(body) % 8)
    return _LEN.pack(len(body)) + body


def read_header(path) -> tuple[dict, int]:
    """(header JSON, file offset of the data section) of a Safetensors file."""
    path = Path(path)
    with path.open("rb") as f:
        raw = f.read(_LEN.size)
        if len(raw) != _LEN.size:
            raise ValueError(f"{path.name}: too short for a Safetensors file")
        (n,) = _LEN.unpack(raw)
        if n > MAX_HEADER_BYTES:
            raise ValueError(f"{path.name}: header length {n} is not plausible")
        body = f.read(n)
    if len(body) != n:
        raise ValueError(f"{path.name}: header cut short ({len(body)} of {n} bytes)")
    return json.loads(body), _LEN.size + n
