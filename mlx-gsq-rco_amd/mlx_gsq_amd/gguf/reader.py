"""GGUF (v2 / v3) directory reader: metadata and tensor extents, no payload reads.

Counterpart of mlx_gsq/gguf/parser.py:72-145 (``GGUFReader``, ``TensorInfo``, ``GGUFError``)
with the same public names, fields and checks: magic, version 2 or 3, unique metadata keys and
tensor names, a positive integer ``general.alignment`` (default 32), element counts that fill
whole blocks, tensors inside the file and not overlapping. The header is parsed from a
read-only memory map, so a multi-GB model costs only the pages of its header.

The file layout is GGUF's published one: magic "GGUF", u32 version, u64 tensor count, u64
metadata count, the metadata key/value pairs (u64-length UTF-8 key, u32 value type, value),
then per tensor its name, u32 rank, u64 dims (innermost first), u32 GGML type and u64 offset
from the data section, which starts at the next multiple of the alignment.
"""
from __future__ import annotations

import json
import mmap
import struct
from collections import defaultdict
from dataclasses import dataclass
from enum import IntEnum
from pathlib import Path
from typing import Any

from .parser import GGMLQuantizationType, QUANT_BLOCK_SIZES


class GGUFError(ValueError):
    pass


class GGUFValueType(IntEnum):
    UINT8 = 0; INT8 = 1; UINT16 = 2; INT16 = 3; UINT32 = 4; INT32 = 5; FLOAT32 = 6
    BOOL = 7; STRING = 8; ARRAY = 9; UINT64 = 10; INT64 = 11; FLOAT64 = 12


# scalar value types -> struct format (little endian)
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


@dataclass(frozen=True)
class TensorInfo:
    name: str
    shape: tuple
    quantization_type: GGMLQuantizationType
    offset: int
    absolute_offset: int
    num_elements: int
    num_bytes: int

    def as_dict(self) -> dict:
        return {
            "name": self.name,
            "gguf_shape": list(self.shape),
            "logical_shape": list(reversed(self.shape)),
            "quantization_type": self.quantization_type.name,
            "quantization_type_id": int(self.quantization_type),
            "offset": self.offset,
            "absolute_offset": self.absolute_offset,
            "num_elements": self.num_elements,
            "num_bytes": self.num_bytes,
        }


class _Cursor:
    """Sequential little-endian reads from a buffer, with end-of-file checks."""

    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> bytes:
        end = self.pos + n
        if n < 0 or end > len(self.buf):
            raise GGUFError("unexpected end of file")
        raw = self.buf[self.pos:end]
        self.pos = end
        return raw

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar("<Q")
        try:
            return self.take(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GGUFError(f"invalid UTF-8 string: {e}") from None

    def value(self, kind: int):
        if kind in _SCALARS:
            return self.scalar(_SCALARS[kind])
        if kind == GGUFValueType.STRING:
            return self.string()
        if kind == GGUFValueType.ARRAY:
            sub = self.scalar("<I")
            n = self.scalar("<Q")
            if sub in _SCALARS and sub != GGUFValueType.BOOL:  # fixed-size items: one slice
                size = struct.calcsize(_SCALARS[sub])
                raw = self.take(size * n)
                return list(struct.unpack("<" + str(n) + _SCALARS[sub][1], raw))
            return [self.value(sub) for _ in range(n)]
        raise GGUFError(f"unsupported metadata type {kind}")


class GGUFReader:
    """Validated GGUF metadata and tensor extents of one file."""

    def __init__(self, path):
        self.path = Path(path).expanduser().resolve()
        self.file_size = self.path.stat().st_size
        with self.path.open("rb") as f:
            if self.file_size < 4:
                raise GGUFError("not a GGUF file")
            with mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
                self._parse(_Cursor(mm))  # slices of the map are copies: nothing outlives it

    def _parse(self, c: _Cursor) -> None:
        if c.take(4) != b"GGUF":
            raise GGUFError("not a GGUF file")
        self.version = c.scalar("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"unsupported GGUF version {self.version}")
        n_tensors, n_kv = c.scalar("<Q"), c.scalar("<Q")
        self.metadata: dict = {}
        for _ in range(n_kv):
            key = c.string()
            if key in self.metadata:
                raise GGUFError(f"duplicate metadata key {key}")
            kind = c.scalar("<I")
            try:
                GGUFValueType(kind)
            except ValueError:
                raise GGUFError(f"unsupported metadata type {kind}") from None
            self.metadata[key] = c.value(kind)
        entries = []
        seen = set()
        for _ in range(n_tensors):
            name = c.string()
            if name in seen:
                raise GGUFError(f"duplicate tensor {name}")
            seen.add(name)
            rank = c.scalar("<I")
            shape = tuple(c.scalar("<Q") for _ in range(rank))
            type_id = c.scalar("<I")
            try:
                qtype = GGMLQuantizationType(type_id)
            except ValueError:
                raise GGUFError(f"unknown GGML type {type_id} for {name}") from None
            entries.append((name, shape, qtype, c.scalar("<Q")))
        align = self.metadata.get("general.alignment", 32)
        if isinstance(align, bool) or not isinstance(align, int) or align < 1:
            raise GGUFError("invalid alignment")
        self.data_offset = -(-c.pos // align) * align
        tensors, extents = [], []
        for name, shape, qtype, offset in entries:
            count = 1
            for dim in shape:
                count *= dim
            per_block, block_bytes = QUANT_BLOCK_SIZES[int(qtype)]
            if count % per_block:
                raise GGUFError(f"invalid {qtype.name} element count for {name}")
            nbytes = count // per_block * block_bytes
            start = self.data_offset + offset
            if start + nbytes > self.file_size:
                raise GGUFError(f"tensor outside file: {name}")
            extents.append((start, start + nbytes, name))
            tensors.append(TensorInfo(name, shape, qtype, offset, start, count, nbytes))
        extents.sort()
        for (_, end, a), (start, _, b) in zip(extents, extents[1:]):
            if end > start:
                raise GGUFError(f"overlapping tensors: {a}, {b}")
        self.tensors = tuple(tensors)
        self._by_name = {t.name: t for t in tensors}

    def tensor(self, name: str) -> TensorInfo:
        return self._by_name[name]

    def analysis(self) -> dict:
        """Summary of the file: source, metadata (long arrays elided), totals, per-type
        tensor/parameter/byte counts and every tensor's extent."""
        dist = defaultdict(lambda: {"tensor_count": 0, "parameter_count": 0, "byte_count": 0})
        for t in self.tensors:
            row = dist[t.quantization_type.name]
            row["tensor_count"] += 1
            row["parameter_count"] += t.num_elements
            row["byte_count"] += t.num_bytes
        meta = {k: ({"kind": "array", "length": len(v)} if isinstance(v, list) and len(v) > 256 else v)
                for k, v in self.metadata.items()}
        return {
            "schema_version": 1,
            "source": {"path": str(self.path), "file_size": self.file_size, "gguf_version": self.version,
                       "data_offset": self.data_offset},
            "metadata": meta,
            "summary": {"total_tensors": len(self.tensors),
                        "total_parameters": sum(t.num_elements for t in self.tensors),
                        "total_tensor_bytes": sum(t.num_bytes for t in self.tensors)},
            "quantization_distribution": dict(sorted(dist.items())),
            "tensors": [t.as_dict() for t in self.tensors],
        }


class GGUFModelAnalyzer:
    @staticmethod
    def parse(model_path) -> dict:
        return GGUFReader(model_path).analysis()


def write_analysis(model_path, output_path) -> dict:
    result = GGUFReader(model_path).analysis()
    Path(output_path).write_text(json.dumps(result, ensure_ascii=False, indent=2) + "\n")
    return result


def get_tensor_quant_distribution(model_path) -> dict:
    return {name: row["tensor_count"] for name, row in GGUFReader(model_path).analysis()["quantization_distribution"].items()}


def get_quant_distribution_with_params(model_path) -> dict:
    return GGUFReader(model_path).analysis()["quantization_distribution"]
