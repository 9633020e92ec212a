"""GGUF (v2 / v3) header reader: typed metadata and validated tensor extents.

Stands in for mlx_gsq/gguf/parser.py:45-144 (``GGUFReader``, ``TensorInfo``, ``GGUFError``):
the same public names and fields, and it accepts and rejects the same files (bad magic,
versions other than 2 and 3, repeated metadata keys or tensor names, an alignment that is not
a positive integer, element counts that do not fill whole blocks, payloads outside the file or
overlapping each other). Written from the published GGUF layout:

    "GGUF" | u32 version | u64 n_tensors | u64 n_kv
    n_kv x      ( str key | u32 type | value )
    n_tensors x ( str name | u32 rank | rank x u64 dim (innermost first) | u32 ggml type | u64 offset )
    zero padding to general.alignment (default 32), then the data section; tensor offsets
    count from its start.

Strings are u64 byte length + UTF-8; arrays are u32 item type + u64 count + items. Only the
header pages of the file are touched: it is read through a read-only memory map, numeric arrays
(tokenizer vocabularies run to 10^5 entries) are decoded in bulk with numpy.
"""
from __future__ import annotations

import math
import mmap
import struct
from dataclasses import dataclass
from enum import IntEnum
from pathlib import Path

import numpy as np

from .parser import GGMLQuantizationType, QUANT_BLOCK_SIZES

MAGIC = b"GGUF"
SUPPORTED_VERSIONS = (2, 3)
DEFAULT_ALIGNMENT = 32


class GGUFError(ValueError):
    """A file that is not a well-formed GGUF v2/v3 file."""


class GGUFValueType(IntEnum):
    UINT8 = 0; INT8 = 1; UINT16 = 2; INT16 = 3; UINT32 = 4; INT32 = 5; FLOAT32 = 6
    BOOL = 7; STRING = 8; ARRAY = 9; UINT64 = 10; INT64 = 11; FLOAT64 = 12


# fixed-width value types -> their little-endian numpy dtype
_FIXED = {
    GGUFValueType.UINT8: np.dtype("<u1"), GGUFValueType.INT8: np.dtype("<i1"),
    GGUFValueType.UINT16: np.dtype("<u2"), GGUFValueType.INT16: np.dtype("<i2"),
    GGUFValueType.UINT32: np.dtype("<u4"), GGUFValueType.INT32: np.dtype("<i4"),
    GGUFValueType.FLOAT32: np.dtype("<f4"), GGUFValueType.BOOL: np.dtype("?"),
    GGUFValueType.UINT64: np.dtype("<u8"), GGUFValueType.INT64: np.dtype("<i8"),
    GGUFValueType.FLOAT64: np.dtype("<f8"),
}
_U32 = struct.Struct("<I")
_U64 = struct.Struct("<Q")


@dataclass(frozen=True)
class TensorInfo:
    """One tensor's directory entry. ``shape`` is GGUF order (innermost first);
    ``absolute_offset`` is the file offset of its first payload byte."""
    name: str
    shape: tuple
    quantization_type: GGMLQuantizationType
    offset: int
    absolute_offset: int
    num_elements: int
    num_bytes: int

    def as_dict(self) -> dict:
        """The manifest record of this tensor (the packed container's per-tensor entry)."""
        return dict(name=self.name, gguf_shape=list(self.shape), logical_shape=list(self.shape[::-1]),
                    quantization_type=self.quantization_type.name,
                    quantization_type_id=int(self.quantization_type), offset=self.offset,
                    absolute_offset=self.absolute_offset, num_elements=self.num_elements,
                    num_bytes=self.num_bytes)


class _HeaderBytes:
    """Bounds-checked little-endian decoding at a moving position of a byte buffer."""

    __slots__ = ("mem", "at")

    def __init__(self, mem: memoryview):
        self.mem, self.at = mem, 0

    def _need(self, n: int) -> int:
        start = self.at
        if n < 0 or start + n > len(self.mem):
            raise GGUFError(f"header ends early: {n} bytes wanted at offset {start}, file has {len(self.mem)}")
        self.at = start + n
        return start

    def u32(self) -> int:
        return _U32.unpack_from(self.mem, self._need(4))[0]

    def u64(self) -> int:
        return _U64.unpack_from(self.mem, self._need(8))[0]

    def text(self) -> str:
        n = self.u64()
        start = self._need(n)
        try:
            return str(self.mem[start:start + n], "utf-8")
        except UnicodeDecodeError as e:
            raise GGUFError(f"string at offset {start} is not UTF-8 ({e.reason})") from None

    def fixed(self, kind: GGUFValueType, count: int) -> np.ndarray:
        dt = _FIXED[kind]
        start = self._need(dt.itemsize * count)
        return np.frombuffer(self.mem, dtype=dt, count=count, offset=start)

    def value_type(self) -> GGUFValueType:
        code = self.u32()
        try:
            return GGUFValueType(code)
        except ValueError:
            raise GGUFError(f"unknown metadata value type {code} at offset {self.at - 4}") from None

    def value(self, kind: GGUFValueType):
        if kind in _FIXED:
            return self.fixed(kind, 1)[0].item()
        if kind is GGUFValueType.STRING:
            return self.text()
        item = self.value_type()  # ARRAY
        count = self.u64()
        if item in _FIXED:
            return self.fixed(item, count).tolist()
        return [self.value(item) for _ in range(count)]


class GGUFReader:
    """The validated header of one GGUF file: ``version``, ``metadata`` (key -> Python value),
    ``tensors`` (directory order), ``data_offset`` and ``file_size``."""

    def __init__(self, path):
        self.path = Path(path).expanduser().resolve()
        self.file_size = self.path.stat().st_size
        if self.file_size < len(MAGIC):
            raise GGUFError(f"{self.path.name}: too short for a GGUF file")
        with self.path.open("rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            view = memoryview(mm)
            try:
                self._read_header(_HeaderBytes(view))
            finally:
                view.release()
        self._by_name = {t.name: t for t in self.tensors}

    def _read_header(self, h: _HeaderBytes) -> None:
        if bytes(h.mem[:4]) != MAGIC:
            raise GGUFError(f"{self.path.name}: no GGUF magic")
        h.at = 4
        self.version = h.u32()
        if self.version not in SUPPORTED_VERSIONS:
            raise GGUFError(f"GGUF version {self.version} is not supported (2 and 3 are)")
        n_tensors, n_kv = h.u64(), h.u64()
        meta: dict = {}
        for _ in range(n_kv):
            key = h.text()
            if key in meta:
                raise GGUFError(f"metadata key {key!r} appears twice")
            meta[key] = h.value(h.value_type())
        self.metadata = meta
        directory = []
        for _ in range(n_tensors):
            name = h.text()
            dims = tuple(h.fixed(GGUFValueType.UINT64, h.u32()).tolist())
            code = h.u32()
            try:
                qtype = GGMLQuantizationType(code)
            except ValueError:
                raise GGUFError(f"tensor {name!r} has unknown GGML type {code}") from None
            directory.append((name, dims, qtype, h.u64()))
        align = meta.get("general.alignment", DEFAULT_ALIGNMENT)
        if not isinstance(align, int) or align <= 0:
            raise GGUFError(f"general.alignment must be a positive integer, not {align!r}")
        self.data_offset = -(-h.at // align) * align
        self.tensors = tuple(self._place(directory))

    def _place(self, directory):
        """TensorInfo per directory entry; every payload whole, inside the file, and disjoint."""
        names = set()
        placed = []
        for name, dims, qtype, rel in directory:
            if name in names:
                raise GGUFError(f"tensor name {name!r} appears twice")
            names.add(name)
            count = math.prod(dims)
            per_block, block_bytes = QUANT_BLOCK_SIZES[int(qtype)]
            blocks, rest = divmod(count, per_block)
            if rest:
                raise GGUFError(f"tensor {name!r}: {count} elements do not fill whole {qtype.name} blocks "
                                f"of {per_block}")
            start = self.data_offset + rel
            nbytes = blocks * block_bytes
            if start + nbytes > self.file_size:
                raise GGUFError(f"tensor {name!r}: bytes [{start}, {start + nbytes}) run past the end of "
                                f"the file ({self.file_size})")
            placed.append(TensorInfo(name, dims, qtype, rel, start, count, nbytes))
        # disjoint payloads: in start order, no payload begins before every earlier one has ended
        reach, holder = -1, None
        for t in sorted(placed, key=lambda t: (t.absolute_offset, t.num_bytes)):
            if t.absolute_offset < reach:
                raise GGUFError(f"tensors {holder!r} and {t.name!r} share payload bytes")
            if t.absolute_offset + t.num_bytes > reach:
                reach, holder = t.absolute_offset + t.num_bytes, t.name
        return placed

    def tensor(self, name: str) -> TensorInfo:
        return self._by_name[name]
