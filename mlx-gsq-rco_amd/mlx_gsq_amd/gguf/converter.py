"""Lossless GGUF -> "mlx-gsq-packed-v1" Safetensors conversion and its SHA-256 verification.

Counterpart of mlx_gsq/gguf/converter.py:22-186 with the same public names and container:
every GGUF tensor becomes a 1-D U8 Safetensors tensor holding its untouched packed bytes (no
dequantization), the header's ``__metadata__`` carries ``format``, ``source_format``,
``architecture``, ``note`` and the compact JSON ``tensor_quantization`` map (qtype, qtype_id,
gguf_shape, logical_shape = reversed, num_elements, block_elements, block_bytes), the header
is padded with spaces to 8 bytes, and a sidecar ``<file>.manifest.json`` records the source
and every tensor's extent (plus the verification hashes). The container is written to a
``.partial`` file and renamed only when complete.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
from pathlib import Path

from .parser import QUANT_BLOCK_SIZES
from .reader import GGUFReader

FORMAT = "mlx-gsq-packed-v1"
COPY_CHUNK_SIZE = 16 * 1024 * 1024


def _container_header(reader: GGUFReader) -> bytes:
    quant = {}
    entries = {}
    cursor = 0
    for t in reader.tensors:
        per_block, block_bytes = QUANT_BLOCK_SIZES[int(t.quantization_type)]
        quant[t.name] = {"qtype": t.quantization_type.name, "qtype_id": int(t.quantization_type),
                         "gguf_shape": list(t.shape), "logical_shape": list(reversed(t.shape)),
                         "num_elements": t.num_elements, "block_elements": per_block, "block_bytes": block_bytes}
        entries[t.name] = {"dtype": "U8", "shape": [t.num_bytes], "data_offsets": [cursor, cursor + t.num_bytes]}
        cursor += t.num_bytes
    header = {"__metadata__": {
        "format": FORMAT,
        "source_format": "GGUF",
        "architecture": str(reader.metadata.get("general.architecture", "")),
        "note": "U8 tensors contain original GGUF packed bytes; custom kernels required",
        "tensor_quantization": json.dumps(quant, separators=(",", ":")),
    }}
    header.update(entries)
    raw = json.dumps(header, ensure_ascii=False, separators=(",", ":")).encode("utf-8")
    return raw + b" " * (-len(raw) % 8)


def build_manifest(reader: GGUFReader, output_name: str) -> dict:
    return {
        "format": FORMAT,
        "container": output_name,
        "source": {"path": str(reader.path), "file_size": reader.file_size, "gguf_version": reader.version,
                   "architecture": reader.metadata.get("general.architecture"),
                   "name": reader.metadata.get("general.name")},
        "tensor_count": len(reader.tensors),
        "tensors": {t.name: t.as_dict() for t in reader.tensors},
    }


def _manifest_path(output: Path) -> Path:
    return output.with_suffix(output.suffix + ".manifest.json")


def _copy(src, dst, offset: int, size: int, name: str) -> None:
    src.seek(offset)
    left = size
    while left:
        chunk = src.read(min(left, COPY_CHUNK_SIZE))
        if not chunk:
            raise IOError(f"short GGUF read for {name}")
        dst.write(chunk)
        left -= len(chunk)


def convert_gguf_to_safetensors(input_path, output_path, *, overwrite: bool = False, verify: bool = True) -> Path:
    """Stream the packed tensors of a GGUF file into a Safetensors container (see module doc);
    with ``verify`` the result is checked tensor by tensor against the GGUF byte ranges and the
    hashes are recorded in the manifest."""
    reader = GGUFReader(input_path)
    output = Path(output_path).expanduser().resolve()
    if output.exists() and not overwrite:
        raise FileExistsError(output)
    output.parent.mkdir(parents=True, exist_ok=True)
    partial = output.with_suffix(output.suffix + ".partial")
    if partial.exists():
        partial.unlink()
    header = _container_header(reader)
    try:
        with reader.path.open("rb") as src, partial.open("xb") as dst:
            dst.write(struct.pack("<Q", len(header)))
            dst.write(header)
            for t in reader.tensors:
                _copy(src, dst, t.absolute_offset, t.num_bytes, t.name)
            dst.flush()
            os.fsync(dst.fileno())
        partial.replace(output)
        mpath = _manifest_path(output)
        mpath.write_text(json.dumps(build_manifest(reader, output.name), ensure_ascii=False, indent=2) + "\n")
        if verify:
            verify_conversion(reader.path, output, mpath, record_hashes=True)
    except BaseException:
        if partial.exists():
            partial.unlink()
        raise
    return output


def _sha256(f, offset: int, size: int) -> str:
    h = hashlib.sha256()
    f.seek(offset)
    left = size
    while left:
        chunk = f.read(min(left, COPY_CHUNK_SIZE))
        if not chunk:
            raise IOError("short read during verification")
        h.update(chunk)
        left -= len(chunk)
    return h.hexdigest()


def verify_conversion(input_path, output_path, manifest_path=None, *, record_hashes: bool = False) -> dict:
    """Check the container's size, every entry (U8, one dimension of the tensor's byte count),
    the manifest's tensor records and the SHA-256 of every tensor's bytes against the GGUF
    source; raises ValueError on the first difference."""
    reader = GGUFReader(input_path)
    output = Path(output_path)
    mpath = Path(manifest_path) if manifest_path else _manifest_path(output)
    manifest = json.loads(mpath.read_text())
    hashes = {}
    with output.open("rb") as packed, reader.path.open("rb") as src:
        header_len = struct.unpack("<Q", packed.read(8))[0]
        header = json.loads(packed.read(header_len))
        base = 8 + header_len
        want_size = base + sum(t.num_bytes for t in reader.tensors)
        if output.stat().st_size != want_size:
            raise ValueError(f"safetensors size mismatch: {output.stat().st_size} != {want_size}")
        for t in reader.tensors:
            entry = header.get(t.name)
            if not entry or entry["dtype"] != "U8" or entry["shape"] != [t.num_bytes]:
                raise ValueError(f"invalid safetensors entry for {t.name}")
            start, end = entry["data_offsets"]
            digest = _sha256(src, t.absolute_offset, t.num_bytes)
            if _sha256(packed, base + start, end - start) != digest:
                raise ValueError(f"packed bytes differ for {t.name}")
            hashes[t.name] = digest
            rec = manifest["tensors"].get(t.name)
            if not rec or any(rec.get(k) != v for k, v in t.as_dict().items()):
                raise ValueError(f"manifest differs for {t.name}")
    result = {"algorithm": "sha256", "status": "passed", "tensor_count": len(hashes),
              "all_packed_bytes_identical": True, "tensor_hashes": hashes}
    if record_hashes:
        manifest["verification"] = result
        mpath.write_text(json.dumps(manifest, ensure_ascii=False, indent=2) + "\n")
    return result


def convert_gguf_to_mlx(input_path, output_dir=".", overwrite: bool = False) -> bool:
    """Older entry point of the reference: converts into ``<output_dir>/model-packed.safetensors``."""
    convert_gguf_to_safetensors(input_path, Path(output_dir) / "model-packed.safetensors", overwrite=overwrite)
    return True
