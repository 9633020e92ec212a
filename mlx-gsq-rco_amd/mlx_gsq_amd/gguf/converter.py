"""GGUF -> packed container conversion, lossless and verified by SHA-256.

Stands in for mlx_gsq/gguf/converter.py:59-186 (``convert_gguf_to_safetensors``,
``verify_conversion``, ``convert_gguf_to_mlx``; same arguments, return values, sidecar
manifest and exception types). The container layout is in ``container.py``.

How it works here:

* One read of the source. Each tensor's payload is copied from a read-only memory map of the
  GGUF file into the container and hashed in the same pass; verification then re-reads only
  the written container and compares its per-tensor digests with those of the copy.
* Nothing half-written is left in place. The container and the sidecar manifest are written
  to temporary files beside their targets, flushed to disk, and renamed over the targets only
  when complete (and, with verification on, checked): a failed conversion leaves no container
  and no stale manifest of its own.
* ``verify_conversion`` on its own hashes the source ranges and the container's tensors over a
  thread pool (``hashlib`` releases the GIL on large buffers).

The sidecar ``<container>.manifest.json`` holds ``format``, ``container`` (file name),
``source`` (path, file_size, gguf_version, architecture, name), ``tensor_count``, ``tensors``
(name -> the reader's ``TensorInfo.as_dict()``) and, after verification, ``verification``
(algorithm, status, tensor_count, all_packed_bytes_identical, tensor_hashes).
"""
from __future__ import annotations

import contextlib
import hashlib
import json
import mmap
import os
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

from . import container
from .reader import GGUFReader

FORMAT = container.FORMAT
CHUNK = 64 * 1024 * 1024  # bytes per write and per hash update
_HASH_THREADS = max(1, min(8, os.cpu_count() or 1))


def _sidecar(output: Path) -> Path:
    return output.with_name(output.name + ".manifest.json")


@contextlib.contextmanager
def _replace_when_done(target: Path):
    """Yield a temporary path beside ``target``; on a clean exit it is renamed over ``target``,
    on any exception (KeyboardInterrupt included) it is deleted."""
    fd, tmp = tempfile.mkstemp(dir=target.parent, prefix=f".{target.name}.", suffix=".tmp")
    os.close(fd)
    tmp = Path(tmp)
    try:
        yield tmp
        os.replace(tmp, target)
    finally:
        if tmp.exists():
            tmp.unlink()


def _write_json(path: Path, doc: dict) -> None:
    with _replace_when_done(path) as tmp:
        tmp.write_text(json.dumps(doc, ensure_ascii=False, indent=2) + "\n")


def _open_map(path: Path):
    """Read-only map of a whole file (an empty file maps to an empty bytes object)."""
    if path.stat().st_size == 0:
        return contextlib.nullcontext(b"")
    f = path.open("rb")
    try:
        return mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    finally:
        f.close()  # the map keeps its own reference to the file


def _digest(buf, start: int, size: int) -> str:
    h = hashlib.sha256()
    with memoryview(buf) as mv:
        for at in range(start, start + size, CHUNK):
            with mv[at:min(at + CHUNK, start + size)] as part:
                h.update(part)
    return h.hexdigest()


def _digests(path: Path, ranges) -> list:
    """SHA-256 hex digest of each (offset, size) range of ``path``; ranges past the end of the
    file raise ValueError."""
    size = path.stat().st_size
    for start, n in ranges:
        if start < 0 or start + n > size:
            raise ValueError(f"{path.name}: range [{start}, {start + n}) lies past the end of the file ({size})")
    with _open_map(path) as buf:
        with ThreadPoolExecutor(_HASH_THREADS) as pool:
            return list(pool.map(lambda r: _digest(buf, *r), ranges))


def _container_digests(path: Path, reader: GGUFReader) -> dict:
    """Check the container's layout against the GGUF directory, then hash its tensors."""
    header, data_start = container.read_header(path)
    expected = data_start + sum(t.num_bytes for t in reader.tensors)
    actual = path.stat().st_size
    if actual != expected:
        raise ValueError(f"{path.name} holds {actual} bytes; its GGUF tensors need {expected}")
    ranges = []
    for t in reader.tensors:
        entry = header.get(t.name)
        if not isinstance(entry, dict) or entry.get("dtype") != "U8" or entry.get("shape") != [t.num_bytes]:
            raise ValueError(f"{path.name}: tensor {t.name!r} is missing or is not U8[{t.num_bytes}]")
        lo, hi = entry.get("data_offsets", (0, -1))
        if hi - lo != t.num_bytes:
            raise ValueError(f"{path.name}: tensor {t.name!r} has data offsets {lo}..{hi}")
        ranges.append((data_start + lo, t.num_bytes))
    return dict(zip((t.name for t in reader.tensors), _digests(path, ranges)))


def _compare(reader: GGUFReader, want: dict, got: dict) -> None:
    for t in reader.tensors:
        if want[t.name] != got[t.name]:
            raise ValueError(f"payload of {t.name!r} in the container is not the GGUF payload "
                             f"(sha256 {got[t.name][:16]}… vs {want[t.name][:16]}…)")


def _record(digests: dict) -> dict:
    return {"algorithm": "sha256", "status": "passed", "tensor_count": len(digests),
            "all_packed_bytes_identical": True, "tensor_hashes": dict(digests)}


def build_manifest(reader: GGUFReader, output_name: str) -> dict:
    """The sidecar manifest of a container named ``output_name`` converted from ``reader``."""
    meta = reader.metadata
    return {
        "format": FORMAT,
        "container": output_name,
        "source": {"path": str(reader.path), "file_size": reader.file_size, "gguf_version": reader.version,
                   "architecture": meta.get("general.architecture"), "name": meta.get("general.name")},
        "tensor_count": len(reader.tensors),
        "tensors": {t.name: t.as_dict() for t in reader.tensors},
    }


def convert_gguf_to_safetensors(input_path, output_path, *, overwrite: bool = False, verify: bool = True) -> Path:
    """Copy every tensor of a GGUF file, byte for byte, into a packed container at
    ``output_path`` and write its sidecar manifest; return the container's resolved path.
    Raises FileExistsError if the container exists and ``overwrite`` is false, GGUFError for a
    malformed source and ValueError if verification finds a difference."""
    reader = GGUFReader(input_path)
    out = Path(output_path).expanduser().resolve()
    if out.exists() and not overwrite:
        raise FileExistsError(out)
    out.parent.mkdir(parents=True, exist_ok=True)
    header = container.build_header(reader.tensors, str(reader.metadata.get("general.architecture", "")))
    copied = {}
    with _replace_when_done(out) as tmp:
        with _open_map(reader.path) as src, tmp.open("wb") as dst:
            dst.write(header)
            with memoryview(src) as mv:
                for t in reader.tensors:
                    h = hashlib.sha256()
                    for at in range(t.absolute_offset, t.absolute_offset + t.num_bytes, CHUNK):
                        with mv[at:min(at + CHUNK, t.absolute_offset + t.num_bytes)] as part:
                            h.update(part)
                            dst.write(part)
                    copied[t.name] = h.hexdigest()
            dst.flush()
            os.fsync(dst.fileno())
        if verify:
            _compare(reader, copied, _container_digests(tmp, reader))
    manifest = build_manifest(reader, out.name)
    if verify:
        manifest["verification"] = _record(copied)
    _write_json(_sidecar(out), manifest)
    return out


def verify_conversion(input_path, output_path, manifest_path=None, *, record_hashes: bool = False) -> dict:
    """Check a container against its GGUF source: layout, every tensor's SHA-256, and the
    manifest's tensor records. Returns the verification record (and stores it in the manifest
    when ``record_hashes``); raises ValueError on the first difference."""
    reader = GGUFReader(input_path)
    out = Path(output_path)
    mpath = Path(manifest_path) if manifest_path else _sidecar(out)
    manifest = json.loads(mpath.read_text())
    source = dict(zip((t.name for t in reader.tensors),
                      _digests(reader.path, [(t.absolute_offset, t.num_bytes) for t in reader.tensors])))
    _compare(reader, source, _container_digests(out, reader))
    recorded = manifest.get("tensors", {})
    for t in reader.tensors:
        want = t.as_dict()
        have = recorded.get(t.name) or {}
        wrong = sorted(k for k, v in want.items() if have.get(k) != v)
        if wrong:
            raise ValueError(f"{mpath.name}: record of {t.name!r} disagrees with the GGUF file on {', '.join(wrong)}")
    result = _record(source)
    if record_hashes:
        manifest["verification"] = result
        _write_json(mpath, manifest)
    return result


def convert_gguf_to_mlx(input_path, output_dir=".", overwrite: bool = False) -> bool:
    """Convert into ``<output_dir>/model-packed.safetensors`` (the reference's old entry point);
    True on success, exceptions as ``convert_gguf_to_safetensors``."""
    convert_gguf_to_safetensors(input_path, Path(output_dir) / "model-packed.safetensors", overwrite=overwrite)
    return True
