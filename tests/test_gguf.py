"""GGUF reader and lossless converter (CPU).

Mirrors the reference's tests/test_gguf.py:14-39 (tiny file parse + lossless convert, bad
magic) and adds the reader's other checks, typed metadata, the container's exact header
layout, a mixed quantized file converted, verified, tampered with and loaded back through
PackedModelStore, and that a failed or interrupted conversion leaves no file behind.
"""
import json
import struct

import numpy as np
import pytest
import torch

from mlx_gsq_amd.gguf import (GGUFError, GGUFReader, convert_gguf_to_mlx, convert_gguf_to_safetensors,
                              verify_conversion)
from mlx_gsq_amd.gguf import container, converter
from mlx_gsq_amd.runtime import PackedModelStore


def _str(s):
    raw = s.encode()
    return struct.pack("<Q", len(raw)) + raw


def _value(kind, v):
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
    if kind in fmt:
        return struct.pack(fmt[kind], v)
    if kind == 8:
        return _str(v)
    sub, items = v  # array
    return struct.pack("<IQ", sub, len(items)) + b"".join(_value(sub, i) for i in items)


def write_gguf(path, metadata, tensors, version=3, alignment=32, offsets=None):
    """metadata: [(key, type, value)]; tensors: [(name, gguf_shape, type_id, payload bytes)].
    Payloads are placed one after another, each at an aligned offset, unless `offsets` says."""
    raw = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata)))
    for key, kind, value in metadata:
        raw += _str(key) + struct.pack("<I", kind) + _value(kind, value)
    cursor, placed = 0, []
    for i, (name, shape, tid, payload) in enumerate(tensors):
        off = offsets[i] if offsets else cursor
        raw += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        raw += struct.pack("<IQ", tid, off)
        placed.append((off, payload))
        cursor = -(-(off + len(payload)) // alignment) * alignment
    raw += bytes(-len(raw) % alignment)
    base = len(raw)
    data = bytearray()
    for off, payload in placed:
        if len(data) < off + len(payload):
            data += bytes(off + len(payload) - len(data))
        data[off:off + len(payload)] = payload
    path.write_bytes(bytes(raw) + bytes(data))
    return base


def test_parse_and_lossless_convert(tmp_path):
    src, out = tmp_path / "tiny.gguf", tmp_path / "tiny.safetensors"
    write_gguf(src, [("general.architecture", 8, "test"), ("general.alignment", 4, 32)],
               [("weight", (2, 2), 0, struct.pack("<ffff", 1, 2, 3, 4))])
    t = GGUFReader(src).tensor("weight")
    assert t.shape == (2, 2) and t.num_bytes == 16 and t.quantization_type.name == "F32"
    convert_gguf_to_safetensors(src, out)
    with out.open("rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        assert n % 8 == 0
        header = json.loads(f.read(n))
        payload = f.read()
    assert header["weight"] == {"dtype": "U8", "shape": [16], "data_offsets": [0, 16]}
    assert header["__metadata__"]["format"] == "mlx-gsq-packed-v1"
    assert payload == struct.pack("<ffff", 1, 2, 3, 4)
    with pytest.raises(FileExistsError):
        convert_gguf_to_safetensors(src, out)


def test_bad_magic(tmp_path):
    p = tmp_path / "bad"
    p.write_bytes(b"bad")
    with pytest.raises(GGUFError):
        GGUFReader(p)


@pytest.mark.parametrize("case", ["version", "dup_key", "dup_tensor", "alignment", "outside", "overlap",
                                  "partial_block", "truncated", "unknown_type"])
def test_reader_rejects(tmp_path, case):
    p = tmp_path / f"{case}.gguf"
    f32 = struct.pack("<ffff", 1, 2, 3, 4)
    meta = [("general.architecture", 8, "t")]
    tens = [("a", (4,), 0, f32)]
    kw = {}
    if case == "version":
        kw["version"] = 1
    elif case == "dup_key":
        meta = meta + [("general.architecture", 8, "u")]
    elif case == "dup_tensor":
        tens = tens + [("a", (4,), 0, f32)]
    elif case == "alignment":
        meta = meta + [("general.alignment", 4, 0)]
    elif case == "overlap":
        tens = tens + [("b", (4,), 0, f32)]
        kw["offsets"] = [0, 8]
    elif case == "partial_block":
        tens = [("q", (100,), 22, bytes(82))]  # IQ2_S blocks hold 256 elements
    elif case == "unknown_type":
        tens = [("q", (4,), 5, f32)]  # GGML type 5 does not exist
    write_gguf(p, meta, tens, **kw)
    if case == "outside":
        p.write_bytes(p.read_bytes()[:-4])
    if case == "truncated":
        p.write_bytes(p.read_bytes()[:30])
    with pytest.raises(GGUFError):
        GGUFReader(p)


def test_metadata_types(tmp_path):
    p = tmp_path / "m.gguf"
    meta = [("general.architecture", 8, "qwen35"), ("general.name", 8, "tiny"), ("u8", 0, 7), ("i8", 1, -3),
            ("u16", 2, 700), ("i16", 3, -700), ("u32", 4, 70000), ("i32", 5, -70000), ("f32", 6, 0.5),
            ("flag", 7, True), ("u64", 10, 1 << 40), ("i64", 11, -(1 << 40)), ("f64", 12, 0.25),
            ("ids", 9, (4, [1, 2, 3])), ("names", 9, (8, ["x", "yz"])), ("long", 9, (5, list(range(300)))),
            ("nested", 9, (9, [(4, [1, 2]), (8, ["a"])])), ("empty", 9, (6, [])),
            ("general.alignment", 4, 64)]
    write_gguf(p, meta, [("w", (256, 2), 12, bytes(2 * 144)), ("n", (8,), 0, bytes(32))], alignment=64)
    r = GGUFReader(p)
    assert r.version == 3 and r.data_offset % 64 == 0
    assert r.metadata["i16"] == -700 and r.metadata["flag"] is True and r.metadata["names"] == ["x", "yz"]
    assert r.metadata["ids"] == [1, 2, 3] and r.metadata["f64"] == 0.25 and r.metadata["i64"] == -(1 << 40)
    assert r.metadata["u64"] == 1 << 40 and r.metadata["f32"] == 0.5 and r.metadata["long"] == list(range(300))
    assert r.metadata["nested"] == [[1, 2], ["a"]] and r.metadata["empty"] == []
    assert all(type(v) is int for v in r.metadata["long"])
    w = r.tensor("w").as_dict()
    assert w == {"name": "w", "gguf_shape": [256, 2], "logical_shape": [2, 256], "quantization_type": "Q4_K",
                 "quantization_type_id": 12, "offset": 0, "absolute_offset": r.data_offset, "num_elements": 512,
                 "num_bytes": 288}
    assert r.tensor("n").offset == 320 and r.tensor("n").absolute_offset == r.data_offset + 320


def test_overlap_past_a_neighbour(tmp_path):
    """Payloads that start inside an earlier one are refused; back to back ones are not."""
    p = tmp_path / "o.gguf"
    write_gguf(p, [], [("big", (64,), 0, bytes(256)), ("mid", (4,), 0, bytes(16)), ("late", (4,), 0, bytes(16))],
               offsets=[0, 32, 128])
    with pytest.raises(GGUFError, match="share payload bytes"):
        GGUFReader(p)
    # back to back and zero-sized tensors at a boundary are fine
    write_gguf(p, [], [("a", (4,), 0, bytes(16)), ("z", (0,), 0, b""), ("b", (4,), 0, bytes(16))],
               offsets=[0, 16, 16])
    assert [t.num_bytes for t in GGUFReader(p).tensors] == [16, 0, 16]


def test_container_header_layout(tmp_path):
    """The exact header the store (and the reference's store) reads."""
    src, out = tmp_path / "h.gguf", tmp_path / "h.safetensors"
    write_gguf(src, [("general.architecture", 8, "qwen35")],
               [("blk.0.q", (512, 3), 17, bytes(3 * 2 * 74)), ("norm", (5,), 0, bytes(20))])
    convert_gguf_to_safetensors(src, out)
    header, start = container.read_header(out)
    assert (start - 8) % 8 == 0
    meta = header.pop("__metadata__")
    assert {k: v for k, v in meta.items() if k != "note"} == {
        "format": "mlx-gsq-packed-v1", "source_format": "GGUF", "architecture": "qwen35",
        "tensor_quantization": json.dumps({
            "blk.0.q": {"qtype": "IQ2_XS", "qtype_id": 17, "gguf_shape": [512, 3], "logical_shape": [3, 512],
                        "num_elements": 1536, "block_elements": 256, "block_bytes": 74},
            "norm": {"qtype": "F32", "qtype_id": 0, "gguf_shape": [5], "logical_shape": [5], "num_elements": 5,
                     "block_elements": 1, "block_bytes": 4}}, separators=(",", ":"))}
    assert header == {"blk.0.q": {"dtype": "U8", "shape": [444], "data_offsets": [0, 444]},
                      "norm": {"dtype": "U8", "shape": [20], "data_offsets": [444, 464]}}
    assert out.stat().st_size == start + 464


def test_mixed_model_convert_verify_load(tmp_path):
    rng = np.random.default_rng(3)
    emb = rng.integers(0, 256, 8 * 2 * 82, dtype=np.uint8).tobytes()      # IQ2_S 8 x 512
    w4 = rng.integers(0, 256, 4 * 144, dtype=np.uint8).tobytes()          # Q4_K 4 x 256
    norm = np.arange(256, dtype=np.float32).tobytes()
    src, out = tmp_path / "m.gguf", tmp_path / "model-packed.safetensors"
    write_gguf(src, [("general.architecture", 8, "qwen35"), ("general.name", 8, "mix")],
               [("token_embd.weight", (512, 8), 22, emb), ("blk.0.w", (256, 4), 12, w4), ("norm", (256,), 0, norm)])
    convert_gguf_to_safetensors(src, out)
    manifest = json.loads((tmp_path / "model-packed.safetensors.manifest.json").read_text())
    assert manifest["verification"]["status"] == "passed" and manifest["tensor_count"] == 3
    store = PackedModelStore(out, device="cpu")
    e = store.weight("token_embd.weight")
    assert e.quantization_type == "IQ2_S" and e.logical_shape == (8, 512) and bytes(e.data.numpy()) == emb
    q = store.weight("blk.0.w")
    assert q.quantization_type_id == 12 and bytes(q.data.numpy()) == w4
    assert torch.equal(store.materialize_plain("norm"), torch.arange(256, dtype=torch.float32))
    # without the sidecar the embedded tensor_quantization map describes the same tensors
    (tmp_path / "model-packed.safetensors.manifest.json").unlink()
    assert PackedModelStore(out, device="cpu").weight("blk.0.w").logical_shape == (4, 256)
    # one changed byte in the container fails verification
    raw = bytearray(out.read_bytes())
    raw[-100] ^= 0xFF
    out.write_bytes(bytes(raw))
    convert_gguf_to_mlx(src, tmp_path / "again")
    with pytest.raises(ValueError, match="is not the GGUF payload"):
        verify_conversion(src, out, tmp_path / "again" / "model-packed.safetensors.manifest.json")


def test_failed_conversion_leaves_nothing(tmp_path, monkeypatch):
    src, out = tmp_path / "f.gguf", tmp_path / "f.safetensors"
    write_gguf(src, [("general.architecture", 8, "t")], [("w", (4,), 0, struct.pack("<ffff", 1, 2, 3, 4))])

    def corrupt(path, reader):  # the written container reads back different
        return {t.name: "0" * 64 for t in reader.tensors}
    monkeypatch.setattr(converter, "_container_digests", corrupt)
    with pytest.raises(ValueError, match="is not the GGUF payload"):
        convert_gguf_to_safetensors(src, out)
    assert sorted(p.name for p in tmp_path.iterdir()) == ["f.gguf"]
    monkeypatch.undo()

    def interrupted(*a, **k):  # the copy stops part way
        raise KeyboardInterrupt
    monkeypatch.setattr(converter.hashlib, "sha256", interrupted)
    with pytest.raises(KeyboardInterrupt):
        convert_gguf_to_safetensors(src, out)
    assert sorted(p.name for p in tmp_path.iterdir()) == ["f.gguf"]


def test_overwrite_and_manifest_check(tmp_path):
    src, out = tmp_path / "v.gguf", tmp_path / "v.safetensors"
    write_gguf(src, [("general.architecture", 8, "t"), ("general.name", 8, "one")],
               [("w", (4,), 0, struct.pack("<ffff", 1, 2, 3, 4))])
    convert_gguf_to_safetensors(src, out, verify=False)
    mpath = tmp_path / "v.safetensors.manifest.json"
    m = json.loads(mpath.read_text())
    assert "verification" not in m and m["source"]["name"] == "one" and m["container"] == "v.safetensors"
    rec = verify_conversion(src, out, record_hashes=True)
    assert rec["status"] == "passed" and rec["tensor_hashes"]["w"] == __import__("hashlib").sha256(
        struct.pack("<ffff", 1, 2, 3, 4)).hexdigest()
    assert json.loads(mpath.read_text())["verification"] == rec
    # a manifest whose record disagrees with the GGUF directory fails verification
    m = json.loads(mpath.read_text())
    m["tensors"]["w"]["num_elements"] = 5
    mpath.write_text(json.dumps(m))
    with pytest.raises(ValueError, match="num_elements"):
        verify_conversion(src, out)
    # a new source over the old container: refused without overwrite, replaced with it
    write_gguf(src, [("general.architecture", 8, "t")], [("w", (4,), 0, struct.pack("<ffff", 5, 6, 7, 8))])
    with pytest.raises(FileExistsError):
        convert_gguf_to_safetensors(src, out)
    convert_gguf_to_safetensors(src, out, overwrite=True)
    assert out.read_bytes().endswith(struct.pack("<ffff", 5, 6, 7, 8))
    assert verify_conversion(src, out)["tensor_count"] == 1
