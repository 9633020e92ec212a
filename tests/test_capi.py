"""CPU tests of the boundary: libgsq.so loads and exports every symbol include/gsq.h
declares, and the host wrappers raise the reference's exception types and messages
(mlx_gsq/runtime/kernels/qmv.py:539-544, qmm.py:569-579, registry.py:28-46) without
touching a GPU."""
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "gsq.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(gsq_\w+)\s*\(", text, re.M)))


def test_library_exports_header_symbols():
    from mlx_gsq_amd import _lib
    lib = _lib.lib()
    syms = header_symbols()
    assert syms and set(syms) == set(_lib.EXPORTS), syms
    for s in syms:
        assert hasattr(lib, s)
    assert lib.gsq_version() == 1


def test_block_bytes_match_format_table():
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import BLOCK_BYTES, TYPE_IDS
    from mlx_gsq_amd.gguf.parser import QUANT_BLOCK_SIZES
    lib = _lib.lib()
    for q, tid in TYPE_IDS.items():
        assert lib.gsq_block_bytes(tid) == BLOCK_BYTES[q] == QUANT_BLOCK_SIZES[tid][1]
    assert lib.gsq_block_bytes(2) == -1  # Q4_0: not a 256-block type of this path


def test_c_validation_errors_without_gpu():
    from mlx_gsq_amd import _lib
    lib = _lib.lib()
    assert lib.gsq_qmv(12, 2, 4, 1, 8, 0, 1, 4, 300, None) == _lib.GSQ_E_VALUE  # K % 256
    assert b"matrix width" in lib.gsq_last_error()
    assert lib.gsq_qmv(12, 3, 4, 1, 8, 0, 1, 4, 256, None) == _lib.GSQ_E_VALUE  # odd packed address
    assert lib.gsq_qmm(99, 2, 4, 1, 8, 0, 1, 4, 256, None) == _lib.GSQ_E_UNSUPPORTED
    assert lib.gsq_qmm(12, 2, 4, 7, 8, 0, 1, 4, 256, None) == _lib.GSQ_E_TYPE
    assert lib.gsq_dequant(99, 2, 1, 16, None) == _lib.GSQ_E_UNSUPPORTED
    assert lib.gsq_set_tables(12, None, 0, 0, None, 0) == _lib.GSQ_E_VALUE  # Q4_K has no codebook
    g = np.zeros((10, 8), np.float32)
    ks = np.zeros(128, np.uint8)
    assert lib.gsq_set_tables(16, g.ctypes.data, 10, 8, ks.ctypes.data, 128) == _lib.GSQ_E_VALUE
    # a ksigns table other than the published one (entry i = i with bit 7 its parity) is refused:
    # the QMV decoders form the sign bytes from that closed form
    from mlx_gsq_amd import tables
    g = np.zeros((256, 8), np.float32)
    bad = tables.ksigns().copy()
    bad[5] ^= 0x80
    assert lib.gsq_set_tables(16, g.ctypes.data, 256, 8, bad.ctypes.data, 128) == _lib.GSQ_E_VALUE
    assert b"published" in lib.gsq_last_error()
    # the fused-prologue QMV: arguments are checked before anything reaches a device
    # (qtype, packed, pre_op, x, pre_a, pre_w, eps, res_out, x_out, y, y_dtype, N, K,
    #  conv_state, conv_w, conv_rows, conv_kernel, conv_out, stream)
    # (fake device addresses 4 KiB apart: no two vectors of up to 2 x 256 fp16 values overlap)
    ok = dict(qt=12, packed=2, op=1, x=1 << 12, a=2 << 12, w=3 << 12, eps=1e-6, res=4 << 12, xo=5 << 12,
              y=6 << 12, ydt=1, n=4, k=256, cs=7 << 12, cw=8 << 12, cr=0, ck=4, co=9 << 12)

    def pre(**kw):
        v = {**ok, **kw}
        return lib.gsq_qmv_pre(v["qt"], v["packed"], v["op"], v["x"], v["a"], v["w"], v["eps"], v["res"], v["xo"],
                               v["y"], v["ydt"], v["n"], v["k"], v["cs"], v["cw"], v["cr"], v["ck"], v["co"], None)
    assert pre(op=7) == _lib.GSQ_E_VALUE and b"pre_op" in lib.gsq_last_error()
    assert pre(w=None) == _lib.GSQ_E_VALUE and b"norm weight" in lib.gsq_last_error()
    assert pre(eps=-1.0) == _lib.GSQ_E_VALUE
    # an output overlapping an input (or the other output) races with the workgroups that
    # still read it
    x0 = ok["x"]
    assert pre(res=x0) == _lib.GSQ_E_VALUE and b"res_out must not alias" in lib.gsq_last_error()
    assert pre(res=ok["a"] + 256) == _lib.GSQ_E_VALUE and b"res_out must not alias" in lib.gsq_last_error()
    assert pre(xo=x0) == _lib.GSQ_E_VALUE and b"x_out must not alias" in lib.gsq_last_error()
    assert pre(xo=x0 - 496) == _lib.GSQ_E_VALUE and b"x_out must not alias" in lib.gsq_last_error()
    assert pre(xo=ok["a"]) == _lib.GSQ_E_VALUE and b"x_out must not alias" in lib.gsq_last_error()
    assert pre(xo=ok["w"] + 16) == _lib.GSQ_E_VALUE and b"x_out must not alias" in lib.gsq_last_error()
    assert pre(xo=ok["res"] + 16) == _lib.GSQ_E_VALUE and b"res_out and x_out" in lib.gsq_last_error()
    # SWIGLU reads 2K values of x: an x_out in its second half overlaps
    assert pre(op=2, xo=x0 + 512) == _lib.GSQ_E_VALUE and b"x_out must not alias" in lib.gsq_last_error()
    assert pre(x=24) == _lib.GSQ_E_VALUE and b"aligned" in lib.gsq_last_error()
    assert pre(cr=5) == _lib.GSQ_E_VALUE  # more convolution rows than outputs
    assert pre(cr=4, ck=9) == _lib.GSQ_E_VALUE and b"kernel" in lib.gsq_last_error()
    assert pre(cr=4, ydt=0) == _lib.GSQ_E_VALUE and b"fp16 y" in lib.gsq_last_error()
    assert pre(cr=4, co=None) == _lib.GSQ_E_VALUE
    assert pre(k=300) == _lib.GSQ_E_VALUE  # K % 256
    # two products of one row in one launch: checked before anything reaches a device; the
    # outputs must not overlap each other or x (workgroups still read x while others write)
    def group2(y0, y1, x, qt1=23, ydt=0):
        return lib.gsq_qmv_group2(17, 2 << 12, 4, y0, qt1, 4 << 12, 4, y1, x, ydt, 256, None)
    assert group2(6 << 12, 6 << 12, 8 << 12) == _lib.GSQ_E_VALUE and b"must not overlap" in lib.gsq_last_error()
    assert group2(6 << 12, (6 << 12) + 8, 8 << 12) == _lib.GSQ_E_VALUE  # 4 fp32 outputs: 16 bytes
    assert group2(6 << 12, 7 << 12, (7 << 12) - 256) == _lib.GSQ_E_VALUE  # x (512 bytes) reaches y1
    assert group2(6 << 12, 7 << 12, None) == _lib.GSQ_E_VALUE and b"NULL" in lib.gsq_last_error()
    assert group2(6 << 12, 7 << 12, 8 << 12, qt1=99) == _lib.GSQ_E_UNSUPPORTED
    assert group2(6 << 12, 7 << 12, 8 << 12, ydt=5) == _lib.GSQ_E_TYPE
    # the decode-step kernels
    assert lib.gsq_add_rms_norm(16, None, 32, 48, 1, 12, 1e-6, 1, None) == _lib.GSQ_E_VALUE  # dim % 8
    assert lib.gsq_add_rms_norm(16, None, 32, 48, 1, 16, 1e-6, 5, None) == _lib.GSQ_E_TYPE
    assert lib.gsq_swiglu(16, 32, 1, 0, 1, None) == _lib.GSQ_E_VALUE


def test_python_validation_mirrors_reference():
    from mlx_gsq_amd.runtime.kernels import decode, decode_weight, quantized_matmul, quantized_matvec
    from mlx_gsq_amd.runtime.store import PackedWeight
    x = torch.zeros(1, 512, dtype=torch.float16)
    p = torch.zeros(2 * 2 * 144, dtype=torch.uint8)
    with pytest.raises(ValueError, match="invalid Q4_K matrix width"):
        quantized_matvec(torch.zeros(1, 300), p, qtype="Q4_K", out_features=2, in_features=300)
    with pytest.raises(ValueError, match="packed size"):
        quantized_matvec(x, p[:-1], qtype="Q4_K", out_features=2, in_features=512)
    with pytest.raises(ValueError, match="input feature size mismatch"):
        quantized_matvec(torch.zeros(1, 256), p, qtype="Q4_K", out_features=2, in_features=512)
    with pytest.raises(KeyError):
        quantized_matvec(x, p, qtype="NOPE", out_features=2, in_features=512)
    with pytest.raises(KeyError):  # a 256-block GGML type with no kernel (reference: KeyError)
        quantized_matvec(x, torch.zeros(2 * 2 * 176, dtype=torch.uint8), qtype="Q5_K", out_features=2, in_features=512)
    with pytest.raises(NotImplementedError, match="no tiled QMM kernel"):
        quantized_matmul(x, p, qtype="Q5_K", out_features=2, in_features=512)
    with pytest.raises(NotImplementedError):
        decode(p, "Q5_K")
    with pytest.raises(TypeError):
        decode(p.to(torch.int8), "Q4_K")
    with pytest.raises(ValueError, match="not block aligned"):
        decode(p[:-1], "Q4_K")
    w = PackedWeight("t", p, (512, 2), (2, 512), "F16", 1, 1024, 576)
    with pytest.raises(TypeError, match="not a supported quantized weight"):
        decode_weight(w)


def test_embedding_validation_mirrors_reference():
    """embedding.py:30-33 and nn/embedding.py:6 checks, before any device work."""
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.nn import GSQEmbedding
    from mlx_gsq_amd.runtime.kernels import iq2_s_embedding
    from mlx_gsq_amd.runtime.store import PackedWeight
    ids = torch.zeros(1, 3, dtype=torch.int32)
    p = torch.zeros(10 * 2 * 82, dtype=torch.uint8)
    with pytest.raises(ValueError, match="divisible by 256"):
        iq2_s_embedding(ids, p, vocab_size=10, dimensions=300)
    with pytest.raises(ValueError, match="size mismatch"):
        iq2_s_embedding(ids, p[:-1], vocab_size=10, dimensions=512)
    w = PackedWeight("e", p, (512, 10), (10, 512), "IQ2_XS", 17, 5120, p.numel())
    with pytest.raises(NotImplementedError, match="IQ2_XS"):
        GSQEmbedding(w)
    rc = _lib.lib().gsq_embedding(22, 1, 1, 0, 3, 10, 300, 16, 1, None)
    assert rc == _lib.GSQ_E_VALUE and b"divisible by 256" in _lib.lib().gsq_last_error()
    rc = _lib.lib().gsq_embedding(22, 1, 1, 2, 3, 10, 512, 16, 1, None)
    assert rc == _lib.GSQ_E_TYPE


def test_codebook_validation():
    from mlx_gsq_amd import tables
    t = tables.synthetic_tables(3)
    for q, g in t.items():
        tables.validate_grid(q, g)
    bad = t["IQ2_XS"].copy()
    bad[0, 0] = 9.0
    with pytest.raises(ValueError, match="outside"):
        tables.validate_grid("IQ2_XS", bad)
    dup = t["IQ3_S"].copy()
    dup[1] = dup[0]
    with pytest.raises(ValueError, match="unique"):
        tables.validate_grid("IQ3_S", dup)
    assert list(tables.ksigns()[:8]) == [0, 129, 130, 3, 132, 5, 6, 135]


def test_missing_codebook_is_an_error(monkeypatch):
    from mlx_gsq_amd import tables
    monkeypatch.delenv("GSQ_CODEBOOKS", raising=False)
    saved = dict(tables._registered)
    tables.clear_tables()
    try:
        with pytest.raises(RuntimeError, match="no codebook"):
            tables.grid("IQ2_XXS")
    finally:
        tables._registered.update(saved)


def test_codebook_file_source(tmp_path, monkeypatch):
    from mlx_gsq_amd import tables
    t = tables.synthetic_tables(4)
    path = tmp_path / "books.npz"
    np.savez(path, **{k: v for k, v in t.items() if k != "IQ1_M"})
    monkeypatch.setenv("GSQ_CODEBOOKS", str(path))
    saved = dict(tables._registered)
    tables.clear_tables()
    try:
        np.testing.assert_array_equal(tables.grid("IQ1_M"), t["IQ1_S"])
        np.testing.assert_array_equal(tables.grid("IQ3_XXS"), t["IQ3_XXS"])
    finally:
        tables.clear_tables()
        tables._registered.update(saved)


def test_fused_linear_concatenates_rows_and_validates():
    import torch
    from mlx_gsq_amd import synth
    from mlx_gsq_amd.nn import GSQFusedLinear
    from mlx_gsq_amd.runtime.store import PackedWeight

    def pw(q, n, k, seed, qid, bb):
        data = torch.from_numpy(synth.make_packed(q, n, k, seed=seed))
        return PackedWeight(name=f"w{seed}", data=data, gguf_shape=(k, n), logical_shape=(n, k),
                            quantization_type=q, quantization_type_id=qid, num_elements=n * k,
                            num_bytes=n * (k // 256) * bb)
    a, b = pw("IQ2_XS", 32, 512, 1, 17, 74), pw("IQ2_XS", 16, 512, 2, 17, 74)
    fused = GSQFusedLinear([a, b])
    assert fused.out_features == 48 and fused.splits == [32, 16] and fused.qtype == "IQ2_XS"
    assert torch.equal(fused.packed_weight, torch.cat([a.data, b.data]))
    with pytest.raises(ValueError):
        GSQFusedLinear([a, pw("IQ4_XS", 16, 512, 3, 23, 136)])
    with pytest.raises(ValueError):
        GSQFusedLinear([a, pw("IQ2_XS", 16, 1024, 4, 17, 74)])
    with pytest.raises(ValueError):
        GSQFusedLinear([])


def test_grouped_linear_groups_by_type_and_validates():
    import torch
    from mlx_gsq_amd import synth
    from mlx_gsq_amd.nn import GSQGroupedLinear
    from mlx_gsq_amd.runtime.store import PackedWeight

    def pw(q, n, k, seed, qid, bb):
        data = torch.from_numpy(synth.make_packed(q, n, k, seed=seed))
        return PackedWeight(name=f"w{seed}", data=data, gguf_shape=(k, n), logical_shape=(n, k),
                            quantization_type=q, quantization_type_id=qid, num_elements=n * k,
                            num_bytes=n * (k // 256) * bb)
    q, k, v = pw("IQ2_XS", 64, 512, 1, 17, 74), pw("IQ2_XS", 16, 512, 2, 17, 74), pw("IQ4_XS", 16, 512, 3, 23, 136)
    g = GSQGroupedLinear([q, v, k])
    assert g.slots == [[0, 2], [1]] and g.out_features == [64, 16, 16]
    assert [p.qtype for p in g.parts] == ["IQ2_XS", "IQ4_XS"]
    assert torch.equal(g.parts[0].packed_weight, torch.cat([q.data, k.data]))
    with pytest.raises(ValueError):
        GSQGroupedLinear([q, pw("IQ2_XS", 16, 1024, 4, 17, 74)])
    with pytest.raises(ValueError):
        GSQGroupedLinear([])



def test_matvec_routing_rule():
    """quantized_matvec's routing (host logic, no GPU): the reference's 8-row threshold, rows
    wider than the vector kernel's registers, and the small fp16 batches of 2^26+ weight matrices
    that the small-batch QMM computes faster (from 5 rows when K > 8192, from 7 otherwise)."""
    from mlx_gsq_amd.runtime.kernels.qmv import routes_to_qmm
    f16, f32 = torch.float16, torch.float32
    big = 1 << 26
    assert routes_to_qmm(8, f16, 64, 512) and routes_to_qmm(8, f32, 64, 512)  # the reference's rule
    assert not routes_to_qmm(7, f16, 64, 512) and not routes_to_qmm(1, f32, 64, 512)
    assert routes_to_qmm(1, f16, 64, 65536 + 256) and not routes_to_qmm(1, f16, 64, 65536)
    assert routes_to_qmm(1, f32, 64, 32768 + 256) and not routes_to_qmm(1, f32, 64, 32768)
    for rows in range(1, 8):
        assert routes_to_qmm(rows, f16, -(-big // 17408), 17408) == (rows >= 5)  # K > 8192
        assert routes_to_qmm(rows, f16, big // 4096, 4096) == (rows >= 7)
        assert not routes_to_qmm(rows, f16, big // 4096 - 1, 4096)  # below 2^26 weights
        assert not routes_to_qmm(rows, f32, big // 4096, 4096)  # fp16 activations only
