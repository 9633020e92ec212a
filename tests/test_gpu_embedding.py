"""GPU parity of the packed embedding gather against the CPU oracle (run on an MI355X).

Mirrors the reference's tests/test_embedding.py:6-18: selected rows of an IQ2_S table, gathered
and rounded to half, equal the CPU dequantizer's rows rounded to half bit for bit. The C-ABI
gather is also checked for every type, both id dtypes, the three output dtypes and ids
outside the table (rows of zeros). Codebooks are the seeded synthetic tables (content not
pinned, as in the other GPU tests).
"""
import ctypes

import numpy as np
import pytest
import torch

from mlx_gsq_amd import _lib, synth, tables
from mlx_gsq_amd.formats import QTYPES, TYPE_IDS
from oracle import gsq_oracle as O

pytestmark = pytest.mark.gpu

TABLES = tables.synthetic_tables(0)


@pytest.fixture(autouse=True, scope="module")
def _codebooks():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    tables.set_tables(TABLES)
    yield


def _rows(packed, qtype, vocab, dims, ids):
    row_bytes = packed.size // vocab
    out = []
    for t in np.asarray(ids).reshape(-1):
        if 0 <= t < vocab:
            out.append(O.dequantize_reference(packed[t * row_bytes:(t + 1) * row_bytes], qtype, TABLES.get(qtype)))
        else:
            out.append(np.zeros(dims, np.float32))
    return np.stack(out).reshape(*np.asarray(ids).shape, dims)


def test_iq2_s_embedding_selected_rows():
    from mlx_gsq_amd.runtime.kernels.embedding import iq2_s_embedding
    vocab, dims = 300, 1024
    packed = synth.make_packed("IQ2_S", vocab, dims, seed=41)
    ids_np = np.array([[0, 17, 299], [5, 5, 123]], dtype=np.int32)
    want = _rows(packed, "IQ2_S", vocab, dims, ids_np)
    p = torch.from_numpy(packed).cuda()
    got16 = iq2_s_embedding(torch.from_numpy(ids_np).cuda(), p, vocab_size=vocab, dimensions=dims,
                            dtype=torch.float16)
    assert got16.shape == (2, 3, dims) and got16.dtype == torch.float16
    np.testing.assert_array_equal(got16.cpu().numpy(), want.astype(np.float16))
    got_bf = iq2_s_embedding(torch.from_numpy(ids_np.astype(np.int64)).cuda(), p, vocab_size=vocab, dimensions=dims)
    assert got_bf.dtype == torch.bfloat16  # the reference's default
    assert torch.equal(got_bf.cpu(), torch.from_numpy(want).to(torch.bfloat16))


@pytest.mark.parametrize("qtype", QTYPES)
def test_embedding_capi_all_types(qtype):
    vocab, dims = 64, 512
    packed = synth.make_packed(qtype, vocab, dims, seed=43)
    ids_np = np.array([3, 0, 63, 63, 64, -1, 17], dtype=np.int64)  # 64 and -1 lie outside the table
    want = _rows(packed, qtype, vocab, dims, ids_np)
    lib = _lib.lib()
    _lib.ensure_tables(qtype, torch.device("cuda:0"))
    p = torch.from_numpy(packed).cuda()
    stream = torch.cuda.current_stream().cuda_stream
    for ids_dtype in (torch.int64, torch.int32):
        ids = torch.from_numpy(ids_np).to(ids_dtype).cuda()
        for odt, cast in ((torch.float32, np.float32), (torch.float16, np.float16)):
            out = torch.full((ids_np.size, dims), 7.0, dtype=odt, device="cuda")
            rc = lib.gsq_embedding(TYPE_IDS[qtype], p.data_ptr(), ids.data_ptr(), _lib.ID_CODES[ids_dtype], ids_np.size,
                                   vocab, dims, out.data_ptr(), _lib.DTYPE_CODES[odt], stream)
            assert rc == 0, lib.gsq_last_error()
            np.testing.assert_array_equal(out.cpu().numpy(), want.astype(cast))


def test_gsq_embedding_store_roundtrip(tmp_path):
    import json
    from safetensors.torch import save_file
    from mlx_gsq_amd.nn import GSQEmbedding
    from mlx_gsq_amd.runtime import PackedModelStore
    vocab, dims = 40, 512
    packed = synth.make_packed("IQ2_S", vocab, dims, seed=44)
    info = {"token_embd.weight": {"qtype": "IQ2_S", "qtype_id": 22, "gguf_shape": [dims, vocab],
                                  "logical_shape": [vocab, dims], "num_elements": vocab * dims,
                                  "block_elements": 256, "block_bytes": 82}}
    path = tmp_path / "m.safetensors"
    save_file({"token_embd.weight": torch.from_numpy(packed)}, str(path),
              metadata={"format": "mlx-gsq-packed-v1", "tensor_quantization": json.dumps(info)})
    emb = GSQEmbedding(PackedModelStore(path).weight("token_embd.weight"), dtype=torch.float16)
    ids_np = np.array([[1, 39, 0]], dtype=np.int32)
    got = emb(torch.from_numpy(ids_np).cuda()).cpu().numpy()
    np.testing.assert_array_equal(got, _rows(packed, "IQ2_S", vocab, dims, ids_np).astype(np.float16))


def test_embedding_many_ids_27b_width():
    """Hundreds of random ids (some outside the table) at the 27B embedding width, bf16 rows: every
    wave's staged 4 KB output span, the partial last wave included, equals the oracle's rows."""
    from mlx_gsq_amd.runtime.kernels.embedding import iq2_s_embedding
    vocab, dims = 1500, 5120
    packed = synth.make_packed("IQ2_S", vocab, dims, seed=45)
    rng = np.random.default_rng(46)
    ids_np = rng.integers(-3, vocab + 3, size=777).astype(np.int64)
    want = _rows(packed, "IQ2_S", vocab, dims, ids_np)
    got = iq2_s_embedding(torch.from_numpy(ids_np).cuda(), torch.from_numpy(packed).cuda(), vocab_size=vocab,
                          dimensions=dims)
    assert torch.equal(got.cpu(), torch.from_numpy(want).to(torch.bfloat16))
