"""Golden vectors (tests/golden/golden.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every committed vector bit for bit (NaN positions included), so a
change to the restatement cannot pass unnoticed. GPU: the device dequantizer reproduces the
synthetic-codebook vectors bit for bit and the fused QMV matches the committed products
(rel-L2 <= 1e-4 in fp32, far inside the 1e-3 north-star gate).
"""
import os

import numpy as np
import pytest

from mlx_gsq_amd import tables
from mlx_gsq_amd.formats import GRID_SHAPES, QTYPES
from oracle import gsq_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def index_grid(q):
    n, c = GRID_SHAPES[q]
    return (np.arange(n)[:, None] * c + np.arange(c)[None, :]).astype(np.float32)


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(np.isnan(a), np.isnan(b)) and \
        np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)])


@pytest.mark.parametrize("qtype", QTYPES)
def test_oracle_reproduces_golden(golden, qtype):
    blocks = golden[f"{qtype}/packed"]
    books = tables.synthetic_tables(0)
    if qtype in GRID_SHAPES:
        assert same(O.dequantize_reference(blocks, qtype, index_grid(qtype)), golden[f"{qtype}/w_index_grid"])
        assert same(O.dequantize_reference(blocks, qtype, books[qtype]), golden[f"{qtype}/w_synthetic_grid"])
    else:
        assert same(O.dequantize_reference(blocks, qtype), golden[f"{qtype}/w"])
    y = O.matmul_reference(golden[f"{qtype}/mm_x"], golden[f"{qtype}/mm_packed"], qtype, 3, 768, books.get(qtype))
    np.testing.assert_array_equal(y, golden[f"{qtype}/mm_y"])


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", QTYPES)
def test_device_matches_golden(golden, qtype):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mlx_gsq_amd.runtime.kernels import decode, quantized_matvec
    tables.set_tables(tables.synthetic_tables(0))
    blocks = torch.from_numpy(golden[f"{qtype}/packed"]).cuda()
    w = decode(blocks, qtype).cpu().numpy()
    want = golden[f"{qtype}/w_synthetic_grid"] if qtype in GRID_SHAPES else golden[f"{qtype}/w"]
    assert same(w, want)
    x = torch.from_numpy(golden[f"{qtype}/mm_x"]).cuda()
    pk = torch.from_numpy(golden[f"{qtype}/mm_packed"]).cuda()
    y = quantized_matvec(x[:1], pk, qtype=qtype, out_features=3, in_features=768, out_dtype=torch.float32)
    ref = golden[f"{qtype}/mm_y"][:1]
    err = np.linalg.norm(y.cpu().numpy() - ref) / np.linalg.norm(ref)
    assert err <= 1e-4, err
