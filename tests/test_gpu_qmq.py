"""GPU parity of the quad-row QMV kernel (gsq_qmv with 3-8 fp16 activation rows, 2 on large
matrices).

gsq_qmv sends 3-8 fp16 rows (2 on matrices of 2^26+ weights with K <= 8192) to the kernel whose
4x4x4 MFMAs multiply four weight rows' decoded groups with up to eight activation rows. Held to the vector kernel's bar against the CPU oracle:
rel-L2 1e-4 and the elementwise tolerance of test_qmv_matches_oracle. The shapes cover rows that
end in a partial quad (N % 4 != 0), an odd superblock count (a half-filled last quad slice),
the 27B widths K = 5120 (two slices per wave, two row slots) and K = 17408 (three slices per
wave, twelve waves), unaligned packed views (the funnel-shift reads) and fp16 outputs.
"""
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


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def qmv(x, packed, qtype, n, k, odt=torch.float32):
    """gsq_qmv through the C-ABI on the current stream (no routing: every row count runs QMV)."""
    lib = _lib.lib()
    _lib.ensure_tables(qtype, x.device)
    y = torch.empty(x.shape[0], n, device=x.device, dtype=odt)
    st = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.gsq_qmv(TYPE_IDS[qtype], packed.data_ptr(), x.data_ptr(), _lib.DTYPE_CODES[x.dtype], y.data_ptr(),
                     _lib.DTYPE_CODES[odt], x.shape[0], n, k, st)
    _lib.check(rc, "gsq_qmv")
    return y


def check(qtype, m, n, k, seed, odt=torch.float32, offset=0):
    print(f"qmq {qtype} M={m} N={n} K={k} offset={offset}", flush=True)
    packed = synth.make_packed(qtype, n, k, seed=seed)
    x = synth.make_x(m, k, seed=seed + 1, dtype=np.float16)
    if offset:
        buf = torch.zeros(packed.size + offset, dtype=torch.uint8, device="cuda")
        buf[offset:] = torch.from_numpy(packed).cuda()
        pd = buf[offset:]
    else:
        pd = torch.from_numpy(packed).cuda()
    y = qmv(torch.from_numpy(x).cuda(), pd, qtype, n, k, odt).float().cpu().numpy()
    want = O.matmul_reference(x, packed, qtype, n, k, TABLES.get(qtype))
    return y, want


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("rows", [3, 4, 5, 8])
def test_qmq_matches_oracle(qtype, rows):
    """1030 rows (a partial last quad) of 3 superblocks (a half-filled quad slice)."""
    y, want = check(qtype, rows, 1030, 768, seed=31)
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)
    np.testing.assert_allclose(y, want, rtol=3e-5, atol=5e-4)


@pytest.mark.parametrize("qtype", ["IQ2_S", "Q4_K", "IQ1_S"])
@pytest.mark.parametrize("rows", [10, 11, 19])
def test_qmq_more_rows_in_launches_of_eight(qtype, rows):
    """gsq_qmv with more than 8 fp16 rows: launches of 8 on the quad-row kernel, a last one of
    3-7 rows there too, one of 1-2 rows on the vector kernel."""
    y, want = check(qtype, rows, 515, 1024, seed=71)
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)
    np.testing.assert_allclose(y, want, rtol=3e-5, atol=5e-4)


@pytest.mark.parametrize("qtype", ["IQ2_S", "Q4_K", "IQ3_XXS"])
def test_qmq_two_rows_on_large_matrices(qtype):
    """Two fp16 rows of a matrix of 2^26 weights with K <= 8192 take the quad-row kernel (its
    rows 2-3 repeat row 1 and are dropped)."""
    y, want = check(qtype, 2, 16384, 4096, seed=91)
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)
    np.testing.assert_allclose(y, want, rtol=3e-5, atol=5e-4)


@pytest.mark.parametrize("qtype", ["IQ2_XS", "IQ4_XS", "IQ3_S", "IQ2_S", "Q4_K", "Q6_K", "IQ1_M"])
@pytest.mark.parametrize("shape", [(3, 262, 5120), (8, 262, 5120), (4, 68, 17408), (6, 36, 17408)])
def test_qmq_27b_widths(qtype, shape):
    m, n, k = shape
    y, want = check(qtype, m, n, k, seed=41)
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)


@pytest.mark.parametrize("shape", [(3, 1, 256), (4, 2, 512), (5, 3, 256), (8, 7, 1280), (3, 5, 4352)])
@pytest.mark.parametrize("qtype", ["IQ3_XXS", "Q6_K", "IQ1_M"])
def test_qmq_tiny_shapes(qtype, shape):
    """1-7 weight rows (a single, partial quad: rows past N read the last row and are dropped),
    one superblock (a half-filled slice), 17 superblocks (an odd count on several waves)."""
    m, n, k = shape
    y, want = check(qtype, m, n, k, seed=81)
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)
    np.testing.assert_allclose(y, want, rtol=3e-5, atol=5e-4)


@pytest.mark.parametrize("qtype", ["Q4_K", "IQ4_XS", "Q2_K", "IQ2_XXS"])
def test_qmq_unaligned_packed_view(qtype):
    """A packed view 2 bytes past a 16-byte boundary: rows and superblocks not 4-byte aligned."""
    y, want = check(qtype, 3, 301, 1024, seed=51, offset=2)
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)


def test_qmq_fp16_output_and_repeat():
    """fp16 outputs, and the same bits on every call (fixed plans, no atomics)."""
    qtype, m, n, k = "IQ2_S", 4, 520, 5120
    packed = torch.from_numpy(synth.make_packed(qtype, n, k, seed=61)).cuda()
    x = torch.from_numpy(synth.make_x(m, k, seed=62, dtype=np.float16)).cuda()
    a = qmv(x, packed, qtype, n, k, torch.float16)
    for _ in range(3):
        assert torch.equal(a, qmv(x, packed, qtype, n, k, torch.float16))
    want = O.matmul_reference(x.cpu().numpy(), packed.cpu().numpy(), qtype, n, k, TABLES.get(qtype))
    assert rel_l2(a.float().cpu().numpy(), want) <= 1e-3
