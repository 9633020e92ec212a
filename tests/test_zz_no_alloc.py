"""gsq_qmm_noalloc (the allocation-free QMM entry point) against gsq_qmm, through the C ABI.

Two calls in a row per kernel, the second with a smaller input, so that the shared scratch
array holds the first call's partials and counters when the second starts. The small-batch
kernel (M <= 16) and tiled plans of at most 64 activation rows pick the same launch plan in both
entry points, so those results are bit-identical; above 64 rows the allocation-free entry point
uses 64-row tiles (its scratch holds their partials for one workgroup per CU) where gsq_qmm uses
128- or 256-row tiles, so those results agree within the QMM tolerance (rel-L2 <= 1e-3 and the
reference's rtol 2e-3 / atol 2e-3 * max|ref|, tests/test_all_qmm.py:38-39) and both match the
oracle to that bar.
"""
import numpy as np
import pytest
import torch

from mlx_gsq_amd import synth, tables
from oracle import gsq_oracle as O

pytestmark = pytest.mark.gpu

TABLES = tables.synthetic_tables(0)


@pytest.fixture(autouse=True, scope="module")
def _setup():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mlx_gsq_amd import _lib
    tables.set_tables(TABLES)
    for q in ("Q4_K", "IQ3_S", "Q6_K", "IQ2_XS", "IQ4_XS", "IQ1_M"):
        _lib.ensure_tables(q, torch.device("cuda:0"))
    _lib.prepare()  # fixed tables; the allocation-free calls below build nothing
    yield


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _call(fn, qtype, packed, x, m, n, k):
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import TYPE_IDS
    y = torch.full((m, n), float("nan"), device="cuda")
    rc = fn(TYPE_IDS[qtype], packed.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, m, n, k,
            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.lib().gsq_last_error()
    return y


# (first call, second call): the second is smaller in M, N and K
PAIRS = [
    (("IQ3_S", 200, 1536, 5120), ("IQ3_S", 40, 1000, 2048)),    # tiled: 256-row vs 64-row tiles, then 64
    (("Q4_K", 600, 2048, 4096), ("Q6_K", 130, 520, 2048)),      # tiled, many split tiles
    (("Q4_K", 16, 5120, 4096), ("IQ2_XS", 5, 1000, 2048)),      # small batch, split row groups
    (("IQ1_M", 11, 1024, 17408), ("IQ4_XS", 2, 520, 1024)),     # small batch, K = 17408, then tiny
]


@pytest.mark.parametrize("pair", PAIRS)
def test_noalloc_matches_qmm_twice(pair):
    from mlx_gsq_amd import _lib
    lib = _lib.lib()
    for i, (qtype, m, n, k) in enumerate(pair):
        print(f"noalloc call {i}: {qtype} M={m} N={n} K={k}", flush=True)
        packed_np = synth.make_packed(qtype, n, k, seed=60 + i)
        x_np = synth.make_x(m, k, seed=70 + i, dtype=np.float16)
        packed = torch.from_numpy(packed_np).cuda()
        x = torch.from_numpy(x_np).cuda()
        got = _call(lib.gsq_qmm_noalloc, qtype, packed, x, m, n, k)
        ref = _call(lib.gsq_qmm, qtype, packed, x, m, n, k)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        if m <= 64:
            assert torch.equal(got, ref), f"call {i}: not bit-identical to gsq_qmm"
        g, r = got.cpu().numpy(), ref.cpu().numpy()
        assert rel_l2(g, r) <= 1e-3
        np.testing.assert_allclose(g, r, rtol=2e-3, atol=2e-3 * np.abs(r).max())
        want = O.matmul_reference(x_np, packed_np, qtype, n, k, TABLES.get(qtype))
        assert rel_l2(g, want) <= 1e-3
        np.testing.assert_allclose(g, want, rtol=2e-3, atol=2e-3 * np.abs(want).max())


def test_noalloc_repeat_is_deterministic():
    """The counters left in the scratch by one call are the zeros the next call needs."""
    from mlx_gsq_amd import _lib
    lib = _lib.lib()
    qtype, m, n, k = "Q4_K", 300, 1536, 5120
    packed = torch.from_numpy(synth.make_packed(qtype, n, k, seed=3)).cuda()
    x = torch.from_numpy(synth.make_x(m, k, seed=4, dtype=np.float16)).cuda()
    first = _call(lib.gsq_qmm_noalloc, qtype, packed, x, m, n, k)
    for _ in range(3):
        again = _call(lib.gsq_qmm_noalloc, qtype, packed, x, m, n, k)
        assert torch.equal(first, again)
