"""GPU parity at the benchmark workload sizes (configs[0]-[3]), checked on sampled output columns.

Every product runs on the device at its full size; the oracle (dequant + float32 matmul,
reference tests/test_all_qmv.py:22, test_all_qmm.py:41-57) then recomputes a seeded sample of
output columns from only those weight rows, which keeps the CPU cost to seconds. The sample
always holds the first and the last row and rows on both sides of every workgroup boundary
the launch plans can produce (multiples of 64 and 256), besides random ones.

Bars: for the fused QMV, rel-L2 <= 1e-4 against the float32 oracle, and every sampled output
within rtol 3e-5 (the reference's QMV tolerance, test_all_qmv.py:23-24) plus an absolute
allowance of max(5e-4, 8 x the float32 oracle's own largest error) of the float64 product of
the same dequantized weights. The reference's absolute 5e-4 is sized for real checkpoint
outputs: the synthetic payloads of configs[0]/[1] (random 6-bit scales, fp16 scales of
|N(0,1)| * 0.01) give outputs of several hundred at K = 5120, where the reference's own float32
CPU path is off by up to ~4e-4 and the kernel's float32 accumulation (group sums scaled once,
offset terms from activation sums) by ~1e-3. One wrong weight moves an output by about
|x| * d * scale (~0.1 and more), far beyond the allowance. For QMM, whose weight operand is
fp16: rel-L2 <= 1e-3
and the reference's QMM tolerance (rtol 2e-3, atol 2e-3 * max|ref|, test_all_qmm.py:38-39).
Codebooks are the seeded synthetic tables (shapes and value sets of the published ones).
"""
import numpy as np
import pytest
import torch

from mlx_gsq_amd import synth, tables
from mlx_gsq_amd.formats import BLOCK_BYTES, QTYPES
from oracle import gsq_oracle as O

pytestmark = pytest.mark.gpu

TABLES = tables.synthetic_tables(0)
SAMPLE = 256


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


def sample_rows(n, seed):
    """SAMPLE distinct weight rows: edges, both sides of 64- and 256-row boundaries, random."""
    rng = np.random.default_rng(seed)
    fixed = {0, n - 1}
    for step in (64, 256):
        for b in rng.choice(np.arange(step, n, step), size=min(16, (n - 1) // step), replace=False):
            fixed.update((int(b) - 1, int(b)))
    rest = rng.choice(n, size=SAMPLE, replace=False)
    rows = sorted(fixed)
    for r in rest:
        if len(rows) >= SAMPLE:
            break
        if int(r) not in fixed:
            rows.append(int(r))
    return np.array(sorted(rows[:SAMPLE]))


def sampled_reference(x, packed, qtype, n, k, rows, f64=False):
    """The oracle's y for the sampled rows: float32 (the reference's CPU path) or the float64
    product of the same (exactly dequantized) weights."""
    row_bytes = (k // 256) * BLOCK_BYTES[qtype]
    sub = packed.reshape(n, row_bytes)[rows].reshape(-1)
    if not f64:
        return O.matmul_reference(x, sub, qtype, len(rows), k, TABLES.get(qtype))
    w = O.dequantize_reference(sub, qtype, TABLES.get(qtype)).reshape(len(rows), k).astype(np.float64)
    return np.asarray(x, np.float64).reshape(-1, k) @ w.T


def check_qmv_bar(got, want, x, packed, qtype, n, k, rows):
    """The vector kernel's bar (module docstring): rel-L2 1e-4, rtol 3e-5 + the absolute allowance."""
    assert rel_l2(got, want) <= 1e-4, rel_l2(got, want)
    truth = sampled_reference(x, packed, qtype, n, k, rows, f64=True)
    err = np.abs(got - truth)
    oracle_err = float(np.abs(want - truth).max())
    ok = err <= 3e-5 * np.abs(truth) + max(5e-4, 8 * oracle_err)
    print(f"max error {err.max():.3g} (float32 oracle {oracle_err:.3g})", flush=True)
    assert ok.all(), (f"{int((~ok).sum())} outputs off: max error {err.max():.3g}, "
                      f"float32 oracle's max error {oracle_err:.3g}")


def check_qmm_bar(got, want):
    """The matrix kernels' bar: rel-L2 1e-3 and the reference's QMM tolerance."""
    assert rel_l2(got, want) <= 1e-3, rel_l2(got, want)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-3 * np.abs(want).max())


def run_matvec(qtype, n, k, seed, m=1):
    """y = x W^T through quantized_matvec's routing (the vector kernel, or the small-batch /
    tiled QMM where the router sends these rows), checked on sampled columns at the bar of the
    kernel that ran."""
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec, routes_to_qmm
    vector = not routes_to_qmm(m, torch.float16, n, k)
    print(f"full-size {'qmv' if vector else 'qmm'} {qtype} M={m} {n}x{k}", flush=True)
    packed = synth.make_packed(qtype, n, k, seed=seed)
    x = synth.make_x(m, k, seed=seed + 1, dtype=np.float16)
    y = quantized_matvec(torch.from_numpy(x).cuda(), torch.from_numpy(packed).cuda(), qtype=qtype,
                         out_features=n, in_features=k, out_dtype=torch.float32).cpu().numpy()
    assert y.shape == (m, n) and np.isfinite(y).all()
    rows = sample_rows(n, seed)
    want = sampled_reference(x, packed, qtype, n, k, rows)
    got = y[:, rows]
    if vector:
        check_qmv_bar(got, want, x, packed, qtype, n, k, rows)
    else:
        check_qmm_bar(got, want)


def run_qmv(qtype, n, k, seed):
    run_matvec(qtype, n, k, seed, m=1)


def test_qmv_configs0_q4k_17408x5120():
    """Q4_K 17408 x 5120, M = 1, fp16 x, fp32 y."""
    run_qmv("Q4_K", 17408, 5120, seed=100)


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("shape", [(17408, 5120), (5120, 17408), (5120, 5120)])
def test_qmv_configs1_27b_shapes(qtype, shape):
    """every type on the 27B layer shapes (1024 x 5120 is covered elsewhere)."""
    n, k = shape
    run_qmv(qtype, n, k, seed=200 + 7 * QTYPES.index(qtype) + (k == 17408) + 2 * (n == k))


# the mixed decoder layer (q / k / v / o / gate / up / down)
LAYER = [("q", "IQ2_XS", 5120, 5120), ("k", "IQ2_XS", 1024, 5120), ("v", "IQ4_XS", 1024, 5120),
         ("o", "IQ3_S", 5120, 5120), ("gate", "IQ2_S", 17408, 5120), ("up", "IQ2_S", 17408, 5120),
         ("down", "Q4_K", 5120, 17408)]


@pytest.mark.parametrize("m", [2, 4, 8, 16])
@pytest.mark.parametrize("proj", LAYER, ids=[p[0] for p in LAYER])
def test_layer_configs3_small_batch(proj, m):
    """every projection of the mixed layer at M = 2..16 through quantized_matvec's
    routing (the vector kernel, or the small-batch QMM with its stream-K split of 17408-row and
    17408-wide products over all CUs), at full size."""
    name, qtype, n, k = proj
    run_matvec(qtype, n, k, seed=500 + 13 * [p[0] for p in LAYER].index(name) + m, m=m)


@pytest.mark.parametrize("qtype", ["IQ3_S", "Q6_K"])
@pytest.mark.parametrize("case", [(182, 17408, 5120), (512, 17408, 5120), (2048, 17408, 5120),
                                  (182, 5120, 17408), (512, 5120, 17408), (2048, 5120, 17408)])
def test_qmm_configs2_shapes(qtype, case):
    """tiled QMM at every M of the config on both shapes (17408 x 5120: 17 x 1024
    weight rows over all CUs; 5120 x 17408: 68 K columns per tile, stream-K split tiles summed
    by the last workgroup)."""
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    m, n, k = case
    print(f"full-size qmm {qtype} M={m} {n}x{k}", flush=True)
    seed = 300 + m + (k == 17408)
    packed = synth.make_packed(qtype, n, k, seed=seed)
    x = synth.make_x(m, k, seed=seed + 1, dtype=np.float16)
    y = quantized_matmul(torch.from_numpy(x).cuda(), torch.from_numpy(packed).cuda(), qtype=qtype,
                         out_features=n, in_features=k, out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(y).all()
    rows = sample_rows(n, seed)
    want = sampled_reference(x, packed, qtype, n, k, rows)
    check_qmm_bar(y[:, rows], want)


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("m", [9, 16])
def test_qmm_small_batch_large_ragged(qtype, m):
    """The small-batch kernel's plan for products of 2^26+ weights (16 waves of 16 rows where
    the type's ring fits, row groups of 256 rows split over the K columns of every CU) on a
    4100 x 16384 matrix, whose last row group holds 4 rows; at M = 9 the rows past M repeat row
    M - 1 and their outputs are dropped. Sampled columns include the last rows."""
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    n, k = 4100, 16384
    print(f"full-size qmm small {qtype} M={m} {n}x{k}", flush=True)
    seed = 700 + m + QTYPES.index(qtype)
    packed = synth.make_packed(qtype, n, k, seed=seed)
    x = synth.make_x(m, k, seed=seed + 1, dtype=np.float16)
    y = quantized_matmul(torch.from_numpy(x).cuda(), torch.from_numpy(packed).cuda(), qtype=qtype,
                         out_features=n, in_features=k, out_dtype=torch.float32).cpu().numpy()
    assert y.shape == (m, n) and np.isfinite(y).all()
    rows = np.union1d(sample_rows(n, seed), np.arange(n - 8, n))
    want = sampled_reference(x, packed, qtype, n, k, rows)
    check_qmm_bar(y[:, rows], want)
