"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Bars (north star): dequantized weights bit-exact; QMV/QMM outputs within rel-L2 1e-3 for
fp32 output and 1e-2 for fp16 output of the oracle's dequant + float32 matmul on the same
seeded inputs. The fused QMV keeps fp32 accumulation of exact fp16 products, so it is also
held to the reference's own QMV tolerance (tests/test_all_qmv.py:24: rtol 3e-5, atol 5e-4).
Codebooks are seeded synthetic tables with the published shapes and value sets (the real
ones come from gguf-py, which is absent here), so table *content* is not pinned by these
tests; indexing, sign and scale arithmetic are.
"""
import numpy as np
import pytest
import torch

from mlx_gsq_amd import synth, tables
from mlx_gsq_amd.formats import QTYPES, packed_size
from oracle import gsq_oracle as O

pytestmark = pytest.mark.gpu

TABLES = tables.synthetic_tables(0)


@pytest.fixture(autouse=True, scope="module")
def _codebooks():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    tables.set_tables(TABLES)
    yield


@pytest.fixture
def vector_kernel_only(monkeypatch):
    """Keep quantized_matvec on gsq_qmv for every row count below the reference's QMM threshold
    (it otherwise sends fp16 batches of 5+ rows to the small-batch QMM kernel), so gsq_qmv's
    multi-row kernels (vector for 2 rows, quad-row for 3-7) stay covered at their own tolerance."""
    from mlx_gsq_amd.runtime.kernels import qmv
    monkeypatch.setattr(qmv, "_small_batch_faster", lambda *a: False)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_bit_exact(qtype):
    from mlx_gsq_amd.runtime.kernels.registry import decode
    print(f"dequant {qtype}", flush=True)
    packed = synth.make_packed(qtype, 64, 1024, seed=11)
    got = decode(dev(packed), qtype).cpu().numpy()
    want = O.dequantize_reference(packed, qtype, TABLES.get(qtype))
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_raw_random_bytes(qtype):
    """Fully random payloads (fp16 fields may be Inf/NaN): same values, same NaN positions."""
    from mlx_gsq_amd.runtime.kernels.registry import decode
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, 37 * O.BLOCK_BYTES[qtype], dtype=np.uint8)
    got = decode(dev(packed), qtype).cpu().numpy()
    want = O.dequantize_reference(packed, qtype, TABLES.get(qtype))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok], want[ok])


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5])
def test_qmv_matches_oracle(qtype, rows, vector_kernel_only):
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
    N, K = 4100, 512  # several rows per workgroup and several staging steps
    print(f"qmv {qtype} M={rows} N={N} K={K}", flush=True)
    packed = synth.make_packed(qtype, N, K, seed=21)
    x = synth.make_x(rows, K, seed=123, dtype=np.float16)
    y = quantized_matvec(dev(x), dev(packed), qtype=qtype, out_features=N, in_features=K,
                         out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)
    np.testing.assert_allclose(y, want, rtol=3e-5, atol=5e-4)


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("xdtype", [np.float32, "bf16"])
def test_qmv_split_precision_inputs(qtype, xdtype):
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
    N, K = 700, 768
    packed = synth.make_packed(qtype, N, K, seed=3)
    x32 = synth.make_x(2, K, seed=9, dtype=np.float32)
    xt = dev(x32) if xdtype is np.float32 else dev(x32).to(torch.bfloat16)
    y = quantized_matvec(xt, dev(packed), qtype=qtype, out_features=N, in_features=K,
                         out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(xt.float().cpu().numpy(), packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("shape", [(1024, 5120), (5200, 5120), (512, 17408)])
def test_qmv_27b_row_widths(qtype, shape):
    """K = 5120 rows go one slice per wave up to 5120 rows and three slices per wave above."""
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
    N, K = shape
    packed = synth.make_packed(qtype, N, K, seed=7)
    x = synth.make_x(1, K, seed=1, dtype=np.float16)
    y = quantized_matvec(dev(x), dev(packed), qtype=qtype, out_features=N, in_features=K,
                         out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)


@pytest.mark.parametrize("qtype", ["Q4_K", "IQ2_S", "IQ3_XXS"])
@pytest.mark.parametrize("rows", [4, 7])
def test_qmv_wide_rows_multi_row(qtype, rows, vector_kernel_only):
    """4 and 7 activation rows of 17408-wide rows: the quad-row kernel (twelve waves of three
    quad slices per row quad; one or two activation quads)."""
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
    N, K = 160, 17408
    packed = synth.make_packed(qtype, N, K, seed=12)
    x = synth.make_x(rows, K, seed=13, dtype=np.float16)
    y = quantized_matvec(dev(x), dev(packed), qtype=qtype, out_features=N, in_features=K,
                         out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y, want) <= 1e-4, rel_l2(y, want)


def test_qmv_unaligned_packed_view_and_odd_rows():
    """A 2-byte (not 16-byte) aligned packed view and an odd N exercise the staged copy's edges."""
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
    for qtype in ("IQ1_S", "Q6_K", "IQ3_S"):
        N, K = 37, 256
        packed = synth.make_packed(qtype, N, K, seed=2)
        big = torch.zeros(packed.size + 64, dtype=torch.uint8, device="cuda")
        big[6:6 + packed.size] = dev(packed)
        view = big[6:6 + packed.size]
        x = synth.make_x(1, K, seed=4, dtype=np.float16)
        y = quantized_matvec(dev(x), view, qtype=qtype, out_features=N, in_features=K,
                             out_dtype=torch.float32).cpu().numpy()
        want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
        assert rel_l2(y, want) <= 1e-4, (qtype, rel_l2(y, want))


@pytest.mark.parametrize("dtype,offset", [(torch.float16, 8), (torch.float16, 2), (torch.bfloat16, 6),
                                          (torch.float32, 4)])
@pytest.mark.parametrize("rows", [1, 2])
def test_qmv_activations_not_16_byte_aligned(dtype, offset, rows):
    """x at a byte offset that is not a multiple of 16 (the reference accepts any array): the
    library stages it into an aligned copy, so the vector kernel gives the same bits as for
    the aligned x."""
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec, routes_to_qmm
    N, K = 300, 1024
    assert not routes_to_qmm(rows, dtype, N, K)
    print(f"qmv unaligned x {dtype} +{offset} M={rows}", flush=True)
    packed = dev(synth.make_packed("IQ3_S", N, K, seed=2))
    x = torch.from_numpy(synth.make_x(rows, K, seed=4, dtype=np.float32)).to("cuda", dtype)
    es = x.element_size()
    big = torch.zeros(x.numel() + 16, dtype=dtype, device="cuda")
    big[offset // es:offset // es + x.numel()] = x.reshape(-1)
    xv = big[offset // es:offset // es + x.numel()].reshape(rows, K)
    assert xv.data_ptr() % 16 == offset % 16 != 0
    kw = dict(qtype="IQ3_S", out_features=N, in_features=K, out_dtype=torch.float32)
    y = quantized_matvec(xv, packed, **kw)
    assert torch.equal(y, quantized_matvec(x, packed, **kw))
    want = O.matmul_reference(x.float().cpu().numpy(), packed.cpu().numpy(), "IQ3_S", N, K, TABLES["IQ3_S"])
    assert rel_l2(y.cpu().numpy(), want) <= 1e-4


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("rows", [8, 16, 33, 100, 128, 182, 257])
def test_qmm_matches_oracle(qtype, rows):
    """Activation tiles of 64 (M <= 64), 128 (M <= 128) and 256 rows, ragged and exact."""
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    N, K = 200, 512
    print(f"qmm {qtype} M={rows}", flush=True)
    packed = synth.make_packed(qtype, N, K, seed=31)
    x = synth.make_x(rows, K, seed=123, dtype=np.float16)
    y = quantized_matmul(dev(x), dev(packed), qtype=qtype, out_features=N, in_features=K,
                         out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y, want) <= 1e-3, rel_l2(y, want)
    scale = np.abs(want).max()
    np.testing.assert_allclose(y, want, rtol=2e-3, atol=2e-3 * scale)  # reference test_all_qmm.py:38-39


# Multi-tile shapes: several 256-row weight tiles, several activation tiles, and K split over
# workgroups (stream-K), including tiles whose partial sums come from many workgroups.
QMM_SHAPES = [
    (300, 520, 2048),   # two 256-row activation tiles (or 128-row), ragged weight tile
    (64, 1000, 1024),   # 64-row activation tiles, four weight tiles
    (512, 2048, 4096),  # 16 tiles x 16 columns: one column per workgroup, 16 partials per tile
    (200, 1536, 5120),  # 20 columns per tile over 6 tiles
]


@pytest.mark.parametrize("qtype", ["Q4_K", "Q6_K", "IQ3_S", "IQ1_M", "IQ2_XS", "IQ4_XS"])
@pytest.mark.parametrize("shape", QMM_SHAPES)
def test_qmm_multi_tile_shapes(qtype, shape):
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    M, N, K = shape
    print(f"qmm {qtype} M={M} N={N} K={K}", flush=True)
    packed = synth.make_packed(qtype, N, K, seed=17)
    x = synth.make_x(M, K, seed=5, dtype=np.float16)
    y = quantized_matmul(dev(x), dev(packed), qtype=qtype, out_features=N, in_features=K,
                         out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y, want) <= 1e-3, rel_l2(y, want)
    scale = np.abs(want).max()
    np.testing.assert_allclose(y, want, rtol=2e-3, atol=2e-3 * scale)


# Small batches (M <= 16) take the small-batch kernel: row groups of 128 weight rows split
# over the K columns of as many workgroups as there are CUs, partial sums of a group summed by
# the last workgroup to finish it. Shapes cover groups split over many workgroups, a ragged
# last group, one column per workgroup and 27B row widths.
SMALL_SHAPES = [
    (1, 1024, 5120),
    (2, 200, 2048),
    (5, 1000, 4096),
    (11, 520, 17408),
    (16, 5120, 1024),
]


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("shape", SMALL_SHAPES)
def test_qmm_small_batch_shapes(qtype, shape):
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    M, N, K = shape
    print(f"qmm small {qtype} M={M} N={N} K={K}", flush=True)
    packed = synth.make_packed(qtype, N, K, seed=29)
    x = synth.make_x(M, K, seed=13, dtype=np.float16)
    y = quantized_matmul(dev(x), dev(packed), qtype=qtype, out_features=N, in_features=K,
                         out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y, want) <= 1e-3, rel_l2(y, want)
    scale = np.abs(want).max()
    np.testing.assert_allclose(y, want, rtol=2e-3, atol=2e-3 * scale)


@pytest.mark.parametrize("qtype", QTYPES)
def test_qmm_small_batch_unaligned_deterministic_fp16_out(qtype):
    """Small batch on a 2-byte aligned packed view: two launches bit-identical, fp16 output
    within 1e-2 of the oracle."""
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    M, N, K = 6, 700, 3072
    print(f"qmm small unaligned {qtype}", flush=True)
    packed = synth.make_packed(qtype, N, K, seed=41)
    big = torch.zeros(packed.size + 64, dtype=torch.uint8, device="cuda")
    big[10:10 + packed.size] = dev(packed)
    view = big[10:10 + packed.size]
    xd = dev(synth.make_x(M, K, seed=3, dtype=np.float16))
    y1 = quantized_matmul(xd, view, qtype=qtype, out_features=N, in_features=K, out_dtype=torch.float32)
    y2 = quantized_matmul(xd, view, qtype=qtype, out_features=N, in_features=K, out_dtype=torch.float32)
    assert torch.equal(y1, y2)
    want = O.matmul_reference(xd.cpu().numpy(), packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y1.cpu().numpy(), want) <= 1e-3
    y16 = quantized_matmul(xd, view, qtype=qtype, out_features=N, in_features=K).float().cpu().numpy()
    assert rel_l2(y16, want) <= 1e-2


@pytest.mark.parametrize("rows", [4, 40])
def test_qmm_activations_not_16_byte_aligned(rows):
    """fp16 activations at an 8-byte offset take the generic kernel (the MFMA kernels read
    16-byte pieces of x); same results within tolerance."""
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    N, K = 300, 1024
    packed = synth.make_packed("IQ3_S", N, K, seed=2)
    x = synth.make_x(rows, K, seed=4, dtype=np.float16)
    big = torch.zeros(x.size + 8, dtype=torch.float16, device="cuda")
    big[4:4 + x.size] = dev(x).reshape(-1)
    xv = big[4:4 + x.size].reshape(rows, K)
    assert xv.data_ptr() % 16 == 8
    y = quantized_matmul(xv, dev(packed), qtype="IQ3_S", out_features=N, in_features=K,
                         out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, "IQ3_S", N, K, TABLES["IQ3_S"])
    assert rel_l2(y, want) <= 1e-3


@pytest.mark.parametrize("qtype", QTYPES)
def test_qmm_unaligned_packed_view_deterministic(qtype):
    """A 2-byte aligned packed view (no 4-byte word reads, superblocks at every offset within
    their 16-byte granules); two launches give bit-identical results (fixed partial-sum order)."""
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    M, N, K = 96, 300, 3072
    print(f"qmm unaligned {qtype}", flush=True)
    packed = synth.make_packed(qtype, N, K, seed=23)
    big = torch.zeros(packed.size + 64, dtype=torch.uint8, device="cuda")
    big[6:6 + packed.size] = dev(packed)
    view = big[6:6 + packed.size]
    x = synth.make_x(M, K, seed=9, dtype=np.float16)
    xd = dev(x)
    y1 = quantized_matmul(xd, view, qtype=qtype, out_features=N, in_features=K, out_dtype=torch.float32)
    y2 = quantized_matmul(xd, view, qtype=qtype, out_features=N, in_features=K, out_dtype=torch.float32)
    assert torch.equal(y1, y2)
    want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
    assert rel_l2(y1.cpu().numpy(), want) <= 1e-3, rel_l2(y1.cpu().numpy(), want)


@pytest.mark.parametrize("qtype", ["Q4_K", "IQ3_S", "Q6_K"])
def test_qmm_fp16_output_and_fp32_input(qtype):
    from mlx_gsq_amd.runtime.kernels.qmm import quantized_matmul
    N, K = 96, 1024
    packed = synth.make_packed(qtype, N, K, seed=8)
    x = synth.make_x(16, K, seed=7, dtype=np.float32)
    want = O.matmul_reference(x, packed, qtype, N, K, TABLES.get(qtype))
    y16 = quantized_matmul(dev(x).half(), dev(packed), qtype=qtype, out_features=N, in_features=K).float().cpu().numpy()
    assert rel_l2(y16, want) <= 1e-2
    y32 = quantized_matmul(dev(x), dev(packed), qtype=qtype, out_features=N, in_features=K).cpu().numpy()
    assert rel_l2(y32, want) <= 1e-3


@pytest.mark.parametrize("rows,n,K", [(5, 300, 4096), (4, 300, 4096), (3, 4096, 4096), (7, 16384, 4096),
                                      (6, 16384, 4096), (5, 4096, 16384), (4, 4096, 16384), (5, 4096, 8192),
                                      (2, 4096, 16384), (8, 5120, 5120)])
def test_matvec_routes_small_fp16_batches(rows, n, K):
    """fp16 batches below the reference's 8 rows stay on gsq_qmv (3-7 rows: the quad-row kernel)
    except on matrices of 2^26+ weights from 5 rows when K > 8192, from 7 otherwise; those and
    8 rows take QMM (fp16-rounded weights, QMM tolerance)."""
    from mlx_gsq_amd.runtime.kernels import qmv
    routed = qmv.routes_to_qmm(rows, torch.float16, n, K)
    assert routed == (rows >= 8 or (n * K >= 1 << 26 and rows >= (5 if K > 8192 else 7)))
    packed = synth.make_packed("Q4_K", n, K, seed=8)
    x = synth.make_x(rows, K, seed=8, dtype=np.float16)
    y = qmv.quantized_matvec(dev(x), dev(packed), qtype="Q4_K", out_features=n, in_features=K,
                             out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, "Q4_K", n, K)
    assert rel_l2(y, want) <= (1e-3 if routed else 1e-4)


def test_matvec_routes_many_rows_to_qmm():
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
    N, K = 64, 512
    packed = synth.make_packed("Q4_K", N, K, seed=1)
    x = synth.make_x(9, K, seed=2, dtype=np.float16)
    y = quantized_matvec(dev(x).reshape(3, 3, K), dev(packed), qtype="Q4_K", out_features=N, in_features=K,
                         out_dtype=torch.float32)
    assert y.shape == (3, 3, N)
    want = O.matmul_reference(x, packed, "Q4_K", N, K)
    assert rel_l2(y.reshape(9, N).cpu().numpy(), want) <= 1e-3


def test_gsq_linear_and_store_roundtrip(tmp_path):
    import json
    from safetensors.torch import save_file
    from mlx_gsq_amd.nn import GSQLinear
    from mlx_gsq_amd.runtime import PackedModelStore
    N, K = 48, 512
    packed = synth.make_packed("IQ2_XS", N, K, seed=4)
    info = {"w": {"qtype": "IQ2_XS", "qtype_id": 17, "gguf_shape": [K, N], "logical_shape": [N, K],
                  "num_elements": N * K, "block_elements": 256, "block_bytes": 74}}
    path = tmp_path / "m.safetensors"
    save_file({"w": torch.from_numpy(packed)}, str(path),
              metadata={"format": "mlx-gsq-packed-v1", "tensor_quantization": json.dumps(info)})
    store = PackedModelStore(path)
    lin = GSQLinear(store.weight("w"))
    x = synth.make_x(1, K, seed=5, dtype=np.float16)
    want = O.matmul_reference(x, packed, "IQ2_XS", N, K, TABLES["IQ2_XS"])
    y1 = lin(dev(x)).float().cpu().numpy()
    assert rel_l2(y1, want) <= 1e-2  # fp16 output, as the reference returns x.dtype
    x4 = synth.make_x(4, K, seed=6, dtype=np.float32)
    y4 = lin(dev(x4)).cpu().numpy()
    assert rel_l2(y4, O.matmul_reference(x4, packed, "IQ2_XS", N, K, TABLES["IQ2_XS"])) <= 1e-3


@pytest.mark.parametrize("rows", [1, 5, 12])
def test_fused_linear_matches_separate_projections(rows):
    """q|k and gate|up style fusion: one launch over the concatenated packed rows gives each
    projection's output (oracle tolerance)."""
    from mlx_gsq_amd.nn import GSQFusedLinear
    from mlx_gsq_amd.runtime.store import PackedWeight
    K = 1024
    shapes = [(512, 17), (128, 18)]
    ws, packs = [], []
    for i, (n, seed) in enumerate(shapes):
        p = synth.make_packed("IQ2_XS", n, K, seed=seed)
        packs.append(p)
        ws.append(PackedWeight(name=f"w{i}", data=dev(p), gguf_shape=(K, n), logical_shape=(n, K),
                               quantization_type="IQ2_XS", quantization_type_id=17, num_elements=n * K,
                               num_bytes=p.size))
    fused = GSQFusedLinear(ws)
    x = synth.make_x(rows, K, seed=6, dtype=np.float32)
    outs = fused(dev(x))
    assert [tuple(o.shape) for o in outs] == [(rows, n) for n, _ in shapes]
    for o, p, (n, _) in zip(outs, packs, shapes):
        want = O.matmul_reference(x, p, "IQ2_XS", n, K, TABLES["IQ2_XS"])
        assert rel_l2(o.cpu().numpy(), want) <= 1e-3


@pytest.mark.parametrize("qtype", ["IQ2_S", "IQ2_XS", "IQ1_M", "Q4_K", "Q6_K"])
def test_qmv_pre_matches_separate_kernels(qtype):
    """gsq_qmv_pre: the residual add + RMSNorm (K = 5120) and the SwiGLU (K = 17408) formed in
    the QMV prologue against the separate kernels (the residual bit for bit, the row within one
    fp16 rounding: the norm's sum runs in another order), the product on the row it wrote bit
    for bit against the plain QMV and within tolerance against the oracle."""
    from mlx_gsq_amd.runtime.kernels import model_ops
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec, quantized_matvec_pre
    g = torch.Generator().manual_seed(11)
    for pre, n, k in (("add_rms_norm", 1536, 5120), ("swiglu", 1024, 17408)):
        packed = synth.make_packed(qtype, n, k, seed=5)
        pd = dev(packed)
        kw = dict(qtype=qtype, out_features=n, in_features=k, out_dtype=torch.float32)
        row = torch.empty(1, k, dtype=torch.float16, device="cuda")
        if pre == "add_rms_norm":
            x = torch.randn(1, k, generator=g).half().cuda()
            d = torch.randn(1, k, generator=g).half().cuda()
            w = (1 + 0.1 * torch.randn(k, generator=g)).half().cuda()
            res = torch.empty_like(x)
            y = quantized_matvec_pre(x, pd, pre=pre, pre_a=d, pre_w=w, eps=1e-6, res_out=res, x_out=row, **kw)
            xs = x.clone()
            want_row = model_ops.add_rms_norm(xs, d, w, 1e-6)
            assert torch.equal(res, xs)
            with pytest.raises(ValueError):  # the residual must go to a new buffer
                quantized_matvec_pre(x, pd, pre=pre, pre_a=d, pre_w=w, eps=1e-6, res_out=x, **kw)
            with pytest.raises(ValueError, match="x_out must not alias"):  # so must the row (in place)
                quantized_matvec_pre(x, pd, pre=pre, pre_w=w, eps=1e-6, x_out=x, **kw)
            with pytest.raises(ValueError, match="x_out must not alias"):
                quantized_matvec_pre(x, pd, pre=pre, pre_a=d, pre_w=w, eps=1e-6, x_out=d, **kw)
            # the GatedDeltaNet convolution of the first 1000 outputs in the epilogue (fp16 y)
            rows, kc = 1000, 4
            state = torch.randn(1, kc - 1, rows, generator=g).half().cuda()
            cw = (0.5 * torch.randn(rows, kc, generator=g)).half().cuda()
            cout = torch.empty(rows, dtype=torch.float32, device="cuda")
            state0 = state.clone()
            y16 = quantized_matvec_pre(x, pd, pre=pre, pre_a=d, pre_w=w, eps=1e-6, conv=(state, cw, cout),
                                       **{**kw, "out_dtype": torch.float16})
            assert rel_l2(y16.float().cpu().numpy(), y.cpu().numpy()) <= 1e-3
            win = torch.cat([state0[0].float(), y16.float()[:, :rows]], dim=0)      # (k, rows)
            acc = (win * cw.float().t()).sum(0)
            assert torch.allclose(cout, acc * torch.sigmoid(acc), rtol=1e-5, atol=1e-5)
            assert torch.equal(state[0], torch.cat([state0[0, 1:], y16[:, :rows]], dim=0))
            # without the add and without outputs asked for
            y0 = quantized_matvec_pre(x, pd, pre=pre, pre_w=w, eps=1e-6, **kw)
            row0 = model_ops.add_rms_norm(x.clone(), None, w, 1e-6)
            assert rel_l2(y0.cpu().numpy(), quantized_matvec(row0, pd, **kw).cpu().numpy()) <= 1e-3
        else:
            x = torch.randn(1, 2 * k, generator=g).half().cuda()
            y = quantized_matvec_pre(x, pd, pre=pre, x_out=row, **kw)
            want_row = model_ops.swiglu(x)
            with pytest.raises(ValueError, match="x_out must not alias"):  # over the up half of x
                quantized_matvec_pre(x, pd, pre=pre, x_out=x[0, k:], **kw)
        assert torch.allclose(row.float(), want_row.float(), rtol=1e-3, atol=1e-6), pre
        assert torch.equal(y, quantized_matvec(row, pd, **kw)), pre
        ref = O.matmul_reference(row.float().cpu().numpy(), packed, qtype, n, k, TABLES.get(qtype))
        assert rel_l2(y.cpu().numpy(), ref) <= 1e-3, pre


@pytest.mark.parametrize("rows", [1, 3])
def test_grouped_linear_mixed_types(rows):
    """q/k/v with mixed types (IQ2_XS, IQ2_XS, IQ4_XS) as one group: every output equals the
    per-type fused launch bit for bit (same kernels and plans) and the oracle within tolerance,
    eagerly and on every replay of a captured graph."""
    from mlx_gsq_amd.nn import GSQFusedLinear, GSQGroupedLinear
    from mlx_gsq_amd.runtime.store import PackedWeight
    K = 1024
    spec = [("IQ2_XS", 17, 512, 21), ("IQ2_XS", 17, 128, 22), ("IQ4_XS", 23, 128, 23)]
    ws, packs = [], []
    for i, (q, qid, n, seed) in enumerate(spec):
        p = synth.make_packed(q, n, K, seed=seed)
        packs.append(p)
        ws.append(PackedWeight(name=f"w{i}", data=dev(p), gguf_shape=(K, n), logical_shape=(n, K),
                               quantization_type=q, quantization_type_id=qid, num_elements=n * K,
                               num_bytes=p.size))
    group = GSQGroupedLinear(ws)
    qk = GSQFusedLinear(ws[:2])
    vv = GSQFusedLinear(ws[2:])
    x = dev(synth.make_x(rows, K, seed=8, dtype=np.float16))
    outs = group(x)
    want = list(qk(x)) + list(vv(x))
    for o, w_, p, (q, _, n, _) in zip(outs, want, packs, spec):
        assert torch.equal(o, w_)
        ref = O.matmul_reference(x.float().cpu().numpy(), p, q, n, K, TABLES.get(q))
        assert rel_l2(o.float().cpu().numpy(), ref) <= 1e-2
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        group(x)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            gout = group(x)
    torch.cuda.current_stream().wait_stream(cap)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for o, w_ in zip(gout, want):
            assert torch.equal(o, w_)
        group(x)  # eager work between replays
        torch.cuda.synchronize()


def test_deterministic_repeat():
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
    N, K = 2048, 5120
    packed = dev(synth.make_packed("IQ3_XXS", N, K, seed=9))
    x = dev(synth.make_x(1, K, seed=3, dtype=np.float16))
    a = quantized_matvec(x, packed, qtype="IQ3_XXS", out_features=N, in_features=K, out_dtype=torch.float32)
    b = quantized_matvec(x, packed, qtype="IQ3_XXS", out_features=N, in_features=K, out_dtype=torch.float32)
    assert torch.equal(a, b)


def test_qmv_hip_graph_replays_match_eager():
    """The QMV launches captured in a HIP graph reproduce the eager results on every replay."""
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import TYPE_IDS
    lib = _lib.lib()
    cases = []
    for i, qtype in enumerate(("Q4_K", "IQ2_S", "IQ1_M", "Q6_K")):
        N, K = 777, 1280
        packed = dev(synth.make_packed(qtype, N, K, seed=60 + i))
        x = dev(synth.make_x(1, K, seed=70 + i, dtype=np.float16))
        _lib.ensure_tables(qtype, packed.device)
        cases.append((TYPE_IDS[qtype], packed, x, torch.empty(1, N, device="cuda"), N, K))

    def launch_all(stream):
        for tid, packed, x, y, N, K in cases:
            assert lib.gsq_qmv(tid, packed.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, 1, N, K, stream) == 0

    launch_all(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = [c[3].clone() for c in cases]
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            launch_all(torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(cap)
    for rep in range(4):
        for c in cases:
            c[3].fill_(float("nan"))          # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert torch.equal(c[3], e), f"replay {rep} differs"


def test_qmm_hip_graph_replays_match_eager():
    """Tiled (stream-K split tiles) and small-batch QMM launches captured in a HIP graph give the
    eager results bit for bit on every replay: the split-tile counters reset themselves, so
    nothing is cleared between calls (gsq_prepare gives the capture stream its workspace)."""
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import TYPE_IDS
    lib = _lib.lib()
    cases = []
    for i, (qtype, M, N, K) in enumerate((("IQ3_S", 200, 1536, 5120), ("Q4_K", 5, 1000, 4096),
                                         ("IQ1_S", 64, 1000, 1024), ("Q6_K", 300, 520, 2048))):
        packed = dev(synth.make_packed(qtype, N, K, seed=80 + i))
        x = dev(synth.make_x(M, K, seed=90 + i, dtype=np.float16))
        _lib.ensure_tables(qtype, packed.device)
        cases.append((TYPE_IDS[qtype], packed, x, torch.empty(M, N, device="cuda"), M, N, K))

    def launch_all(stream):
        for tid, packed, x, y, M, N, K in cases:
            assert lib.gsq_qmm(tid, packed.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, M, N, K, stream) == 0

    launch_all(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = [c[3].clone() for c in cases]
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    _lib.prepare(stream=cap)
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            launch_all(torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(cap)
    for rep in range(4):
        for c in cases:
            c[3].fill_(float("nan"))          # eager work between replays
        launch_all(torch.cuda.current_stream().cuda_stream)  # eager QMM calls between replays
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert torch.equal(c[3], e), f"eager call before replay {rep} differs"
            c[3].fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert torch.equal(c[3], e), f"replay {rep} differs"
