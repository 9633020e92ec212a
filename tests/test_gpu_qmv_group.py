"""GPU parity of the two-product QMV launch (gsq_qmv_group2, GSQGroupedLinear's one-row path).

Each output is held to the vector kernel's bar against the CPU oracle (rel-L2 1e-4 at
K = 5120, as test_qmv_27b_row_widths) and to the product computed alone by gsq_qmv (the same
decoders; the alone launch may pick another plan, so agreement within 1e-6 rel-L2 rather than
bit for bit). GSQ_QMV_GROUP_NO_FALLBACK makes the entry point refuse products its shared
kernel does not take, so the cases meant for that kernel cannot pass through the one-by-one
fallback unnoticed.
"""
import numpy as np
import pytest
import torch

from mlx_gsq_amd import synth, tables
from mlx_gsq_amd.formats import TYPE_IDS
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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def alone(q, packed, x, n, k, odt):
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
    return quantized_matvec(x, packed, qtype=q, out_features=n, in_features=k, out_dtype=odt)


# (type 0, rows 0, type 1, rows 1): q|k + v of the configs[3] layer, two 1024-row products, and
# every type the shared kernel takes at least once (all but Q6_K and IQ3_S, whose rings at
# K = 5120 are two items deep, so their items are not decoded in pairs)
PAIRS = [("IQ2_XS", 6144, "IQ4_XS", 1024), ("IQ1_S", 700, "Q4_K", 1300), ("IQ1_M", 300, "IQ2_S", 2000),
         ("IQ2_XXS", 513, "IQ3_XXS", 64), ("Q2_K", 333, "IQ1_S", 100), ("IQ4_XS", 1024, "IQ2_XS", 1024)]


@pytest.mark.parametrize("pair", PAIRS, ids=[f"{a}+{b}" for a, _, b, _ in PAIRS])
def test_group2_shared_kernel(pair, monkeypatch):
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec_group2
    q0, n0, q1, n1 = pair
    K = 5120
    print(f"qmv group2 {q0} {n0} + {q1} {n1} K={K}", flush=True)
    monkeypatch.setenv("GSQ_QMV_GROUP_NO_FALLBACK", "1")
    p0, p1 = synth.make_packed(q0, n0, K, seed=41), synth.make_packed(q1, n1, K, seed=42)
    x = synth.make_x(1, K, seed=43, dtype=np.float16)
    xd, d0, d1 = dev(x), dev(p0), dev(p1)
    y0, y1 = quantized_matvec_group2(xd, d0, d1, qtypes=(q0, q1), out_features=(n0, n1), in_features=K,
                                     out_dtype=torch.float32)
    assert y0.shape == (1, n0) and y1.shape == (1, n1)
    for y, q, p, d, n in ((y0, q0, p0, d0, n0), (y1, q1, p1, d1, n1)):
        got = y.cpu().numpy()
        want = O.matmul_reference(x, p, q, n, K, TABLES.get(q))
        assert rel_l2(got, want) <= 1e-4, (q, rel_l2(got, want))
        sep = alone(q, d, xd, n, K, torch.float32).cpu().numpy()
        assert rel_l2(got, sep) <= 1e-6, (q, rel_l2(got, sep))


def test_group2_fp16_output_and_repeat(monkeypatch):
    """fp16 outputs, and the same bits on every call (fixed plans, no atomics)."""
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec_group2
    monkeypatch.setenv("GSQ_QMV_GROUP_NO_FALLBACK", "1")
    K = 5120
    p0, p1 = synth.make_packed("IQ2_XS", 1536, K, seed=5), synth.make_packed("IQ4_XS", 256, K, seed=6)
    xd = dev(synth.make_x(1, K, seed=7, dtype=np.float16))
    kw = dict(qtypes=("IQ2_XS", "IQ4_XS"), out_features=(1536, 256), in_features=K)
    a = quantized_matvec_group2(xd, dev(p0), dev(p1), **kw)
    assert a[0].dtype == torch.float16
    for _ in range(3):
        b = quantized_matvec_group2(xd, dev(p0), dev(p1), **kw)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    want = O.matmul_reference(xd.cpu().numpy(), p0, "IQ2_XS", 1536, K, TABLES.get("IQ2_XS"))
    assert rel_l2(a[0].float().cpu().numpy(), want) <= 1e-3


@pytest.mark.parametrize("case", [("Q6_K", 300, "IQ2_S", 200, 5120), ("IQ3_S", 700, "Q4_K", 1300, 5120),
                                  ("IQ2_S", 160, "Q4_K", 96, 17408), ("IQ2_XS", 256, "IQ4_XS", 64, 1024)])
def test_group2_products_the_shared_kernel_refuses(case, monkeypatch):
    """Q6_K and IQ3_S (items not decoded in pairs at K = 5120) and rows of other than 20
    superblocks: refused with the switch set, computed one by one without it."""
    from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec_group2
    q0, n0, q1, n1, K = case
    p0, p1 = synth.make_packed(q0, n0, K, seed=51), synth.make_packed(q1, n1, K, seed=52)
    x = synth.make_x(1, K, seed=53, dtype=np.float16)
    kw = dict(qtypes=(q0, q1), out_features=(n0, n1), in_features=K, out_dtype=torch.float32)
    monkeypatch.setenv("GSQ_QMV_GROUP_NO_FALLBACK", "1")
    with pytest.raises(NotImplementedError, match="shared kernel"):
        quantized_matvec_group2(dev(x), dev(p0), dev(p1), **kw)
    monkeypatch.delenv("GSQ_QMV_GROUP_NO_FALLBACK")
    y0, y1 = quantized_matvec_group2(dev(x), dev(p0), dev(p1), **kw)
    for y, q, p, n in ((y0, q0, p0, n0), (y1, q1, p1, n1)):
        want = O.matmul_reference(x, p, q, n, K, TABLES.get(q))
        assert rel_l2(y.cpu().numpy(), want) <= 1e-4


def test_grouped_linear_one_row_one_launch(monkeypatch):
    """GSQGroupedLinear(q, k, v) at K = 5120 on one row: the shared kernel's outputs against the
    per-type fused launches and the oracle, eagerly and on every replay of a captured graph."""
    from mlx_gsq_amd.nn import GSQFusedLinear, GSQGroupedLinear
    from mlx_gsq_amd.runtime.store import PackedWeight
    monkeypatch.setenv("GSQ_QMV_GROUP_NO_FALLBACK", "1")
    K = 5120
    spec = [("IQ2_XS", 512, 61), ("IQ2_XS", 128, 62), ("IQ4_XS", 128, 63)]
    ws, packs = [], []
    for i, (q, n, seed) in enumerate(spec):
        p = synth.make_packed(q, n, K, seed=seed)
        packs.append(p)
        ws.append(PackedWeight(name=f"w{i}", data=dev(p), gguf_shape=(K, n), logical_shape=(n, K),
                               quantization_type=q, quantization_type_id=TYPE_IDS[q], num_elements=n * K,
                               num_bytes=p.size))
    group = GSQGroupedLinear(ws)
    x = dev(synth.make_x(1, K, seed=64, dtype=np.float16))
    outs = group(x)
    want = list(GSQFusedLinear(ws[:2])(x)) + list(GSQFusedLinear(ws[2:])(x))
    for o, w_, p, (q, n, _) in zip(outs, want, packs, spec):
        assert o.shape == (1, n)
        assert rel_l2(o.float().cpu().numpy(), w_.float().cpu().numpy()) <= 1e-3
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
        for o, e in zip(gout, outs):
            assert torch.equal(o, e)
        group(x)  # eager work between replays
        torch.cuda.synchronize()
