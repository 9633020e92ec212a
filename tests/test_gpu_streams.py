"""QMM on several streams and under HIP graph capture.

Tiled and small-batch QMM launches exchange split-tile partials through a workspace the library
keeps per (device, stream), so launches on different streams never share one: the same products
enqueued concurrently on two streams give the single-stream results bit for bit (the split
tiles are summed in a fixed order). Capturing QMM on a stream that has no workspace yet fails
cleanly (before anything is enqueued) until gsq_prepare gives it one.
"""
import numpy as np
import pytest
import torch

from mlx_gsq_amd import synth, tables
from oracle import gsq_oracle as O

pytestmark = pytest.mark.gpu

TABLES = tables.synthetic_tables(0)


@pytest.fixture(autouse=True, scope="module")
def _codebooks():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    tables.set_tables(TABLES)
    yield


def _cases(specs, seed0):
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import TYPE_IDS
    out = []
    for i, (qtype, m, n, k) in enumerate(specs):
        packed = synth.make_packed(qtype, n, k, seed=seed0 + i)
        x = synth.make_x(m, k, seed=seed0 + 50 + i, dtype=np.float16)
        _lib.ensure_tables(qtype, torch.device("cuda:0"))
        out.append((qtype, TYPE_IDS[qtype], packed, x, torch.from_numpy(packed).cuda(), torch.from_numpy(x).cuda(),
                    torch.empty(m, n, device="cuda"), m, n, k))
    return out


def _launch(lib, cases, stream):
    for _, tid, _, _, pd, xd, y, m, n, k in cases:
        rc = lib.gsq_qmm(tid, pd.data_ptr(), xd.data_ptr(), 1, y.data_ptr(), 0, m, n, k, stream)
        assert rc == 0, lib.gsq_last_error()


def test_qmm_two_streams_concurrently():
    from mlx_gsq_amd import _lib
    lib = _lib.lib()
    # split tiles on both streams (tiled and small-batch kernels), several launches each
    a = _cases((("IQ3_S", 200, 1536, 5120), ("Q4_K", 5, 1000, 4096), ("Q6_K", 300, 520, 2048)), 10)
    b = _cases((("IQ2_XS", 64, 1000, 1024), ("Q6_K", 11, 520, 17408), ("IQ4_XS", 512, 2048, 4096)), 20)
    main = torch.cuda.current_stream()
    _launch(lib, a, main.cuda_stream)
    _launch(lib, b, main.cuda_stream)
    torch.cuda.synchronize()
    ref_a = [c[6].clone() for c in a]
    ref_b = [c[6].clone() for c in b]
    for c in a + b:  # the single-stream results match the oracle
        qtype, _, packed, x, _, _, y, m, n, k = c
        want = O.matmul_reference(x, packed, qtype, n, k, TABLES.get(qtype))
        got = y.cpu().numpy()
        assert float(np.linalg.norm(got - want) / np.linalg.norm(want)) <= 1e-3, qtype
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for rep in range(6):
        for c in a + b:
            c[6].fill_(float("nan"))
        go = torch.cuda.Event()
        go.record(main)
        s1.wait_event(go)
        s2.wait_event(go)
        for i in range(3):  # interleaved enqueue: the streams' kernels overlap on the device
            _launch(lib, a[i:i + 1], s1.cuda_stream)
            _launch(lib, b[i:i + 1], s2.cuda_stream)
        torch.cuda.synchronize()
        for c, r in zip(a, ref_a):
            assert torch.equal(c[6], r), f"stream 1, {c[0]}, repeat {rep}"
        for c, r in zip(b, ref_b):
            assert torch.equal(c[6], r), f"stream 2, {c[0]}, repeat {rep}"


def test_qmm_capture_needs_prepared_stream():
    from mlx_gsq_amd import _lib
    lib = _lib.lib()
    cases = _cases((("Q4_K", 40, 600, 2048),), 40)
    _launch(lib, cases, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = cases[0][6].clone()
    # a fresh stream has no workspace: the call under capture is refused, nothing is enqueued
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    _, tid, _, _, pd, xd, y, m, n, k = cases[0]
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            rc = lib.gsq_qmm(tid, pd.data_ptr(), xd.data_ptr(), 1, y.data_ptr(), 0, m, n, k, cap.cuda_stream)
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    assert rc == _lib.GSQ_E_VALUE
    assert b"gsq_prepare" in lib.gsq_last_error()
    # prepared, the same capture works and replays the eager result
    cap2 = torch.cuda.Stream()
    _lib.prepare(stream=cap2)
    cap2.wait_stream(torch.cuda.current_stream())
    graph2 = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap2):
        with torch.cuda.graph(graph2, stream=cap2):
            _launch(lib, cases, cap2.cuda_stream)
    torch.cuda.current_stream().wait_stream(cap2)
    for rep in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        graph2.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {rep}"
