"""Benchmark of the quantized-linear hot path on one MI355X.

Workload: fused QMV at M=1 over all 11 types on the 27B layer
shapes N x K in {5120x5120, 1024x5120, 17408x5120, 5120x17408}. One step = one pass over
the 44 (type, shape) products with seeded random packed weights resident in HBM (about
0.9 GB of distinct weights, well beyond the 256 MB MALL, so every launch streams its weights
from HBM). The step is captured once in a HIP graph and replayed; the eager (one launch call
per product) step time is reported beside it.

Printed JSON line (one, on stdout):
  value         whole-step throughput: algorithmic bytes of the 44 launches / graph step time
  roofline      the dominant QMV launch (Q6_K 17408x5120, the step's longest): its algorithmic bytes
                / its time per launch (median of 5 loops of 128 back-to-back launches, HIP
                events on the launch stream), against the 8 TB/s HBM peak; `traffic` comes from the committed
                rocprofv3 counter summary (profiles/qmv_traffic.json) when it covers the
                same kernel and shape, else null
  per_type      per-type GB/s and fraction of peak over its 4 shapes (kernel time)
  per_type_graph the same from per_launch_graph_us: each product launched 32 times inside one
                captured HIP graph (no eager launch cost), median of 3 replays
  per_launch_us time per launch of every (type, shape): median of 3 loops of 32 back-to-back
                launches of that product alone over 8 rotating weight copies (HIP events)
  qmm           tiled QMM (configs[2]: IQ3_S and Q6_K, both shapes, M in {182, 512, 2048}):
                TFLOP/s and fraction of the 2.5 PFLOP/s dense fp16 MFMA peak per case
  layer_crossover  configs[3]: QMV vs QMM time per projection of the mixed layer, M in 1..16
  decode_stack  configs[4]: 448 GEMVs (64 layers, 8.34 GB) in one HIP graph: GB/s, tokens/s
  decode_stack_fused  the same products with q|k and gate|up fused (320 launches)
  decode_stack_grouped  the same through GSQGroupedLinear / GSQLinear modules (fp16 outputs; q|k
                and v as one two-product launch, gate|up fused: 256 launches)
  model_decode  single-token decode of the whole 27B Qwen3.5-hybrid model (norms, GatedDeltaNet,
                attention, MLP, lm_head) as one HIP graph per step: model tokens/s; `batched`:
                8 sequences decoded together (tokens/s over all of them); `prefill`: one
                182-token prompt (the reference's published prefill length)
  cpu_baseline  the numpy oracle (dequant + float32 matmul) on the configs[1] products, all host threads

Algorithmic bytes per QMV launch = N*(K/256)*block_bytes + M*K*2 (x fp16) + M*N*4 (y fp32).

Extra modes for counter collection (rocprofv3 --pmc runs):
  --profile-case Q6_K:17408x5120   only launches of that product (rotating 8 weight copies);
                                   TYPE:NxK:M for M activation rows
  --copy-bytes N                   only a plain device-to-device copy of N bytes
  --qmm-profile-case IQ3_S:512x17408x5120   only launches of that QMM product
  --model-decode                   only the model_decode leg (for kernel traces of the step)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mlx-gsq-rco_amd")]

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
SHAPES = ((5120, 5120), (1024, 5120), (17408, 5120), (5120, 17408))
METRIC = "QMV GB/s & % HBM peak (M=1); QMM TFLOPS & % MFMA peak (M=512); per type"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qmv_traffic.json")
ROOF_REPS, ROOF_REPEATS = 128, 5  # roofline kernel timing: 5 loops of 128 back-to-back launches
CASE_REPS, CASE_REPEATS = 32, 3    # per-product timing: 3 loops of 32 back-to-back launches
ROOF_CASE = ("Q6_K", 17408, 5120)  # the step's longest launch, whose rocprofv3 summary is committed


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_device_packed(qtype, n, k, seed, device):
    """Seeded random packed matrix generated on the device (fp16 scale fields fixed up)."""
    import torch
    from mlx_gsq_amd.formats import BLOCK_BYTES
    from mlx_gsq_amd.synth import _FP16_FIELDS
    bb = BLOCK_BYTES[qtype]
    nblocks = n * (k // 256)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    raw = torch.randint(0, 256, (nblocks, bb), dtype=torch.uint8, device=device, generator=g)
    scale = (torch.randn(nblocks, device=device, generator=g).abs() * 0.01).to(torch.float16)
    bits = scale.view(torch.int16).to(torch.int32) & 0xFFFF
    if qtype == "IQ1_M":
        w = raw[:, 48:56].contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
        for i in range(4):
            nib = (bits >> (4 * i)) & 0xF
            w[:, i] = (w[:, i] & 0x0FFF) | (nib << 12)
        raw[:, 48:56] = w.to(torch.int16).view(torch.uint8).reshape(nblocks, 8)
    else:
        for off in _FP16_FIELDS[qtype]:
            raw[:, off:off + 2] = scale.view(torch.uint8).reshape(nblocks, 2)
    return raw.reshape(-1)


def qmv_bytes(qtype, n, k, m=1):
    from mlx_gsq_amd.formats import BLOCK_BYTES
    return n * (k // 256) * BLOCK_BYTES[qtype] + m * k * 2 + m * n * 4


_CPU_BOOKS = None


def _cpu_init():
    global _CPU_BOOKS
    from threadpoolctl import threadpool_limits
    from mlx_gsq_amd import tables
    threadpool_limits(1)  # one BLAS thread per worker process
    _CPU_BOOKS = tables.synthetic_tables(0)


def _cpu_chunk(args):
    """One chunk of rows: oracle dequant, then the float32 matmul; (total s, matmul s)."""
    from oracle import gsq_oracle as O
    q, sub, x, rows, k = args
    t0 = time.perf_counter()
    w = O.dequantize_reference(sub, q, _CPU_BOOKS.get(q)).reshape(rows, k)
    t1 = time.perf_counter()
    y = x @ w.T
    t2 = time.perf_counter()
    assert y.shape == (1, rows)
    return t2 - t0, t2 - t1


def cpu_baseline(budget_s: float = 25.0, chunk_rows: int = 512):
    """The reference's CPU path (dequantize to float32, then a float32 matmul; reference.py:10-18,
    tests/test_all_qmv.py:22), restated by the numpy oracle, on the headline workload: the 44
    products of configs[1] (11 types x 4 shapes, M = 1), in chunks of `chunk_rows` weight rows
    spread over worker processes, one per host core of the GPU's share (at most 16; separate
    processes, since the oracle's table gathers hold the GIL), each with one BLAS thread. Runs
    before bench.py touches the GPU (the workers are fresh interpreters). Products run in a fixed
    order until the budget is spent: the sample is every product started before then, each
    completed. Payloads are generated (untimed) per product. Reports dequant + matmul GB/s
    (algorithmic bytes, as the GPU figures) and the matmul-only rate of the same chunks on their
    already dequantized float32 weights."""
    import multiprocessing as mp
    import numpy as np
    from concurrent.futures import ProcessPoolExecutor
    from mlx_gsq_amd import synth
    from mlx_gsq_amd.formats import QTYPES
    workers = max(1, min(16, os.cpu_count() or 1))
    products = [(q, n, k) for q in QTYPES for (n, k) in SHAPES]
    done, total_b, wall, mm_t, work_t = 0, 0, 0.0, 0.0, 0.0
    with ProcessPoolExecutor(workers, mp_context=mp.get_context("spawn"), initializer=_cpu_init) as ex:
        list(ex.map(_cpu_init_probe, range(workers)))  # workers started and warm before timing
        order = sorted(range(len(products)), key=lambda i: (i % 4, i))  # shapes interleaved over types
        for i in order:
            if wall >= budget_s:
                break
            q, n, k = products[i]
            packed = synth.make_packed(q, n, k, seed=900 + i).reshape(n, -1)
            x = synth.make_x(1, k, seed=901 + i, dtype=np.float16).astype(np.float32)
            jobs = [(q, packed[r:r + chunk_rows].reshape(-1), x, min(chunk_rows, n - r), k)
                    for r in range(0, n, chunk_rows)]
            t0 = time.perf_counter()
            res = list(ex.map(_cpu_chunk, jobs))
            wall += time.perf_counter() - t0
            work_t += sum(r[0] for r in res)
            mm_t += sum(r[1] for r in res)
            total_b += qmv_bytes(q, n, k)
            done += 1
    return {"value": round(total_b / wall / 1e9, 3), "unit": "GB/s", "cores": workers, "kind": "port",
            "sample": f"numpy oracle dequant + fp32 matmul (the reference's CPU path), {done} of the "
                      f"{len(products)} configs[1] products (M=1, shapes interleaved over the types) in "
                      f"{chunk_rows}-row chunks on {workers} worker processes, {wall:.1f} s",
            "products_done": done, "wall_s": round(wall, 2),
            "matmul_only_GBs": round(total_b / (mm_t / workers) / 1e9, 3) if mm_t > 0 else None,
            "matmul_share_of_work": round(mm_t / work_t, 4) if work_t > 0 else None,
            "host_cpus": os.cpu_count()}


def _cpu_init_probe(_):
    return os.getpid()


class QmvCases:
    """The 44 (type, shape) products of one step, resident on the device."""

    def __init__(self, device):
        import torch
        from mlx_gsq_amd import _lib, tables
        from mlx_gsq_amd.formats import QTYPES, TYPE_IDS
        self.lib = _lib.lib()
        self.torch = torch
        tables.set_tables(tables.synthetic_tables(0))
        self.cases = []
        for ti, q in enumerate(QTYPES):
            _lib.ensure_tables(q, device)
            for si, (n, k) in enumerate(SHAPES):
                packed = make_device_packed(q, n, k, seed=1000 + 10 * ti + si, device=device)
                x = torch.randn(1, k, device=device, generator=torch.Generator(device=device).manual_seed(si)).half()
                y = torch.empty(1, n, device=device, dtype=torch.float32)
                self.cases.append((q, TYPE_IDS[q], n, k, packed, x, y))
        torch.cuda.synchronize()
        log(f"resident packed weights: {sum(c[4].numel() for c in self.cases) / 1e9:.3f} GB in {len(self.cases)} matrices")

    def launch(self, c, stream):
        q, tid, n, k, packed, x, y = c
        rc = self.lib.gsq_qmv(tid, packed.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, 1, n, k, stream)
        if rc:
            raise RuntimeError(self.lib.gsq_last_error().decode())

    def step_bytes(self):
        return sum(qmv_bytes(c[0], c[2], c[3]) for c in self.cases)


def run_qmv(steps, warmup, device):
    import torch
    qc = QmvCases(device)
    stream = torch.cuda.current_stream(device)
    sh = stream.cuda_stream
    for _ in range(warmup):
        for c in qc.cases:
            qc.launch(c, sh)
    torch.cuda.synchronize()
    # eager pass: one launch call per product, back to back
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for s in range(steps):
        for c in qc.cases:
            qc.launch(c, sh)
    t1.record(stream)
    torch.cuda.synchronize()
    eager_ms = t0.elapsed_time(t1) / steps
    # graph: one step captured once, replayed `steps` times
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(device)
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            for c in qc.cases:
                qc.launch(c, torch.cuda.current_stream(device).cuda_stream)
    stream.wait_stream(cap)
    for _ in range(max(1, warmup)):
        graph.replay()
    torch.cuda.synchronize()
    g0 = torch.cuda.Event(enable_timing=True)
    g1 = torch.cuda.Event(enable_timing=True)
    g0.record(stream)
    for _ in range(steps):
        graph.replay()
    g1.record(stream)
    torch.cuda.synchronize()
    graph_ms = g0.elapsed_time(g1) / steps
    # per-product kernel time: loops of back-to-back launches of that product alone, eager and
    # inside a captured graph
    per_launch = [case_loop(c[0], c[2], c[3], CASE_REPS, device, repeats=CASE_REPEATS) for c in qc.cases]
    per_graph = [case_graph(c[0], c[2], c[3], CASE_REPS, device) for c in qc.cases]
    return qc, (per_launch, per_graph), eager_ms, graph_ms


QMM_TYPES = ("IQ3_S", "Q6_K")
QMM_SHAPES = ((17408, 5120), (5120, 17408))
QMM_ROWS = (182, 512, 2048)


def run_qmm(device, reps=10):
    """QMM for IQ3_S and Q6_K at both 27B shapes, M in {182, 512, 2048} rows of fp16
    activations, fp32 output; time per launch from HIP events on the launch stream.

    Beside each product, ``dense_fp16_library`` times the vendor library's dense fp16 GEMM
    (torch.mm with fp32 output, hipBLASLt on ROCm) on the same weights already dequantized to
    fp16, the operand the QMM rounds to: what a plain GEMM reaches on these shapes with no
    dequantization in it at all, for scale."""
    import torch
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import TYPE_IDS
    lib = _lib.lib()
    out = {}
    dense = {}
    stream = torch.cuda.current_stream(device)
    for q in QMM_TYPES:
        _lib.ensure_tables(q, device)
        for (n, k) in QMM_SHAPES:
            packed = make_device_packed(q, n, k, seed=77, device=device)
            w32 = torch.empty(n * k, device=device, dtype=torch.float32)
            assert lib.gsq_dequant(TYPE_IDS[q], packed.data_ptr(), n * k // 256, w32.data_ptr(),
                                   stream.cuda_stream) == 0, lib.gsq_last_error()
            w16 = w32.view(n, k).half()
            del w32
            for m in QMM_ROWS:
                x = torch.randn(m, k, device=device).half()
                y = torch.empty(m, n, device=device, dtype=torch.float32)
                args = (TYPE_IDS[q], packed.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, m, n, k, stream.cuda_stream)
                assert lib.gsq_qmm(*args) == 0, lib.gsq_last_error()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    lib.gsq_qmm(*args)
                e1.record(stream)
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / reps
                tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
                out[f"{q} {n}x{k} M={m}"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
                                              "frac": round(tf / FP16_PEAK_TFLOPS, 4)}
                def library_gemm():
                    torch.mm(x, w16.t(), out_dtype=torch.float32)
                    return 0

                lib_us = _time_launches(library_gemm, stream, reps)
                ltf = 2.0 * m * n * k / (lib_us * 1e-6) / 1e12
                dense[f"{q} {n}x{k} M={m}"] = {"us": round(lib_us, 1), "TFLOP/s": round(ltf, 1),
                                                "frac": round(ltf / FP16_PEAK_TFLOPS, 4),
                                                "qmm_time_over_library": round(ms * 1e3 / lib_us, 3)}
                del x, y
            del packed, w16
    m512 = [v["frac"] for kk, v in out.items() if kk.endswith("M=512")]
    out["mean_frac_M512"] = round(sum(m512) / len(m512), 4)
    d512 = [v["frac"] for kk, v in dense.items() if kk.endswith("M=512")]
    dense["mean_frac_M512"] = round(sum(d512) / len(d512), 4)
    dense["what"] = ("torch.mm(x fp16, W fp16 dequantized beforehand, out_dtype=float32): the vendor "
                     "GEMM (hipBLASLt) with no dequantization, same shapes, HIP events")
    out["dense_fp16_library"] = dense
    return out


# configs[3]/[4]: the mixed-type decoder layer (name, type, N, K)
LAYER = (("q", "IQ2_XS", 5120, 5120), ("k", "IQ2_XS", 1024, 5120), ("v", "IQ4_XS", 1024, 5120),
         ("o", "IQ3_S", 5120, 5120), ("gate", "IQ2_S", 17408, 5120), ("up", "IQ2_S", 17408, 5120),
         ("down", "Q4_K", 5120, 17408))
CROSS_ROWS = (1, 2, 3, 4, 5, 6, 7, 8, 16)


def _time_launches(fn, stream, reps):
    """Mean time of `reps` launches of fn (HIP events); None if the library refuses the call."""
    import torch
    if fn() != 0:
        return None
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3  # us


def run_crossover(device, reps=20):
    """per projection of the mixed layer and M in {1..8, 16}, QMV vs QMM time (HIP
    events, weights resident); the crossover is the smallest M at which QMM is faster. gsq_qmm
    runs the small-batch kernel for M <= 16 fp16 rows. `routed_us` follows quantized_matvec's
    routing (QMM from 8 rows; on matrices of 2^26+ weights from 5 when K > 8192, else from 7); `best_us` takes the faster."""
    from mlx_gsq_amd.runtime.kernels.qmm import QMM_MIN_ROWS
    from mlx_gsq_amd.runtime.kernels.qmv import _small_batch_faster
    import torch
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import TYPE_IDS
    lib = _lib.lib()
    stream = torch.cuda.current_stream(device)
    sh = stream.cuda_stream
    out = {}
    for (name, q, n, k) in LAYER:
        _lib.ensure_tables(q, device)
        packed = make_device_packed(q, n, k, seed=300, device=device)
        row = {}
        for m in CROSS_ROWS:
            x = torch.randn(m, k, device=device).half()
            y = torch.empty(m, n, device=device, dtype=torch.float32)
            a = (TYPE_IDS[q], packed.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, m, n, k, sh)
            tv = _time_launches(lambda: lib.gsq_qmv(*a), stream, reps)
            tm = _time_launches(lambda: lib.gsq_qmm(*a), stream, reps)
            if tv is None:
                from mlx_gsq_amd import _lib as L
                note = L.lib().gsq_last_error().decode()
            routed = "qmm" if (m >= QMM_MIN_ROWS or _small_batch_faster(m, torch.float16, n, k)) else "qmv"
            row[f"M={m}"] = {"qmv_us": None if tv is None else round(tv, 2), "qmm_us": round(tm, 2),
                             "routed": routed}
            if tv is None:
                row[f"M={m}"]["qmv_refused"] = note
        cross = next((m for m in CROSS_ROWS if row[f"M={m}"]["qmv_us"] is None
                      or row[f"M={m}"]["qmm_us"] < row[f"M={m}"]["qmv_us"]), None)
        out[f"{name} {q} {n}x{k}"] = {"rows": row, "qmm_faster_from_M": cross}
        del packed
    def best(r):  # the routed time: QMV where it runs and is faster, else QMM
        return r["qmm_us"] if r["qmv_us"] is None else min(r["qmv_us"], r["qmm_us"])
    def routed(r):
        return r["qmm_us"] if r["routed"] == "qmm" or r["qmv_us"] is None else r["qmv_us"]
    totals = {f"M={m}": {"qmm_us": round(sum(v["rows"][f"M={m}"]["qmm_us"] for v in out.values()), 2),
                         "best_us": round(sum(best(v["rows"][f"M={m}"]) for v in out.values()), 2),
                         "routed_us": round(sum(routed(v["rows"][f"M={m}"]) for v in out.values()), 2)}
              for m in CROSS_ROWS}
    return {"per_projection": out, "layer_total": totals}


def run_embedding(device, vocab=248320, dims=5120, tokens=(1, 4096), reps=20):
    """Packed IQ2_S embedding gather (the reference's token-embedding lookup, 27B shape: a
    248320 x 5120 IQ2_S table, 407 MB) for a decode step (1 token) and a prefill batch; bf16
    rows. Bytes = packed rows read + output written; HIP events on the launch stream."""
    import torch
    from mlx_gsq_amd import _lib, tables
    from mlx_gsq_amd.formats import TYPE_IDS
    tables.set_tables(tables.synthetic_tables(0))
    _lib.ensure_tables("IQ2_S", device)
    lib = _lib.lib()
    packed = make_device_packed("IQ2_S", vocab, dims, seed=77, device=device)
    stream = torch.cuda.current_stream(device)
    res = {}
    for t in tokens:
        ids = torch.randint(0, vocab, (t,), dtype=torch.int64, device=device,
                            generator=torch.Generator(device=device).manual_seed(t))
        out = torch.empty((t, dims), dtype=torch.bfloat16, device=device)

        def launch():
            rc = lib.gsq_embedding(TYPE_IDS["IQ2_S"], packed.data_ptr(), ids.data_ptr(), 1, t, vocab, dims,
                                   out.data_ptr(), 2, stream.cuda_stream)
            if rc:
                raise RuntimeError(lib.gsq_last_error().decode())

        for _ in range(3):
            launch()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        nbytes = t * (dims // 256) * 82 + t * dims * 2
        res[f"tokens={t}"] = {"us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                              "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"embedding: {res}")
    return {"table": f"IQ2_S {vocab}x{dims}", "out": "bf16", **res}


# The mixed layer with the projections that share a type and an input fused (q|k, gate|up):
# the same weights and bytes in 5 launches per layer instead of 7 (GSQFusedLinear).
LAYER_FUSED = (("qk", "IQ2_XS", 6144, 5120), ("v", "IQ4_XS", 1024, 5120), ("o", "IQ3_S", 5120, 5120),
               ("gateup", "IQ2_S", 34816, 5120), ("down", "Q4_K", 5120, 17408))


def run_stack(device, layers=64, reps=10, fused=False):
    """one decode token of the 448 projection GEMVs (64 layers x the 7 projections of
    the mixed layer, distinct random weights per layer, 8.34 GB resident) at M=1, captured in one
    HIP graph and replayed; aggregate GB/s and implied linear-layer tokens/s. fused: the same
    products with q|k and gate|up as one launch each (320 launches)."""
    import torch
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import TYPE_IDS
    lib = _lib.lib()
    stream = torch.cuda.current_stream(device)
    mats, total = [], 0
    spec = LAYER_FUSED if fused else LAYER
    xs = {k: torch.randn(1, k, device=device).half() for k in (5120, 17408)}
    ys = {n: torch.empty(1, n, device=device, dtype=torch.float32) for (_, _, n, _) in spec}
    for (_, q, _, _) in spec:
        _lib.ensure_tables(q, device)
    for layer in range(layers):
        for (name, q, n, k) in spec:
            p = make_device_packed(q, n, k, seed=5000 + len(mats), device=device)
            mats.append((TYPE_IDS[q], p, n, k))
            total += qmv_bytes(q, n, k)
    torch.cuda.synchronize()

    def step(sh):
        for (tid, p, n, k) in mats:
            rc = lib.gsq_qmv(tid, p.data_ptr(), xs[k].data_ptr(), 1, ys[n].data_ptr(), 0, 1, n, k, sh)
            if rc:
                raise RuntimeError(lib.gsq_last_error().decode())

    step(stream.cuda_stream)
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(device)
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            step(torch.cuda.current_stream(device).cuda_stream)
    stream.wait_stream(cap)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    gbs = total / (ms * 1e-3) / 1e9
    res = {"gemvs": len(mats) if not fused else 7 * layers, "launches": len(mats), "bytes": int(total),
           "ms_per_token": round(ms, 4), "GB/s": round(gbs, 1),
           "frac": round(gbs / HBM_PEAK_GBS, 4), "linear_tokens_per_s": round(1e3 / ms, 1),
           "mix": "per layer: q 5120x5120 IQ2_XS, k/v 1024x5120 IQ2_XS/IQ4_XS, o 5120x5120 IQ3_S, "
                  "gate/up 17408x5120 IQ2_S, down 5120x17408 Q4_K"
                  + ("; q|k and gate|up fused into one launch each" if fused else "")}
    del mats
    torch.cuda.empty_cache()
    return res


def run_stack_grouped(device, layers=64, reps=10):
    """configs[4] through the modules a model uses: per layer GSQGroupedLinear(q, k, v) (q|k
    IQ2_XS and v IQ4_XS in one two-product launch), GSQLinear(o), GSQGroupedLinear(gate, up)
    (one IQ2_S launch) and GSQLinear(down), at M=1 with fp16 outputs, the 64 layers captured in
    one HIP graph and replayed (4 launches per layer)."""
    import torch
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import BLOCK_BYTES, TYPE_IDS
    from mlx_gsq_amd.nn import GSQGroupedLinear, GSQLinear
    from mlx_gsq_amd.runtime.store import PackedWeight
    total, n_mats = 0, [0]

    def weight(q, n, k):
        nonlocal total
        data = make_device_packed(q, n, k, seed=7000 + n_mats[0], device=device)
        n_mats[0] += 1
        total += qmv_bytes(q, n, k)
        return PackedWeight(name=f"m{n_mats[0]}", data=data, gguf_shape=(k, n), logical_shape=(n, k),
                            quantization_type=q, quantization_type_id=TYPE_IDS[q], num_elements=n * k,
                            num_bytes=n * (k // 256) * BLOCK_BYTES[q])
    spec = {name: (q, n, k) for (name, q, n, k) in LAYER}
    for q in {q for (_, q, _, _) in LAYER}:
        _lib.ensure_tables(q, device)
    mods = []
    for _ in range(layers):
        w = {name: weight(*spec[name]) for name in spec}
        mods.append((GSQGroupedLinear([w["q"], w["k"], w["v"]]), GSQLinear(w["o"]),
                     GSQGroupedLinear([w["gate"], w["up"]]), GSQLinear(w["down"])))
    x5 = torch.randn(1, 5120, device=device).half()
    x17 = torch.randn(1, 17408, device=device).half()

    def step():
        for qkv, o, gu, down in mods:
            qkv(x5)
            o(x5)
            gu(x5)
            down(x17)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(device)
    cap.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(cap):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            step()
    stream = torch.cuda.current_stream(device)
    stream.wait_stream(cap)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    gbs = total / (ms * 1e-3) / 1e9
    res = {"gemvs": 7 * layers, "launches": 4 * layers, "bytes": int(total), "ms_per_token": round(ms, 4),
           "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "linear_tokens_per_s": round(1e3 / ms, 1),
           "mix": "as decode_stack; GSQGroupedLinear(q,k,v) and (gate,up), fp16 outputs"}
    del mods, graph
    torch.cuda.empty_cache()
    return res


# packed type of each projection of the synthetic 27B checkpoint (the configs[4] mix extended to
# the GatedDeltaNet projections, the embedding and the output head)
MODEL_TYPES = {"attn_qkv": "IQ2_XS", "attn_gate": "IQ2_XS", "ssm_out": "IQ3_S", "attn_q": "IQ2_XS",
               "attn_k": "IQ2_XS", "attn_v": "IQ4_XS", "attn_output": "IQ3_S", "ffn_gate": "IQ2_S",
               "ffn_up": "IQ2_S", "ffn_down": "Q4_K", "output": "Q6_K", "token_embd": "IQ2_S"}


class SyntheticQwen35Store:
    """Random packed weights of the 27B Qwen3.5-hybrid shapes on the device, behind the store
    interface build_qwen35 reads (weights are not meaningful; the step's work is)."""

    def __init__(self, args, device):
        import torch
        from mlx_gsq_amd.formats import BLOCK_BYTES, TYPE_IDS
        from mlx_gsq_amd.runtime.store import PackedWeight
        self.device, self.weights, self.plains = device, {}, {}
        self.packed_bytes = 0
        a, H = args, args.hidden_size
        g = torch.Generator(device=device)
        g.manual_seed(11)

        def packed(name, kind, n, k):
            q = MODEL_TYPES[kind]
            data = make_device_packed(q, n, k, seed=20000 + len(self.weights), device=device)
            self.weights[name] = PackedWeight(name=name, data=data, gguf_shape=(k, n), logical_shape=(n, k),
                                              quantization_type=q, quantization_type_id=TYPE_IDS[q],
                                              num_elements=n * k, num_bytes=n * (k // 256) * BLOCK_BYTES[q])
            self.packed_bytes += n * (k // 256) * BLOCK_BYTES[q]

        def plain(name, *shape, fill=None):
            t = torch.randn(*shape, device=device, generator=g) * 0.1
            self.plains[name] = t + fill if fill is not None else t

        packed("token_embd.weight", "token_embd", a.vocab_size, H)
        packed("output.weight", "output", a.vocab_size, H)
        plain("output_norm.weight", H, fill=1.0)
        for i in range(a.num_hidden_layers):
            p = f"blk.{i}."
            plain(p + "attn_norm.weight", H, fill=1.0)
            plain(p + "post_attention_norm.weight", H, fill=1.0)
            packed(p + "ffn_gate.weight", "ffn_gate", a.intermediate_size, H)
            packed(p + "ffn_up.weight", "ffn_up", a.intermediate_size, H)
            packed(p + "ffn_down.weight", "ffn_down", H, a.intermediate_size)
            if a.is_linear(i):
                packed(p + "attn_qkv.weight", "attn_qkv", a.conv_dim, H)
                packed(p + "attn_gate.weight", "attn_gate", a.value_dim, H)
                packed(p + "ssm_out.weight", "ssm_out", H, a.value_dim)
                plain(p + "ssm_alpha.weight", a.linear_num_value_heads, H)
                plain(p + "ssm_beta.weight", a.linear_num_value_heads, H)
                plain(p + "ssm_conv1d.weight", a.conv_dim, a.linear_conv_kernel_dim)
                plain(p + "ssm_a", a.linear_num_value_heads, fill=-1.0)
                plain(p + "ssm_dt.bias", a.linear_num_value_heads)
                plain(p + "ssm_norm.weight", a.linear_value_head_dim, fill=1.0)
            else:
                packed(p + "attn_q.weight", "attn_q", a.num_attention_heads * a.head_dim * 2, H)
                packed(p + "attn_k.weight", "attn_k", a.num_key_value_heads * a.head_dim, H)
                packed(p + "attn_v.weight", "attn_v", a.num_key_value_heads * a.head_dim, H)
                packed(p + "attn_output.weight", "attn_output", H, a.num_attention_heads * a.head_dim)
                plain(p + "attn_q_norm.weight", a.head_dim, fill=1.0)
                plain(p + "attn_k_norm.weight", a.head_dim, fill=1.0)

    def weight(self, name):
        return self.weights[name]

    def materialize_plain(self, name):
        return self.plains[name]


def run_model_decode(device, max_len=1024, prompt=8, steps=32, batches=(8,)):
    """§8(f) rank 4: single-token decode steps of the 27B Qwen3.5-hybrid model (64 layers, random
    packed weights in the MODEL_TYPES mix, fp16 activations) as one HIP graph per step
    (GraphDecoder), after an eager prefill of `prompt` tokens; model tokens/s, and the packed
    bytes read per token over the step time. Then the same for `batches` sequences decoded
    together (one step = one token of each; the projections run as small-batch products)."""
    import torch
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.models import GraphDecoder, Qwen35Args, build_qwen35
    args = Qwen35Args()
    for q in set(MODEL_TYPES.values()):
        _lib.ensure_tables(q, device)
    store = SyntheticQwen35Store(args, device)
    model = build_qwen35(store, dtype=torch.float16, args=args)
    # bytes one token reads: every packed matrix except the embedding table (one row of it)
    emb = store.weights["token_embd.weight"]
    per_token = store.packed_bytes - emb.num_bytes + emb.num_bytes // args.vocab_size
    def step_ms(batch):
        cache = model.new_cache(batch=batch, max_len=max_len, device=device)
        ids = torch.randint(0, args.vocab_size, (batch, prompt + steps + 1), device=device)
        with torch.no_grad():
            model(ids[:, :prompt], cache)
            dec = GraphDecoder(model, cache, batch=batch)
            dec.step(ids[:, prompt:prompt + 1])
            torch.cuda.synchronize()
            stream = torch.cuda.current_stream(device)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(steps):
                dec.step(ids[:, prompt + 1 + i:prompt + 2 + i])
            e1.record(stream)
            torch.cuda.synchronize()
        del dec, cache
        torch.cuda.empty_cache()
        return e0.elapsed_time(e1) / steps

    def prefill_ms(tokens):
        ids = torch.randint(0, args.vocab_size, (1, tokens), device=device)
        with torch.no_grad():
            model(ids, model.new_cache(batch=1, max_len=tokens, device=device))  # warm-up
            cache = model.new_cache(batch=1, max_len=tokens, device=device)
            torch.cuda.synchronize()
            stream = torch.cuda.current_stream(device)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            model(ids, cache)
            e1.record(stream)
            torch.cuda.synchronize()
        del cache
        torch.cuda.empty_cache()
        return e0.elapsed_time(e1)

    ms = step_ms(1)
    res = {"model": "Qwen3.5-hybrid 27B shapes (64 layers: 48 GatedDeltaNet, 16 attention), synthetic weights",
           "ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
           "packed_bytes_per_token": int(per_token),
           "packed_GB/s": round(per_token / (ms * 1e-3) / 1e9, 1),
           "frac": round(per_token / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "context": f"prefill {prompt} tokens, then {steps} timed graph steps (KV buffer {max_len})",
           "types": MODEL_TYPES, "batched": {}}
    for b in batches:
        ms_b = step_ms(b)
        res["batched"][f"B={b}"] = {"ms_per_step": round(ms_b, 4), "tokens_per_s": round(b * 1e3 / ms_b, 1)}
    # prefill of the reference's published prompt length (eager: tiled QMM projections, the
    # GatedDeltaNet sequence kernels, attention on torch ops), logits of every position
    pms = prefill_ms(182)
    res["prefill"] = {"tokens": 182, "ms": round(pms, 2), "tokens_per_s": round(182e3 / pms, 1)}
    del model, store
    torch.cuda.empty_cache()
    return res


def qmm_profile_case(spec, reps, device):
    """Launch one QMM product TYPE:MxNxK `reps` times (for rocprofv3 runs)."""
    import torch
    from mlx_gsq_amd import _lib, tables
    from mlx_gsq_amd.formats import TYPE_IDS
    q, shape = spec.split(":")
    m, n, k = (int(v) for v in shape.split("x"))
    tables.set_tables(tables.synthetic_tables(0))
    _lib.ensure_tables(q, device)
    lib = _lib.lib()
    packed = make_device_packed(q, n, k, seed=77, device=device)
    x = torch.randn(m, k, device=device).half()
    y = torch.empty(m, n, device=device, dtype=torch.float32)
    sh = torch.cuda.current_stream(device).cuda_stream
    for _ in range(reps):
        rc = lib.gsq_qmm(TYPE_IDS[q], packed.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, m, n, k, sh)
        assert rc == 0, lib.gsq_last_error()
    torch.cuda.synchronize()
    print(json.dumps({"qmm_profile_case": spec, "reps": reps, "flop_per_launch": 2 * m * n * k}), flush=True)


def case_loop(q, n, k, reps, device, warmup=8, repeats=1, m=1):
    """`repeats` timed loops of `reps` back-to-back launches of one (type, shape) product with `m`
    activation rows over 8 rotating weight copies on the current stream, after `warmup` untimed
    ones; returns the median over the loops of the mean time per launch (us), each from a HIP
    event pair on that stream."""
    import torch
    from mlx_gsq_amd import _lib, tables
    from mlx_gsq_amd.formats import TYPE_IDS
    tables.set_tables(tables.synthetic_tables(0))
    _lib.ensure_tables(q, device)
    lib = _lib.lib()
    copies = [make_device_packed(q, n, k, seed=500 + i, device=device) for i in range(8)]
    x = torch.randn(m, k, device=device).half()
    y = torch.empty(m, n, device=device, dtype=torch.float32)
    stream = torch.cuda.current_stream(device)
    sh = stream.cuda_stream

    def launch(i):
        rc = lib.gsq_qmv(TYPE_IDS[q], copies[i % 8].data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, m, n, k, sh)
        if rc:
            raise RuntimeError(lib.gsq_last_error().decode())

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    per = []
    for _ in range(repeats):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            launch(i)
        e1.record(stream)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e3 / reps)
    return statistics.median(per)


def case_graph(q, n, k, reps, device, repeats=3):
    """The same product launched `reps` times (8 rotating weight copies) inside one captured HIP
    graph, replayed `repeats` times: median time per launch (us) without the host's eager launch
    cost (the form the model's decode step runs in)."""
    import torch
    from mlx_gsq_amd import _lib, tables
    from mlx_gsq_amd.formats import TYPE_IDS
    tables.set_tables(tables.synthetic_tables(0))
    _lib.ensure_tables(q, device)
    lib = _lib.lib()
    copies = [make_device_packed(q, n, k, seed=500 + i, device=device) for i in range(8)]
    x = torch.randn(1, k, device=device).half()
    y = torch.empty(1, n, device=device, dtype=torch.float32)
    stream = torch.cuda.current_stream(device)
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(device)
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            sh = torch.cuda.current_stream(device).cuda_stream
            for i in range(reps):
                rc = lib.gsq_qmv(TYPE_IDS[q], copies[i % 8].data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, 1, n, k, sh)
                if rc:
                    raise RuntimeError(lib.gsq_last_error().decode())
    stream.wait_stream(cap)
    graph.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(repeats):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e3 / reps)
    del graph
    return statistics.median(per)


def profile_case(spec, reps, device):
    """Only one (type, shape) product, TYPE:NxK (one activation row) or TYPE:NxK:M (M rows
    through gsq_qmv): the loop the roofline figure is timed with."""
    q, shape, *rows = spec.split(":")
    n, k = (int(v) for v in shape.split("x"))
    m = int(rows[0]) if rows else 1
    us = case_loop(q, n, k, reps, device, repeats=ROOF_REPEATS, m=m)
    print(json.dumps({"profile_case": spec, "reps": reps, "repeats": ROOF_REPEATS, "warmup": 8,
                      "bytes_per_launch": qmv_bytes(q, n, k, m),
                      "us_per_launch": round(us, 3)}), flush=True)


def copy_case(nbytes, reps, device):
    """Plain device-to-device copy of `nbytes` (the counter scale reference)."""
    import torch
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "reps": reps}), flush=True)


def load_traffic(kernel_case):
    """HBM bytes per launch of `kernel_case` ("TYPE NxK") from the committed counter summary
    (FETCH_SIZE + WRITE_SIZE of that launch, scaled by the same counters on a known copy)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    c = t.get("cases", {}).get(kernel_case)
    return None if c is None else c.get("hbm_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-qmm", action="store_true")
    ap.add_argument("--no-layer", action="store_true", help="skip the mixed-layer crossover and 448-GEMV stack")
    ap.add_argument("--profile-case", default=None, help="TYPE:NxK, launch only that product")
    ap.add_argument("--copy-bytes", type=int, default=0, help="run only a plain copy of this many bytes")
    ap.add_argument("--qmm-profile-case", default=None, help="TYPE:MxNxK, launch only that QMM product")
    ap.add_argument("--model-decode", action="store_true", help="run only the Qwen3.5-hybrid decode-step leg")
    ap.add_argument("--embedding-case", type=int, default=0, help="run only the embedding gather of this many ids")
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode "
              "(QMV/QMM would shard along N: a GPU's rows are one contiguous byte range of the packed matrix)", file=sys.stderr)
        sys.exit(2)
    # the CPU baseline runs first, in fresh worker processes, before anything touches the GPU
    cpu = None if (args.no_cpu or args.copy_bytes or args.profile_case or args.qmm_profile_case
                   or args.model_decode or args.embedding_case) else cpu_baseline()
    import torch
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.copy_bytes:
        copy_case(args.copy_bytes, args.reps, device)
        return
    if args.profile_case:
        profile_case(args.profile_case, args.reps, device)
        return
    if args.qmm_profile_case:
        qmm_profile_case(args.qmm_profile_case, args.reps, device)
        return
    if args.embedding_case:
        print(json.dumps({"embedding": run_embedding(device, tokens=(args.embedding_case,), reps=args.reps)}),
              flush=True)
        return
    if args.model_decode:
        from mlx_gsq_amd import tables
        tables.set_tables(tables.synthetic_tables(0))
        print(json.dumps({"model_decode": run_model_decode(device)}), flush=True)
        return
    qc, (per_launch, per_graph), eager_ms, graph_ms = run_qmv(args.steps, args.warmup, device)
    qmm = {} if args.no_qmm else run_qmm(device)
    crossover = {} if args.no_layer else run_crossover(device)
    stack = {} if args.no_layer else run_stack(device)
    stack_fused = {} if args.no_layer else run_stack(device, fused=True)
    stack_grouped = {} if args.no_layer else run_stack_grouped(device)
    model_decode = {} if args.no_layer else run_model_decode(device)
    emb = {} if args.no_layer else run_embedding(device)
    from mlx_gsq_amd.formats import QTYPES
    step_bytes = qc.step_bytes()
    value = step_bytes / (graph_ms * 1e-3) / 1e9
    per_type, per_type_graph = {}, {}
    launches, launches_graph = {}, {}
    for i, c in enumerate(qc.cases):
        launches[f"{c[0]} {c[2]}x{c[3]}"] = round(per_launch[i], 2)
        launches_graph[f"{c[0]} {c[2]}x{c[3]}"] = round(per_graph[i], 2)
    for ti, q in enumerate(QTYPES):
        idx = range(4 * ti, 4 * ti + 4)
        b = sum(qmv_bytes(qc.cases[i][0], qc.cases[i][2], qc.cases[i][3]) for i in idx)
        for times, out in ((per_launch, per_type), (per_graph, per_type_graph)):
            gbs = b / (sum(times[i] for i in idx) * 1e-6) / 1e9
            out[q] = {"GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    # the roofline kernel: Q6_K 17408x5120, the longest launch of the step (checked below), timed
    # on its own as 5 loops of 128 back-to-back launches, median loop (the loop of
    # --profile-case, which the committed kernel trace runs)
    dq, dn, dk = ROOF_CASE
    dom_case = f"{dq} {dn}x{dk}"
    longest = max(range(len(qc.cases)), key=lambda i: per_launch[i])
    longest_case = f"{qc.cases[longest][0]} {qc.cases[longest][2]}x{qc.cases[longest][3]}"
    dom_bytes = qmv_bytes(dq, dn, dk)
    dom_us = case_loop(dq, dn, dk, ROOF_REPS, device, repeats=ROOF_REPEATS)
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    kernel_time = sum(per_launch) * 1e-6
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(graph_ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "configs[1]: QMV M=1, 11 types x NxK {5120x5120,1024x5120,17408x5120,5120x17408}",
                   "global_batch": 1, "launches_per_step": len(qc.cases), "x": "fp16", "y": "fp32",
                   "step": "one HIP graph of the 44 launches"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic(dom_case),
                     "kernel": f"qmv_kernel<{dq}> M=1", "case": dom_case, "bytes_per_launch": int(dom_bytes),
                     "us_per_launch": round(dom_us, 3), "longest_launch_of_step": longest_case,
                     "timing": f"median of {ROOF_REPEATS} loops of HIP events "
                     f"around {ROOF_REPS} back-to-back launches (8 rotating weight copies) on the launch stream"},
        "eager_ms_per_step": round(eager_ms, 4),
        "kernel_time_GBs": round(step_bytes / kernel_time / 1e9, 1),
        "mean_type_frac": round(sum(v["frac"] for v in per_type.values()) / len(per_type), 4),
        "per_type": per_type,
        "mean_type_frac_graph": round(sum(v["frac"] for v in per_type_graph.values()) / len(per_type_graph), 4),
        "per_type_graph": per_type_graph,
        "per_launch_us": launches,
        "per_launch_graph_us": launches_graph,
        "qmm": qmm,
        "layer_crossover": crossover,
        "decode_stack": stack,
        "decode_stack_fused": stack_fused,
        "decode_stack_grouped": stack_grouped,
        "model_decode": model_decode,
        "embedding": emb,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
