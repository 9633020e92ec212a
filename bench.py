"""Benchmark of the quantized-linear hot path on one MI355X.

Workload: fused QMV at M=1 over all 11 types on the 27B layer
shapes N x K in {5120x5120, 1024x5120, 17408x5120, 5120x17408}. One step = one pass over
the 44 (type, shape) products with seeded random packed weights resident in HBM (about
0.9 GB of distinct weights, larger than the 256 MB MALL, so every launch streams from HBM).

Printed JSON line:
  value      whole-step HBM throughput: algorithmic bytes of the 44 launches / step time
  roofline   the dominant QMV kernel (largest share of step time): its algorithmic bytes
             per launch / its average launch time from HIP events on the launch stream,
             against the 8 TB/s HBM peak
  per_type   per-type GB/s and fraction of peak over its 4 shapes
  qmm        tiled QMM at M=512 (configs[2] subset): TFLOP/s and fraction of dense fp16 peak
  cpu_baseline  the numpy oracle (dequant + float32 matmul, one thread) on a bounded sample

Algorithmic bytes per QMV launch = N*(K/256)*block_bytes + M*K*2 (x fp16) + M*N*4 (y fp32).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mlx-gsq-rco_amd")]

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
SHAPES = ((5120, 5120), (1024, 5120), (17408, 5120), (5120, 17408))
METRIC = "QMV GB/s & % HBM peak (M=1); QMM TFLOPS & % MFMA peak (M=512); per type"


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


def cpu_baseline(budget_s: float = 12.0):
    """numpy oracle (the reference's CPU path restated) on one 1024x5120 matrix per type."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from mlx_gsq_amd import synth, tables
    from mlx_gsq_amd.formats import QTYPES
    from oracle import gsq_oracle as O
    books = tables.synthetic_tables(0)
    n, k = 1024, 5120
    total_b, total_t, mm_t = 0, 0.0, 0.0
    reps = 0
    with threadpool_limits(1):
        t_start = time.perf_counter()
        while time.perf_counter() - t_start < budget_s or reps == 0:
            for q in QTYPES:
                p = synth.make_packed(q, n, k, seed=5)
                x = synth.make_x(1, k, seed=6, dtype=np.float16)
                t0 = time.perf_counter()
                w = O.dequantize_reference(p, q, books.get(q)).reshape(n, k)
                t1 = time.perf_counter()
                y = x.astype(np.float32) @ w.T
                t2 = time.perf_counter()
                total_t += t2 - t0
                mm_t += t2 - t1
                total_b += qmv_bytes(q, n, k)
                assert y.shape == (1, n)
            reps += 1
    return {"value": round(total_b / total_t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"numpy oracle dequant + fp32 matmul, 11 types x {n}x{k}, M=1, {reps} pass(es), 1 thread",
            "matmul_only_s_per_pass": round(mm_t / reps, 4), "host_cpus": os.cpu_count()}


def run_qmv_sweep(steps, warmup, device):
    import torch
    from mlx_gsq_amd import _lib, tables
    from mlx_gsq_amd.formats import QTYPES, TYPE_IDS
    lib = _lib.lib()
    tables.set_tables(tables.synthetic_tables(0))
    cases = []
    for ti, q in enumerate(QTYPES):
        _lib.ensure_tables(q, device)
        for si, (n, k) in enumerate(SHAPES):
            packed = make_device_packed(q, n, k, seed=1000 + 10 * ti + si, device=device)
            x = torch.randn(1, k, device=device, generator=torch.Generator(device=device).manual_seed(si)).half()
            y = torch.empty(1, n, device=device, dtype=torch.float32)
            cases.append((q, n, k, packed, x, y))
    torch.cuda.synchronize()
    log(f"resident packed weights: {sum(c[3].numel() for c in cases) / 1e9:.3f} GB in {len(cases)} matrices")
    stream = torch.cuda.current_stream(device)
    sh = stream.cuda_stream

    def launch(c):
        q, n, k, packed, x, y = c
        rc = lib.gsq_qmv(TYPE_IDS[q], packed.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 0, 1, n, k, sh)
        if rc:
            raise RuntimeError(lib.gsq_last_error().decode())

    for _ in range(warmup):
        for c in cases:
            launch(c)
    torch.cuda.synchronize()
    # per-type event brackets (launches of one type are contiguous in `cases`)
    ntypes = len(QTYPES)
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(ntypes)]
           for _ in range(steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for s in range(steps):
        for ti in range(ntypes):
            evs[s][ti][0].record(stream)
            for c in cases[4 * ti: 4 * ti + 4]:
                launch(c)
            evs[s][ti][1].record(stream)
    stop.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    type_ms = [sum(evs[s][ti][0].elapsed_time(evs[s][ti][1]) for s in range(steps)) for ti in range(ntypes)]
    step_bytes = sum(qmv_bytes(c[0], c[1], c[2]) for c in cases)
    per_type = {}
    for ti, q in enumerate(QTYPES):
        b = sum(qmv_bytes(q, n, k) for (n, k) in SHAPES)
        gbs = b * steps / (type_ms[ti] * 1e-3) / 1e9
        per_type[q] = {"GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                       "us_per_launch": round(type_ms[ti] * 1e3 / steps / 4, 2)}
    dom = max(range(ntypes), key=lambda i: type_ms[i])
    dq = QTYPES[dom]
    dom_bytes = sum(qmv_bytes(dq, n, k) for (n, k) in SHAPES) / 4
    dom_us = type_ms[dom] * 1e3 / steps / 4
    return {
        "total_ms": total_ms, "step_bytes": step_bytes, "per_type": per_type,
        "dominant": {"kernel": f"qmv_kernel<{dq}> (type id {TYPE_IDS[dq]})", "qtype": dq,
                     "bytes_per_launch": dom_bytes, "us_per_launch": dom_us},
        "mean_type_frac": sum(v["frac"] for v in per_type.values()) / ntypes,
    }


def run_qmm(device, reps=10):
    import torch
    from mlx_gsq_amd import _lib
    from mlx_gsq_amd.formats import TYPE_IDS
    lib = _lib.lib()
    out = {}
    stream = torch.cuda.current_stream(device)
    for q in ("IQ3_S", "Q6_K"):
        for (n, k) in ((17408, 5120), (5120, 17408)):
            m = 512
            packed = make_device_packed(q, n, k, seed=77, device=device)
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
            out[f"{q} {n}x{k} M={m}"] = {"ms": round(ms, 3), "TFLOP/s": round(tf, 1),
                                          "frac": round(tf / FP16_PEAK_TFLOPS, 4)}
            del packed, x, y
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-qmm", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode "
              "(QMV/QMM would shard along N with no exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    res = run_qmv_sweep(args.steps, args.warmup, device)
    qmm = {} if args.no_qmm else run_qmm(device)
    cpu = None if args.no_cpu else cpu_baseline()
    ms_per_step = res["total_ms"] / args.steps
    value = res["step_bytes"] / (ms_per_step * 1e-3) / 1e9
    dom = res["dominant"]
    achieved = dom["bytes_per_launch"] / (dom["us_per_launch"] * 1e-6) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "configs[1]: QMV M=1, 11 types x NxK {5120x5120,1024x5120,17408x5120,5120x17408}",
                   "global_batch": 1, "launches_per_step": 44, "x": "fp16", "y": "fp32"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": dom["kernel"], "bytes_per_launch": int(dom["bytes_per_launch"]),
                     "us_per_launch": round(dom["us_per_launch"], 3)},
        "mean_type_frac": round(res["mean_type_frac"], 4),
        "per_type": res["per_type"],
        "qmm": qmm,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
