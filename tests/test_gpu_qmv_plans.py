"""QMV parity under launch plans other than the default (run on an MI355X).

The QMV launch plan (waves per workgroup, ring depth target, workgroups per CU, the
one-slice-per-wave limit, ring fill rate, activation staging, paired items) is read from GSQ_QMV_TUNING
once when libgsq.so loads, so each plan runs in a child process of its own. Each child checks
a few types and both 27B row widths against the oracle at the QMV tolerance (rel-L2 1e-4) and
elementwise within 1e-4 relative / 1e-5 of the largest output (the 5120- and 17408-wide rows
give outputs in the thousands, where the reference's fixed atol of 5e-4 is below fp32
summation-order noise).
"""
import os
import subprocess
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import sys, os
sys.path[:0] = [os.environ["GSQ_ROOT"], os.path.join(os.environ["GSQ_ROOT"], "mlx-gsq-rco_amd")]
import numpy as np, torch
from mlx_gsq_amd import synth, tables
from mlx_gsq_amd.runtime.kernels.qmv import quantized_matvec
from oracle import gsq_oracle as O
books = tables.synthetic_tables(0)
tables.set_tables(books)
dev = torch.device("cuda:0")
for qtype, N, K, rows in (("Q6_K", 1100, 5120, 1), ("IQ2_S", 5200, 5120, 1), ("IQ1_M", 300, 17408, 1),
                          ("Q4_K", 700, 5120, 2), ("IQ3_XXS", 900, 512, 1), ("Q2_K", 5202, 5120, 1)):
    print(f"plan {os.environ['GSQ_QMV_TUNING']} {qtype} M={rows} N={N} K={K}", flush=True)
    packed = synth.make_packed(qtype, N, K, seed=31)
    x = synth.make_x(rows, K, seed=32, dtype=np.float16)
    y = quantized_matvec(torch.from_numpy(x).to(dev), torch.from_numpy(packed).to(dev), qtype=qtype,
                         out_features=N, in_features=K, out_dtype=torch.float32).cpu().numpy()
    want = O.matmul_reference(x, packed, qtype, N, K, books.get(qtype))
    err = float(np.linalg.norm(y - want) / np.linalg.norm(want))
    assert err <= 1e-4, (qtype, err)
    np.testing.assert_allclose(y, want, rtol=1e-4, atol=1e-5 * float(np.abs(want).max()))
print("plan ok", flush=True)
"""

# waves, in-flight KiB, workgroups per CU, one-slice-per-wave row limit, its waves, fill, x in LDS,
# paired items
PLANS = [
    "8,64,2,0,12,2,0,1",       # two workgroups per CU, three slices per wave everywhere, x from global
    "12,128,1,17408,12,3,1,1",  # one slice per wave for every K=5120 matrix, deeper fill
    "16,96,1,5120,9,1,1,0",    # more waves than the 3-slice variant allows (clamped), 3 row slots, no pairs
]


@pytest.mark.parametrize("plan", PLANS)
def test_qmv_parity_under_launch_plan(plan):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    env = dict(os.environ, GSQ_QMV_TUNING=plan, GSQ_ROOT=ROOT)
    r = subprocess.run([sys.executable, "-c", CHILD], env=env, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    assert "plan ok" in r.stdout
