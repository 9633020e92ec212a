"""Write the golden vectors of the quantized-linear path (tests/golden/golden.npz).

Produced by this repository's CPU restatement of the reference dequantizers
(oracle/gsq_oracle.py), which the closed-form tests in tests/test_oracle.py pin. The
reference ships no golden data and its own oracle (gguf-py) is not installed here, so these
vectors are a regression net for the restatement and the device path, not an independent
source. Per type: 6 seeded superblocks (the last two with raw random bytes in every field,
NaN/Inf included), their float32 dequantization under two codebooks (an index-encoding one,
grid[i][c] = i * coords + c, and the seeded synthetic one of mlx_gsq_amd.tables), and
y = x @ W.T for a 2 x 768 fp16 x against a 3 x 768 weight.

Run from the repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mlx-gsq-rco_amd")]

from mlx_gsq_amd import synth, tables  # noqa: E402
from mlx_gsq_amd.formats import GRID_SHAPES, QTYPES  # noqa: E402
from oracle import gsq_oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def index_grid(q):
    n, c = GRID_SHAPES[q]
    return (np.arange(n)[:, None] * c + np.arange(c)[None, :]).astype(np.float32)


def main():
    books = tables.synthetic_tables(0)
    data = {}
    for i, q in enumerate(QTYPES):
        packed = synth.make_packed(q, 1, 1024, seed=100 + i)              # 4 blocks, finite scales
        rng = np.random.default_rng(200 + i)
        raw = rng.integers(0, 256, 2 * O.BLOCK_BYTES[q], dtype=np.uint8)  # 2 blocks, raw bytes
        blocks = np.concatenate([packed, raw])
        data[f"{q}/packed"] = blocks
        if q in GRID_SHAPES:
            data[f"{q}/w_index_grid"] = O.dequantize_reference(blocks, q, index_grid(q))
            data[f"{q}/w_synthetic_grid"] = O.dequantize_reference(blocks, q, books[q])
        else:
            data[f"{q}/w"] = O.dequantize_reference(blocks, q)
        wpk = synth.make_packed(q, 3, 768, seed=300 + i)
        x = synth.make_x(2, 768, seed=400 + i, dtype=np.float16)
        data[f"{q}/mm_packed"] = wpk
        data[f"{q}/mm_x"] = x
        data[f"{q}/mm_y"] = O.matmul_reference(x, wpk, q, 3, 768, books.get(q))
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}: {len(data)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
