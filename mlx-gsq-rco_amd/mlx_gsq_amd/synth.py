"""Seeded synthetic packed weights and activations for the benchmark configurations.

Payloads are uniform random bytes, which already makes every grid index, sign bit and
scale field uniform over its valid range (all bit patterns are valid). Only the fp16
scale fields are overwritten with |N(0,1)| * 0.01 so that no NaN/Inf appears:
``d@0`` for the IQ types, ``d, dmin@0,2`` for Q4_K, ``d, dmin@80,82`` for Q2_K,
``d@208`` for Q6_K, and for IQ1_M (no stored ``d``) the fp16 bits go into the top
nibbles of its four scale words (mlx_gsq/runtime/kernels/iq_lookup_decode.py:34-35).
"""
from __future__ import annotations

import numpy as np

from .formats import BLOCK_BYTES, BLOCK_ELEMENTS

_FP16_FIELDS = {
    "IQ1_S": (0,), "IQ2_XXS": (0,), "IQ2_XS": (0,), "IQ2_S": (0,), "IQ3_XXS": (0,),
    "IQ3_S": (0,), "IQ4_XS": (0,), "Q4_K": (0, 2), "Q2_K": (80, 82), "Q6_K": (208,),
}


def _scale_bits(rng, n: int) -> np.ndarray:
    return (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float16).view(np.uint16)


def make_packed(qtype: str, out_features: int, in_features: int, seed: int = 0) -> np.ndarray:
    """Random packed weight of shape ``out_features x in_features`` as flat uint8."""
    if in_features % BLOCK_ELEMENTS:
        raise ValueError("in_features must be a multiple of 256")
    bb = BLOCK_BYTES[qtype]
    nblocks = out_features * (in_features // BLOCK_ELEMENTS)
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    if qtype == "IQ1_M":
        bits = _scale_bits(rng, nblocks).astype(np.uint16)
        w = np.ascontiguousarray(raw[:, 48:56]).view("<u2").copy()
        for i in range(4):
            nib = (bits >> (4 * i)) & 0xF
            w[:, i] = (w[:, i] & 0x0FFF) | (nib << 12)
        raw[:, 48:56] = w.view(np.uint8).reshape(nblocks, 8)
    else:
        for off in _FP16_FIELDS[qtype]:
            bits = _scale_bits(rng, nblocks)
            raw[:, off:off + 2] = bits.view(np.uint8).reshape(nblocks, 2)
    return raw.reshape(-1)


def make_x(rows: int, in_features: int, seed: int = 0, dtype=np.float16) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((rows, in_features)).astype(dtype)
