"""Codebooks (lookup grids) of the IQ formats and the ksigns table.

The reference takes its codebooks from gguf-py at runtime
(``gguf.quants.<T>.init_grid()``, ``IQ2_XXS.ksigns``; mlx_gsq/runtime/kernels/
iq_lookup_decode.py:46-53, iq3_s_decode.py:56-61, mlx_gsq/quant/reference.py:21-27) and
passes them to its kernels as runtime buffers. This module does the same: kernels never
embed codebook content, they receive it through ``gsq_set_tables``.

Codebook sources, in order:

1. tables registered explicitly with :func:`set_tables` (or :func:`use_tables`);
2. gguf-py (``gguf>=0.17``), when it is importable -- the reference's own source;
3. a ``.npz`` file named by the ``GSQ_CODEBOOKS`` environment variable, holding one
   ``(entries, coords)`` float32 array per type name (e.g. ``IQ2_XS``).

If none provides a codebook, the grid types raise ``RuntimeError``; nothing falls back
to made-up values. :func:`synthetic_tables` builds tables with the published shapes and
value sets for benchmarks and tests; they are not the real codebooks and must be
registered explicitly.

``ksigns`` has a closed form: entry ``i`` is ``i`` with bit 7 set to the parity of ``i``
(every sign byte has an even number of negative signs).
"""
from __future__ import annotations

import os

import numpy as np

from .formats import GRID_SHAPES, GRID_SOURCE, GRID_VALUE_SETS

_registered: dict[str, np.ndarray] = {}
_uploaded_versions: dict = {}
_version = 0


def ksigns() -> np.ndarray:
    i = np.arange(128, dtype=np.uint8)
    parity = np.array([bin(int(v)).count("1") & 1 for v in range(128)], dtype=np.uint8)
    return (i | (parity << 7)).astype(np.uint8)


def validate_grid(qtype: str, grid) -> np.ndarray:
    """Check a codebook against the invariants every published table satisfies."""
    src = GRID_SOURCE.get(qtype, qtype)
    if src not in GRID_SHAPES:
        raise KeyError(qtype)
    g = np.asarray(grid, dtype=np.float32)
    shape = GRID_SHAPES[src]
    if g.size != shape[0] * shape[1]:
        raise ValueError(f"{qtype} codebook must have {shape[0]}x{shape[1]} values, got {g.shape}")
    g = g.reshape(shape)
    allowed = np.array(GRID_VALUE_SETS[src], dtype=np.float32)
    if not np.isin(g, allowed).all():
        bad = np.unique(g[~np.isin(g, allowed)])[:8]
        raise ValueError(f"{qtype} codebook holds values outside {tuple(allowed)}: {bad}")
    if len(np.unique(g, axis=0)) != shape[0]:
        raise ValueError(f"{qtype} codebook entries are not unique")
    return np.ascontiguousarray(g)


def _from_gguf(qtype: str):
    try:
        from gguf import quants  # type: ignore
    except Exception:
        return None
    cls = getattr(quants, GRID_SOURCE.get(qtype, qtype), None)
    if cls is None:
        return None
    cls.init_grid()
    return np.asarray(cls.grid, dtype=np.float32).reshape(GRID_SHAPES[qtype])


def _from_file(qtype: str):
    path = os.environ.get("GSQ_CODEBOOKS")
    if not path:
        return None
    with np.load(path, allow_pickle=False) as f:
        name = qtype if qtype in f.files else GRID_SOURCE.get(qtype, qtype)
        if name not in f.files:
            return None
        return np.asarray(f[name], dtype=np.float32)


def set_tables(tables: dict) -> None:
    """Register codebooks ``{qtype: (entries, coords) array}`` for the device kernels."""
    global _version
    for q, g in tables.items():
        _registered[q] = validate_grid(q, g)
    for q, src in GRID_SOURCE.items():
        if src in tables and q not in tables:
            _registered[q] = _registered[src]
    _version += 1


def clear_tables() -> None:
    global _version
    _registered.clear()
    _version += 1


def grid(qtype: str) -> np.ndarray:
    """The codebook for ``qtype`` from the first available source (see module doc)."""
    if qtype in _registered:
        return _registered[qtype]
    for source in (_from_gguf, _from_file):
        g = source(qtype)
        if g is not None:
            _registered[qtype] = validate_grid(qtype, g)
            return _registered[qtype]
    raise RuntimeError(
        f"no codebook for {qtype}: install gguf>=0.17, set GSQ_CODEBOOKS=<file.npz>, "
        "or register one with mlx_gsq_amd.tables.set_tables")


def version() -> int:
    return _version


def synthetic_tables(seed: int = 0) -> dict:
    """Seeded codebooks with the published shapes and value sets (NOT the real grids).

    Entries are unique and sorted by their packed code, like the published tables.
    For benchmarks and tests of the indexing, sign and scale arithmetic.
    """
    rng = np.random.default_rng(seed)
    out = {}
    for q in ("IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S"):
        n, c = GRID_SHAPES[q]
        vals = np.array(GRID_VALUE_SETS[q], dtype=np.float32)
        k = len(vals)
        codes = rng.choice(k ** c, size=n, replace=False)
        codes.sort()
        digits = (codes[:, None] // (k ** np.arange(c)[None, :])) % k
        out[q] = vals[digits].astype(np.float32)
    out["IQ1_M"] = out["IQ1_S"]
    return out
