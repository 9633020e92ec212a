"""CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this module, and only as the checker / the timed CPU baseline. The product path
(``mlx_gsq_amd``) never imports it and fails loudly when the HIP library is missing.

What it restates
----------------
The reference's oracle is ``dequantize_reference`` (mlx_gsq/quant/reference.py:10-18),
which calls gguf-py's ``gguf.dequantize`` (third-party, pinned ``gguf>=0.17`` in the
reference's pyproject.toml:13; not installed in this image) on ``(nblocks, block_bytes)``
rows and flattens the float32 result. This module restates that arithmetic twice:

* ``dequantize_reference`` -- block-vectorised numpy, one function per type, following the
  reference's validated decoder kernels k_decode.py:17-81, iq_lookup_decode.py:6-39 and
  iq3_s_decode.py:7-41 (which the reference checks bit-exactly against gguf-py in
  tests/test_metal_decoders.py:9-23).
* ``dequantize_scalar`` -- an independent per-element loop for small inputs, following the
  QMM decode bodies qmm.py:38-143 (a different source text of the same formulas).

Codebooks (grids) are parameters: the real ones live in gguf-py, which is absent here.
``ksigns_table`` is the closed form of gguf-py's ``IQ2_XXS.ksigns`` (even-parity sign bytes).

Exactness: every dequantized value is a product of an fp16 scale with small integers or
codebook values and fits in fp32's 24-bit significand, so all products are exact and
results do not depend on evaluation order; Q2_K and Q4_K round once in their final
subtraction of two exact terms (the same single rounding gguf-py performs).

Pinning (see tests/test_oracle.py): closed-form special blocks for every K-quant field,
index-encoding codebooks for every grid type, the ksigns parity closed form, agreement of
the two restatements, and committed golden vectors (tests/golden/).
"""
from __future__ import annotations

import numpy as np

QTYPES = ("IQ1_M", "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS",
          "IQ3_S", "IQ4_XS", "Q2_K", "Q4_K", "Q6_K")
BLOCK_BYTES = {"IQ1_M": 56, "IQ1_S": 50, "IQ2_XXS": 66, "IQ2_XS": 74, "IQ2_S": 82,
               "IQ3_XXS": 98, "IQ3_S": 110, "IQ4_XS": 136, "Q2_K": 84, "Q4_K": 144, "Q6_K": 210}
GRID_TYPES = ("IQ1_M", "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S")
KVALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                   dtype=np.float32)  # k_decode.py:77
F32 = np.float32


def ksigns_table() -> np.ndarray:
    """128 sign bytes: bits 0-6 = index, bit 7 = parity of the index (even total parity)."""
    i = np.arange(128, dtype=np.uint8)
    par = np.array([bin(int(v)).count("1") & 1 for v in i], dtype=np.uint8)
    return (i | (par << 7)).astype(np.uint8)


def _blocks(packed, qtype: str) -> np.ndarray:
    raw = np.frombuffer(packed, dtype=np.uint8) if isinstance(packed, (bytes, bytearray)) \
        else np.asarray(packed, dtype=np.uint8).reshape(-1)
    bb = BLOCK_BYTES[qtype]
    if raw.size % bb:
        raise ValueError(f"{qtype} payload size {raw.size} is not divisible by {bb}")
    return raw.reshape(-1, bb)


def _f16(raw: np.ndarray, off: int) -> np.ndarray:
    return np.ascontiguousarray(raw[:, off:off + 2]).view(np.float16).reshape(-1).astype(F32)


def _u16(raw: np.ndarray, off: int, count: int) -> np.ndarray:
    return np.ascontiguousarray(raw[:, off:off + 2 * count]).view("<u2").astype(np.uint32)


def _u32(raw: np.ndarray, off: int, count: int) -> np.ndarray:
    return np.ascontiguousarray(raw[:, off:off + 4 * count]).view("<u4").astype(np.int64)


_E = np.arange(256)


def _q2_k(raw, grid, ks):  # k_decode.py:18-30
    chunk, in_chunk = _E // 128, _E % 128
    plane, pos = in_chunk // 32, in_chunk % 32
    q = (raw[:, 16 + chunk * 32 + pos] >> (2 * plane)) & 3
    sm = raw[:, _E // 16]
    d, dmin = _f16(raw, 80)[:, None], _f16(raw, 82)[:, None]
    return d * (sm & 15).astype(F32) * q.astype(F32) - dmin * (sm >> 4).astype(F32)


def _q4_k_scales(raw):  # k_decode.py:38-46
    s = raw[:, 4:16].astype(np.uint32)
    sc = np.empty((raw.shape[0], 8), np.uint32)
    mn = np.empty((raw.shape[0], 8), np.uint32)
    for g in range(4):
        sc[:, g] = s[:, g] & 63
        mn[:, g] = s[:, 4 + g] & 63
        sc[:, 4 + g] = (s[:, 8 + g] & 15) | ((s[:, g] >> 2) & 48)
        mn[:, 4 + g] = (s[:, 8 + g] >> 4) | ((s[:, 4 + g] >> 2) & 48)
    return sc, mn


def _q4_k(raw, grid, ks):  # k_decode.py:31-50
    group, pos = _E // 32, _E % 32
    q = (raw[:, 16 + (group // 2) * 32 + pos] >> (4 * (group & 1))) & 15
    sc, mn = _q4_k_scales(raw)
    d, dmin = _f16(raw, 0)[:, None], _f16(raw, 2)[:, None]
    return d * sc[:, group].astype(F32) * q.astype(F32) - dmin * mn[:, group].astype(F32)


def _q6_k(raw, grid, ks):  # k_decode.py:51-65
    chunk, in_chunk = _E // 128, _E % 128
    ql_half, ql_pos = in_chunk // 64, in_chunk % 64
    ql = (raw[:, chunk * 64 + ql_pos] >> (4 * ql_half)) & 15
    qh_plane, qh_pos = in_chunk // 32, in_chunk % 32
    qh = (raw[:, 128 + chunk * 32 + qh_pos] >> (2 * qh_plane)) & 3
    q = (ql.astype(np.int32) | (qh.astype(np.int32) << 4)) - 32
    scale = raw[:, 192:208].view(np.int8)[:, _E // 16].astype(np.int32)
    d = _f16(raw, 208)[:, None]
    return d * scale.astype(F32) * q.astype(F32)


def _iq4_xs(raw, grid, ks):  # k_decode.py:66-80
    group, pos = _E // 32, _E % 32
    scales_h = raw[:, 2].astype(np.uint32) | (raw[:, 3].astype(np.uint32) << 8)
    low = (raw[:, 4 + group // 2] >> (4 * (group & 1))) & 15
    high = (scales_h[:, None] >> (2 * group)) & 3
    scale = (low.astype(np.int32) | (high.astype(np.int32) << 4)) - 32
    q = (raw[:, 8 + group * 16 + (pos & 15)] >> (4 * (pos // 16))) & 15
    d = _f16(raw, 0)[:, None]
    return d * scale.astype(F32) * KVALUES[q]


def _iq3_s(raw, grid, ks):  # iq3_s_decode.py:16-40
    group, within = _E // 32, _E % 32
    lane, comp = within // 8, within % 8
    d = _f16(raw, 0)[:, None]
    sbyte = raw[:, 106 + (group >> 1)].astype(np.uint32)
    snib = np.where(group & 1, sbyte >> 4, sbyte & 15)
    db = d * (1 + 2 * snib).astype(F32)
    qbase = group * 8 + lane * 2
    qh = raw[:, 66 + group].astype(np.uint32)
    lo = raw[:, 2 + qbase].astype(np.uint32) | ((qh << (8 - 2 * lane)) & 256)
    hi = raw[:, 2 + qbase + 1].astype(np.uint32) | ((qh << (7 - 2 * lane)) & 256)
    gi = np.where(comp < 4, lo, hi)
    mag = grid.reshape(-1)[gi * 4 + (comp & 3)]
    neg = (raw[:, 74 + group * 4 + lane].astype(np.uint32) >> comp) & 1
    return np.where(neg != 0, -db * mag, db * mag)


def _iq3_xxs(raw, grid, ks):  # iq_lookup_decode.py:7-12
    g, p = _E // 32, _E % 32
    l, c = p // 8, p % 8
    u = _u32(raw, 66, 8)[:, g]
    d = _f16(raw, 0)[:, None] * (F32(0.5) + (u >> 28).astype(F32)) * F32(0.5)
    si = (u >> (7 * l)) & 127
    neg = (ks[si].astype(np.uint32) >> c) & 1
    qi = raw[:, 2 + g * 8 + l * 2 + (c >= 4)].astype(np.uint32)
    v = grid.reshape(-1)[qi * 4 + (c & 3)]
    return np.where(neg != 0, -d * v, d * v)


def _iq2_xs(raw, grid, ks):  # iq_lookup_decode.py:13-17
    g, p = _E // 16, _E % 16
    sub, c = p // 8, p % 8
    o = g * 2 + sub
    q = _u16(raw, 2, 32)[:, o]
    sb = raw[:, 66 + g // 2].astype(np.uint32)
    sc = (sb >> (4 * (g & 1))) & 15
    d = _f16(raw, 0)[:, None] * (F32(0.5) + sc.astype(F32)) * F32(0.25)
    neg = (ks[(q >> 9) & 127].astype(np.uint32) >> c) & 1
    v = grid.reshape(-1)[(q & 511) * 8 + c]
    return np.where(neg != 0, -d * v, d * v)


def _iq2_s(raw, grid, ks):  # iq_lookup_decode.py:18-22
    g, p = _E // 16, _E % 16
    sub, c = p // 8, p % 8
    o = g * 2 + sub
    hi = (raw[:, 66 + o // 4].astype(np.uint32) >> (2 * (o & 3))) & 3
    qi = raw[:, 2 + o].astype(np.uint32) | (hi << 8)
    sb = raw[:, 74 + g // 2].astype(np.uint32)
    sc = (sb >> (4 * (g & 1))) & 15
    d = _f16(raw, 0)[:, None] * (F32(0.5) + sc.astype(F32)) * F32(0.25)
    neg = (raw[:, 34 + o].astype(np.uint32) >> c) & 1
    v = grid.reshape(-1)[qi * 8 + c]
    return np.where(neg != 0, -d * v, d * v)


def _iq2_xxs(raw, grid, ks):  # iq_lookup_decode.py:23-26
    g, p = _E // 32, _E % 32
    l, c = p // 8, p % 8
    u = np.stack([_u32(raw, 2 + gg * 8 + 4, 1)[:, 0] for gg in range(8)], axis=1)[:, g]
    d = _f16(raw, 0)[:, None] * (F32(0.5) + (u >> 28).astype(F32)) * F32(0.25)
    si = (u >> (7 * l)) & 127
    neg = (ks[si].astype(np.uint32) >> c) & 1
    qi = raw[:, 2 + g * 8 + l].astype(np.uint32)
    v = grid.reshape(-1)[qi * 8 + c]
    return np.where(neg != 0, -d * v, d * v)


def _iq1_s(raw, grid, ks):  # iq_lookup_decode.py:27-30
    g, p = _E // 32, _E % 32
    l, c = p // 8, p % 8
    h = _u16(raw, 34, 8)[:, g]
    qi = raw[:, 2 + g * 4 + l].astype(np.uint32) | (((h >> (3 * l)) & 7) << 8)
    d = _f16(raw, 0)[:, None] * (2 * ((h >> 12) & 7) + 1).astype(F32)
    delta = np.where(h & 32768, F32(-0.125), F32(0.125))
    return d * (grid.reshape(-1)[qi * 8 + c] + delta)


def _iq1_m_d(raw):  # iq_lookup_decode.py:34-35
    w = _u16(raw, 48, 4)
    bits = ((w[:, 0] & 61440) >> 12) | ((w[:, 1] & 61440) >> 8) | ((w[:, 2] & 61440) >> 4) | (w[:, 3] & 61440)
    return bits.astype(np.uint16).view(np.float16).astype(F32)


def _iq1_m(raw, grid, ks):  # iq_lookup_decode.py:31-37
    g, p = _E // 32, _E % 32
    sg, r = p // 16, p % 16
    sub, c = r // 8, r % 8
    o = g * 4 + sg * 2 + sub
    hb = raw[:, 32 + o // 2].astype(np.uint32)
    hn = (hb >> (4 * (o & 1))) & 15
    qi = raw[:, o].astype(np.uint32) | ((hn & 7) << 8)
    delta = np.where(hn & 8, F32(-0.125), F32(0.125))
    w = _u16(raw, 48, 4)
    d = _iq1_m_d(raw)[:, None]
    sci = g * 2 + sg
    sc = (w[:, sci // 4] >> (3 * (sci & 3))) & 7
    return d * (2 * sc + 1).astype(F32) * (grid.reshape(-1)[qi * 8 + c] + delta)


_DECODERS = {"Q2_K": _q2_k, "Q4_K": _q4_k, "Q6_K": _q6_k, "IQ4_XS": _iq4_xs,
             "IQ3_S": _iq3_s, "IQ3_XXS": _iq3_xxs, "IQ2_XS": _iq2_xs, "IQ2_S": _iq2_s,
             "IQ2_XXS": _iq2_xxs, "IQ1_S": _iq1_s, "IQ1_M": _iq1_m}


def _check_tables(qtype, grid, ksigns):
    if qtype in GRID_TYPES and grid is None:
        raise ValueError(f"{qtype} needs its codebook (grid) as a parameter")
    g = None if grid is None else np.asarray(grid, dtype=F32)
    ks = ksigns_table() if ksigns is None else np.asarray(ksigns, dtype=np.uint8)
    return g, ks


def dequantize_reference(packed, qtype: str, grid=None, ksigns=None) -> np.ndarray:
    """Packed superblocks -> flat float32 weights (contract of reference.py:10-18)."""
    if qtype not in _DECODERS:
        raise NotImplementedError(qtype)
    raw = _blocks(packed, qtype)
    g, ks = _check_tables(qtype, grid, ksigns)
    with np.errstate(over="ignore", invalid="ignore"):
        out = _DECODERS[qtype](raw, g, ks)
    return np.asarray(out, dtype=F32).reshape(-1)


# ----------------------------------------------------------------------------------------
# Second restatement: one element at a time, following the QMM decode bodies qmm.py:38-143.
# ----------------------------------------------------------------------------------------
def _h(b, off):
    return float(np.frombuffer(bytes(b[off:off + 2]), dtype=np.float16)[0])


def _scalar_value(qtype, b, g, p, grid, ks):
    f32 = np.float32
    if qtype == "IQ1_M":  # qmm.py:39-50
        sg, r = p // 16, p % 16
        sub, c = r // 8, r % 8
        o = g * 4 + sg * 2 + sub
        hn = (int(b[32 + o // 2]) >> (4 * (o & 1))) & 15
        qi = int(b[o]) | ((hn & 7) << 8)
        delta = -0.125 if hn & 8 else 0.125
        w = [int(b[48 + 2 * i]) | (int(b[49 + 2 * i]) << 8) for i in range(4)]
        dbits = ((w[0] & 61440) >> 12) | ((w[1] & 61440) >> 8) | ((w[2] & 61440) >> 4) | (w[3] & 61440)
        d = float(np.array([dbits], np.uint16).view(np.float16)[0])
        sci = g * 2 + sg
        sc = (w[sci // 4] >> (3 * (sci & 3))) & 7
        return f32(f32(d) * f32(2 * sc + 1)) * f32(f32(grid[qi][c]) + f32(delta))
    if qtype == "IQ1_S":  # qmm.py:51-57
        l, c = p // 8, p % 8
        h = int(b[34 + g * 2]) | (int(b[35 + g * 2]) << 8)
        qi = int(b[2 + g * 4 + l]) | (((h >> (3 * l)) & 7) << 8)
        d = f32(_h(b, 0)) * f32(2 * ((h >> 12) & 7) + 1)
        delta = -0.125 if h & 32768 else 0.125
        return d * f32(f32(grid[qi][c]) + f32(delta))
    if qtype == "IQ2_XXS":  # qmm.py:58-65
        l, c = p // 8, p % 8
        q = b[2 + g * 8: 2 + g * 8 + 8]
        u = int(q[4]) | (int(q[5]) << 8) | (int(q[6]) << 16) | (int(q[7]) << 24)
        d = f32(_h(b, 0)) * f32(0.5 + (u >> 28)) * f32(0.25)
        neg = (int(ks[(u >> (7 * l)) & 127]) >> c) & 1
        v = f32(grid[int(q[l])][c])
        return -d * v if neg else d * v
    if qtype in ("IQ2_XS", "IQ2_S"):  # qmm.py:66-80
        e = g * 32 + p
        gg, pp = e // 16, e % 16
        sub, c = pp // 8, pp % 8
        o = gg * 2 + sub
        if qtype == "IQ2_XS":
            q = int(b[2 + o * 2]) | (int(b[3 + o * 2]) << 8)
            sc = (int(b[66 + gg // 2]) >> (4 * (gg & 1))) & 15
            neg = (int(ks[(q >> 9) & 127]) >> c) & 1
            qi = q & 511
        else:
            hi = (int(b[66 + o // 4]) >> (2 * (o & 3))) & 3
            qi = int(b[2 + o]) | (hi << 8)
            sc = (int(b[74 + gg // 2]) >> (4 * (gg & 1))) & 15
            neg = (int(b[34 + o]) >> c) & 1
        d = f32(_h(b, 0)) * f32(0.5 + sc) * f32(0.25)
        v = f32(grid[qi][c])
        return -d * v if neg else d * v
    if qtype == "IQ3_XXS":  # qmm.py:81-88
        l, c = p // 8, p % 8
        u = sum(int(b[66 + g * 4 + i]) << (8 * i) for i in range(4))
        d = f32(_h(b, 0)) * f32(0.5 + (u >> 28)) * f32(0.5)
        neg = (int(ks[(u >> (7 * l)) & 127]) >> c) & 1
        qi = int(b[2 + g * 8 + l * 2 + (1 if c >= 4 else 0)])
        v = f32(grid[qi][c & 3])
        return -d * v if neg else d * v
    if qtype == "IQ3_S":  # qmm.py:89-101
        l, c = p // 8, p % 8
        sbyte = int(b[106 + (g >> 1)])
        snib = (sbyte >> 4) if (g & 1) else (sbyte & 15)
        db = f32(_h(b, 0)) * f32(1 + 2 * snib)
        qh = int(b[66 + g])
        if c < 4:
            gi = int(b[2 + g * 8 + l * 2]) | ((qh << (8 - 2 * l)) & 256)
        else:
            gi = int(b[2 + g * 8 + l * 2 + 1]) | ((qh << (7 - 2 * l)) & 256)
        neg = (int(b[74 + g * 4 + l]) >> c) & 1
        mag = f32(grid[gi][c & 3])
        return -db * mag if neg else db * mag
    if qtype == "IQ4_XS":  # qmm.py:102-110
        scales_h = int(b[2]) | (int(b[3]) << 8)
        low = (int(b[4 + g // 2]) >> (4 * (g & 1))) & 15
        high = (scales_h >> (2 * g)) & 3
        scale = (low | (high << 4)) - 32
        q = (int(b[8 + g * 16 + (p & 15)]) >> (4 * (p // 16))) & 15
        return f32(_h(b, 0)) * f32(scale) * KVALUES[q]
    if qtype == "Q2_K":  # qmm.py:111-118
        e = g * 32 + p
        chunk, in_chunk = e // 128, e % 128
        plane, pos = in_chunk // 32, in_chunk % 32
        q = (int(b[16 + chunk * 32 + pos]) >> (2 * plane)) & 3
        sm = int(b[e // 16])
        return f32(_h(b, 80)) * f32(sm & 15) * f32(q) - f32(_h(b, 82)) * f32(sm >> 4)
    if qtype == "Q4_K":  # qmm.py:119-132
        s = b[4:16]
        q = (int(b[16 + (g // 2) * 32 + p]) >> (4 * (g & 1))) & 15
        if g < 4:
            sc, mn = int(s[g]) & 63, int(s[4 + g]) & 63
        else:
            gg = g - 4
            sc = (int(s[8 + gg]) & 15) | ((int(s[gg]) >> 2) & 48)
            mn = (int(s[8 + gg]) >> 4) | ((int(s[4 + gg]) >> 2) & 48)
        return f32(_h(b, 0)) * f32(sc) * f32(q) - f32(_h(b, 2)) * f32(mn)
    if qtype == "Q6_K":  # qmm.py:133-142
        e = g * 32 + p
        chunk, in_chunk = e // 128, e % 128
        ql_half, ql_pos = in_chunk // 64, in_chunk % 64
        ql = (int(b[chunk * 64 + ql_pos]) >> (4 * ql_half)) & 15
        qh_plane, qh_pos = in_chunk // 32, in_chunk % 32
        qh = (int(b[128 + chunk * 32 + qh_pos]) >> (2 * qh_plane)) & 3
        q = (ql | (qh << 4)) - 32
        scale = int(np.int8(np.uint8(b[192 + e // 16])))
        return f32(_h(b, 208)) * f32(scale) * f32(q)
    raise NotImplementedError(qtype)


def dequantize_scalar(packed, qtype: str, grid=None, ksigns=None) -> np.ndarray:
    """Element-by-element restatement (slow; for a few blocks)."""
    raw = _blocks(packed, qtype)
    g, ks = _check_tables(qtype, grid, ksigns)
    grid2 = None if g is None else g.reshape(g.shape[0], -1)
    out = np.empty(raw.shape[0] * 256, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        for bi in range(raw.shape[0]):
            b = raw[bi]
            for e in range(256):
                out[bi * 256 + e] = _scalar_value(qtype, b, e // 32, e % 32, grid2, ks)
    return out


def matmul_reference(x, packed, qtype: str, out_features: int, in_features: int,
                     grid=None, ksigns=None) -> np.ndarray:
    """y = x_f32 @ dequant(W).T in float32 (reference tests/test_all_qmv.py:22)."""
    w = dequantize_reference(packed, qtype, grid, ksigns).reshape(out_features, in_features)
    xf = np.asarray(x, dtype=F32).reshape(-1, in_features)
    return xf @ w.T
