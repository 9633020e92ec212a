"""Pins for the CPU oracle (oracle/gsq_oracle.py); CPU only.

Each test builds blocks with a field *encoder* written from the superblock layout (the
inverse direction of the decoders under test), chooses scales so that the expected
weights are small integers or exact binary fractions, and checks the oracle decodes
exactly what was encoded. Grid types use index-encoding codebooks
(``grid[i][c] = i * coords + c``) so a wrong index or coordinate gives a wrong value.
A planted mistake in any index, shift or sign of the oracle fails at least one test.
"""
import numpy as np
import pytest

from oracle import gsq_oracle as O

RNG = np.random.default_rng(1234)


def f16b(v):
    return np.array([v], np.float16).view(np.uint8)


def index_grid(q):
    n, c = {"IQ1_S": (2048, 8), "IQ1_M": (2048, 8), "IQ2_XXS": (256, 8), "IQ2_XS": (512, 8),
            "IQ2_S": (1024, 8), "IQ3_XXS": (256, 4), "IQ3_S": (512, 4)}[q]
    return (np.arange(n)[:, None] * c + np.arange(c)[None, :]).astype(np.float32)


def test_ksigns_closed_form():
    ks = O.ksigns_table()
    assert list(ks[:8]) == [0, 129, 130, 3, 132, 5, 6, 135]
    assert all(bin(int(v)).count("1") % 2 == 0 for v in ks)
    assert list(ks & 127) == list(range(128))


# ------------------------------- K-quants --------------------------------------------
def enc_q4k_scales(sc, mn):
    b = np.zeros(12, np.uint8)
    for j in range(4):
        b[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return b


def enc_q4k(d, dmin, sc, mn, q):
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = f16b(d), f16b(dmin)
    b[4:16] = enc_q4k_scales(sc, mn)
    for e in range(256):
        g, p = divmod(e, 32)
        b[16 + (g // 2) * 32 + p] |= (q[e] & 15) << (4 * (g & 1))
    return b


def test_q4_k_fields():
    sc = RNG.integers(0, 64, 8)
    mn = RNG.integers(0, 64, 8)
    q = RNG.integers(0, 16, 256)
    g = np.arange(256) // 32
    w = O.dequantize_reference(enc_q4k(1.0, 0.0, sc, mn, q), "Q4_K")
    np.testing.assert_array_equal(w, (sc[g] * q).astype(np.float32))
    w = O.dequantize_reference(enc_q4k(0.0, 1.0, sc, mn, q), "Q4_K")
    np.testing.assert_array_equal(w, (-mn[g]).astype(np.float32))
    w = O.dequantize_reference(enc_q4k(0.5, 0.25, sc, mn, q), "Q4_K")
    np.testing.assert_array_equal(w, (0.5 * sc[g] * q - 0.25 * mn[g]).astype(np.float32))


def enc_q2k(d, dmin, sc, mn, q):
    b = np.zeros(84, np.uint8)
    b[0:16] = (sc & 15) | ((mn & 15) << 4)
    for e in range(256):
        chunk, r = divmod(e, 128)
        plane, pos = divmod(r, 32)
        b[16 + chunk * 32 + pos] |= (q[e] & 3) << (2 * plane)
    b[80:82], b[82:84] = f16b(d), f16b(dmin)
    return b


def test_q2_k_fields():
    sc, mn, q = RNG.integers(0, 16, 16), RNG.integers(0, 16, 16), RNG.integers(0, 4, 256)
    s = np.arange(256) // 16
    w = O.dequantize_reference(enc_q2k(1.0, 1.0, sc, mn, q), "Q2_K")
    np.testing.assert_array_equal(w, (sc[s] * q - mn[s]).astype(np.float32))


def enc_q6k(d, scales, q):
    b = np.zeros(210, np.uint8)
    v = (q + 32).astype(np.uint8)
    for e in range(256):
        chunk, r = divmod(e, 128)
        half, lpos = divmod(r, 64)
        b[chunk * 64 + lpos] |= (v[e] & 15) << (4 * half)
        plane, hpos = divmod(r, 32)
        b[128 + chunk * 32 + hpos] |= (v[e] >> 4) << (2 * plane)
    b[192:208] = scales.astype(np.int8).view(np.uint8)
    b[208:210] = f16b(d)
    return b


def test_q6_k_fields():
    scales, q = RNG.integers(-128, 128, 16), RNG.integers(-32, 32, 256)
    w = O.dequantize_reference(enc_q6k(1.0, scales, q), "Q6_K")
    np.testing.assert_array_equal(w, (scales[np.arange(256) // 16] * q).astype(np.float32))
    # ql = qh = 0 gives q = -32 everywhere
    b = enc_q6k(0.5, scales, np.full(256, -32))
    np.testing.assert_array_equal(O.dequantize_reference(b, "Q6_K"),
                                  (-16.0 * scales[np.arange(256) // 16]).astype(np.float32))


def enc_iq4xs(d, scale6, q):
    b = np.zeros(136, np.uint8)
    b[0:2] = f16b(d)
    sh = 0
    for g in range(8):
        b[4 + g // 2] |= (scale6[g] & 15) << (4 * (g & 1))
        sh |= int(scale6[g] >> 4) << (2 * g)
    b[2], b[3] = sh & 255, sh >> 8
    for e in range(256):
        g, p = divmod(e, 32)
        b[8 + g * 16 + (p & 15)] |= (q[e] & 15) << (4 * (p // 16))
    return b


def test_iq4_xs_fields():
    scale6, q = RNG.integers(0, 64, 8), RNG.integers(0, 16, 256)
    w = O.dequantize_reference(enc_iq4xs(1.0, scale6, q), "IQ4_XS")
    kv = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113])
    np.testing.assert_array_equal(w, ((scale6[np.arange(256) // 32] - 32) * kv[q]).astype(np.float32))


# ------------------------------- grid types ------------------------------------------
def test_iq3_s_fields():
    idx = RNG.integers(0, 512, 64)   # entry per 4 elements
    sgn = RNG.integers(0, 2, 256)
    nib = RNG.integers(0, 16, 8)
    b = np.zeros(110, np.uint8)
    b[0:2] = f16b(1.0)
    for g in range(8):
        for e in range(8):
            k = g * 8 + e
            b[2 + k] = idx[k] & 255
            b[66 + g] |= (idx[k] >> 8) << e
    for i in range(256):
        b[74 + i // 8] |= sgn[i] << (i % 8)
    for g in range(8):
        b[106 + g // 2] |= nib[g] << (4 * (g & 1))
    grid = index_grid("IQ3_S")
    w = O.dequantize_reference(b, "IQ3_S", grid)
    e = np.arange(256)
    expect = (1 + 2 * nib[e // 32]) * grid[idx[e // 4], e % 4] * np.where(sgn == 1, -1, 1)
    np.testing.assert_array_equal(w, expect.astype(np.float32))


def test_iq3_xxs_fields():
    ks = O.ksigns_table()
    idx = RNG.integers(0, 256, 64)
    sidx = RNG.integers(0, 128, 32)
    sc = RNG.integers(0, 16, 8)
    b = np.zeros(98, np.uint8)
    b[0:2] = f16b(2.0)
    b[2:66] = idx
    for g in range(8):
        u = int(sc[g]) << 28
        for l in range(4):
            u |= int(sidx[g * 4 + l]) << (7 * l)
        b[66 + 4 * g: 70 + 4 * g] = np.array([u], "<u4").view(np.uint8)
    grid = index_grid("IQ3_XXS")
    w = O.dequantize_reference(b, "IQ3_XXS", grid)
    e = np.arange(256)
    signs = (ks[sidx[e // 8]] >> (e % 8)) & 1
    expect = (0.5 + sc[e // 32]) * grid[idx[e // 4], e % 4] * np.where(signs == 1, -1, 1)
    np.testing.assert_array_equal(w, expect.astype(np.float32))


def test_iq2_xxs_fields():
    ks = O.ksigns_table()
    idx = RNG.integers(0, 256, 32)
    sidx = RNG.integers(0, 128, 32)
    sc = RNG.integers(0, 16, 8)
    b = np.zeros(66, np.uint8)
    b[0:2] = f16b(4.0)
    for g in range(8):
        b[2 + 8 * g: 6 + 8 * g] = idx[4 * g: 4 * g + 4]
        u = int(sc[g]) << 28
        for l in range(4):
            u |= int(sidx[g * 4 + l]) << (7 * l)
        b[6 + 8 * g: 10 + 8 * g] = np.array([u], "<u4").view(np.uint8)
    grid = index_grid("IQ2_XXS")
    w = O.dequantize_reference(b, "IQ2_XXS", grid)
    e = np.arange(256)
    signs = (ks[sidx[e // 8]] >> (e % 8)) & 1
    expect = (0.5 + sc[e // 32]) * grid[idx[e // 8], e % 8] * np.where(signs == 1, -1, 1)
    np.testing.assert_array_equal(w, expect.astype(np.float32))


def test_iq2_xs_fields():
    ks = O.ksigns_table()
    idx = RNG.integers(0, 512, 32)
    sidx = RNG.integers(0, 128, 32)
    sc = RNG.integers(0, 16, 16)
    b = np.zeros(74, np.uint8)
    b[0:2] = f16b(4.0)
    q = (idx | (sidx << 9)).astype("<u2")
    b[2:66] = q.view(np.uint8)
    for s in range(16):
        b[66 + s // 2] |= sc[s] << (4 * (s & 1))
    grid = index_grid("IQ2_XS")
    w = O.dequantize_reference(b, "IQ2_XS", grid)
    e = np.arange(256)
    signs = (ks[sidx[e // 8]] >> (e % 8)) & 1
    expect = (0.5 + sc[e // 16]) * grid[idx[e // 8], e % 8] * np.where(signs == 1, -1, 1)
    np.testing.assert_array_equal(w, expect.astype(np.float32))


def test_iq2_s_fields():
    idx = RNG.integers(0, 1024, 32)
    sbytes = RNG.integers(0, 256, 32)
    sc = RNG.integers(0, 16, 16)
    b = np.zeros(82, np.uint8)
    b[0:2] = f16b(4.0)
    b[2:34] = idx & 255
    b[34:66] = sbytes
    for o in range(32):
        b[66 + o // 4] |= (idx[o] >> 8) << (2 * (o & 3))
    for s in range(16):
        b[74 + s // 2] |= sc[s] << (4 * (s & 1))
    grid = index_grid("IQ2_S")
    w = O.dequantize_reference(b, "IQ2_S", grid)
    e = np.arange(256)
    signs = (sbytes[e // 8] >> (e % 8)) & 1
    expect = (0.5 + sc[e // 16]) * grid[idx[e // 8], e % 8] * np.where(signs == 1, -1, 1)
    np.testing.assert_array_equal(w, expect.astype(np.float32))


def test_iq1_s_fields():
    idx = RNG.integers(0, 2048, 32)
    sc = RNG.integers(0, 8, 8)
    neg = RNG.integers(0, 2, 8)
    b = np.zeros(50, np.uint8)
    b[0:2] = f16b(1.0)
    b[2:34] = idx & 255
    for g in range(8):
        h = int(sc[g]) << 12 | int(neg[g]) << 15
        for l in range(4):
            h |= int(idx[4 * g + l] >> 8) << (3 * l)
        b[34 + 2 * g: 36 + 2 * g] = np.array([h], "<u2").view(np.uint8)
    grid = index_grid("IQ1_S")
    w = O.dequantize_reference(b, "IQ1_S", grid)
    e = np.arange(256)
    delta = np.where(neg[e // 32] == 1, -0.125, 0.125)
    expect = (2 * sc[e // 32] + 1) * (grid[idx[e // 8], e % 8] + delta)
    np.testing.assert_array_equal(w, expect.astype(np.float32))


def test_iq1_m_fields():
    idx = RNG.integers(0, 2048, 32)
    neg = RNG.integers(0, 2, 32)
    sc = RNG.integers(0, 8, 16)
    dbits = int(np.array([0.75], np.float16).view(np.uint16)[0])
    b = np.zeros(56, np.uint8)
    b[0:32] = idx & 255
    for o in range(32):
        nib = int(idx[o] >> 8) | (int(neg[o]) << 3)
        b[32 + o // 2] |= nib << (4 * (o & 1))
    words = np.zeros(4, np.uint32)
    for s in range(16):
        words[s // 4] |= int(sc[s]) << (3 * (s % 4))
    for i in range(4):
        words[i] |= ((dbits >> (4 * i)) & 15) << 12
    b[48:56] = words.astype("<u2").view(np.uint8)
    grid = index_grid("IQ1_M")
    w = O.dequantize_reference(b, "IQ1_M", grid)
    e = np.arange(256)
    delta = np.where(neg[e // 8] == 1, -0.125, 0.125)
    expect = 0.75 * (2 * sc[e // 16] + 1) * (grid[idx[e // 8], e % 8] + delta)
    np.testing.assert_array_equal(w, expect.astype(np.float32))


# ------------------------------- cross-checks ----------------------------------------
@pytest.mark.parametrize("qtype", O.QTYPES)
def test_vectorised_matches_scalar(qtype):
    raw = RNG.integers(0, 256, 3 * O.BLOCK_BYTES[qtype], dtype=np.uint8)
    grid = index_grid(qtype) if qtype in O.GRID_TYPES else None
    a = O.dequantize_reference(raw, qtype, grid)
    b = O.dequantize_scalar(raw, qtype, grid)
    np.testing.assert_array_equal(a[np.isfinite(a)], b[np.isfinite(a)])
    assert np.array_equal(np.isfinite(a), np.isfinite(b))


def test_block_alignment_error():
    with pytest.raises(ValueError):
        O.dequantize_reference(np.zeros(145, np.uint8), "Q4_K")


def test_matmul_reference_is_dense_product():
    raw = RNG.integers(0, 256, 2 * 2 * 144, dtype=np.uint8)
    raw.reshape(-1, 144)[:, 0:4] = np.frombuffer(np.array([0.01, 0.02], np.float16).tobytes(), np.uint8)
    x = RNG.standard_normal((3, 512)).astype(np.float32)
    w = O.dequantize_reference(raw, "Q4_K").reshape(2, 512)
    y = O.matmul_reference(x, raw, "Q4_K", 2, 512)
    np.testing.assert_allclose(y, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-5, atol=1e-5)
