"""GGUF superblock formats handled by the quantized-linear path.

Every supported type packs 256 weights into one superblock of ``BLOCK_BYTES[qtype]``
bytes. Type ids and block sizes are GGML's published type traits, the same table the
reference validates against (mlx_gsq/gguf/parser.py:26-42).

Byte layouts (offsets inside one superblock) follow the reference decoders
mlx_gsq/runtime/kernels/k_decode.py:18-80, iq_lookup_decode.py:6-39 and
iq3_s_decode.py:16-40:

=======  ====  ===========================================================================
type     bb    fields
=======  ====  ===========================================================================
Q2_K     84    scales[16]@0 (lo nibble scale, hi nibble min per 16), qs[64]@16, d@80, dmin@82
Q4_K     144   d@0, dmin@2, scales[12]@4 (6-bit packed), qs[128]@16
Q6_K     210   ql[128]@0, qh[64]@128, scales int8[16]@192, d@208
IQ4_XS   136   d@0, scales_h u16@2, scales_l[4]@4, qs[128]@8
IQ3_S    110   d@0, qs[64]@2, qh[8]@66, signs[32]@74, scales[4]@106
IQ3_XXS  98    d@0, qs[64]@2, aux u32[8]@66
IQ2_XXS  66    d@0, then per 32-group 8 bytes: 4 grid bytes + u32 aux
IQ2_XS   74    d@0, qs u16[32]@2, scales[8]@66
IQ2_S    82    d@0, qs[32]@2, signs[32]@34, qh[8]@66, scales[8]@74
IQ1_S    50    d@0, qs[32]@2, qh u16[8]@34
IQ1_M    56    qs[32]@0, qh[16]@32, scales u16[4]@48 (fp16 d in the top nibbles)
=======  ====  ===========================================================================
"""
from __future__ import annotations

QTYPES = ("IQ1_M", "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS",
          "IQ3_S", "IQ4_XS", "Q2_K", "Q4_K", "Q6_K")

TYPE_IDS = {
    "Q2_K": 10, "Q4_K": 12, "Q6_K": 14, "IQ2_XXS": 16, "IQ2_XS": 17,
    "IQ3_XXS": 18, "IQ1_S": 19, "IQ3_S": 21, "IQ2_S": 22, "IQ4_XS": 23, "IQ1_M": 29,
}
TYPE_NAMES = {v: k for k, v in TYPE_IDS.items()}

BLOCK_ELEMENTS = 256
BLOCK_BYTES = {
    "IQ1_M": 56, "IQ1_S": 50, "IQ2_XXS": 66, "IQ2_XS": 74, "IQ2_S": 82,
    "IQ3_XXS": 98, "IQ3_S": 110, "IQ4_XS": 136, "Q2_K": 84, "Q4_K": 144, "Q6_K": 210,
}

# Codebook shape per grid type: (entries, coordinates). The entry count is fixed by
# the index width each format stores (8, 9, 10 or 11 bits).
GRID_SHAPES = {
    "IQ1_S": (2048, 8), "IQ1_M": (2048, 8), "IQ2_XXS": (256, 8), "IQ2_XS": (512, 8),
    "IQ2_S": (1024, 8), "IQ3_XXS": (256, 4), "IQ3_S": (512, 4),
}
# Coordinate values each published codebook draws from. They are the only values the
# device tables accept, which keeps every table entry exact in fp16.
GRID_VALUE_SETS = {
    "IQ1_S": (-1.0, 0.0, 1.0), "IQ1_M": (-1.0, 0.0, 1.0),
    "IQ2_XXS": (8.0, 25.0, 43.0), "IQ2_XS": (8.0, 25.0, 43.0),
    "IQ2_S": (8.0, 25.0, 43.0, 62.0),
    "IQ3_XXS": (4.0, 12.0, 20.0, 28.0, 36.0, 44.0, 52.0, 62.0),
    "IQ3_S": (1.0, 3.0, 5.0, 7.0, 9.0, 11.0, 13.0, 15.0),
}
# IQ1_M decodes against the IQ1_S codebook.
GRID_SOURCE = {"IQ1_M": "IQ1_S"}
# Types whose signs go through the 128-entry even-parity ksigns table.
USES_KSIGNS = ("IQ2_XXS", "IQ2_XS", "IQ3_XXS")

# Non-linear 4-bit value table of IQ4_XS (k_decode.py:77, qmv.py:260).
KVALUES_IQ4NL = (-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113)

IQ1_DELTA = 0.125


def block_bytes(qtype: str) -> int:
    return BLOCK_BYTES[qtype]


def packed_size(qtype: str, out_features: int, in_features: int) -> int:
    """Bytes of an ``out_features x in_features`` weight packed row-major in superblocks."""
    return out_features * (in_features // BLOCK_ELEMENTS) * BLOCK_BYTES[qtype]


def bits_per_weight(qtype: str) -> float:
    return BLOCK_BYTES[qtype] * 8.0 / BLOCK_ELEMENTS
