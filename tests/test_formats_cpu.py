"""Host-side layout conversions: the MFMA-tiled value order is a lossless
permutation of the reference's value codes (checked against an independent
bit-by-bit tiling written from the layout definition)."""

import numpy as np

from oracle import tq_oracle as O
from turboquant_pro_amd import formats as F


def _tile(codes, vb):
    """codes (16, 128) -> tiled bytes, straight from the layout definition:
    unit (lg, c) holds tokens 4lg..4lg+3 x channels 8c..8c+7, the code of
    token u / channel nt at bit (2nt + u//2)*2vb + (u%2)*vb."""
    unit = 128 * vb // 32
    out = np.zeros((64, unit * 8), np.uint8)
    for lg in range(4):
        for c in range(16):
            for u in range(4):
                for nt in range(8):
                    v = int(codes[4 * lg + u, 8 * c + nt])
                    bit = (2 * nt + u // 2) * 2 * vb + (u % 2) * vb
                    for k in range(vb):
                        out[16 * lg + c, bit + k] = (v >> k) & 1
    return np.packbits(out, axis=1, bitorder="little").reshape(-1)


def test_untile_inverts_tile():
    rng = np.random.default_rng(0)
    for vb in (3, 4):
        codes = rng.integers(0, 2 ** vb, size=(32, 128), dtype=np.uint8)
        tiled = np.concatenate([_tile(codes[:16], vb), _tile(codes[16:], vb)])
        assert tiled.size == 32 * 128 * vb // 8
        assert np.array_equal(F.untile_value_rows(tiled, vb), codes)


def test_pack_values_matches_oracle_pack():
    rng = np.random.default_rng(1)
    for vb in (2, 3, 4):
        for n in (1, 8, 13, 256):
            c = rng.integers(0, 2 ** vb, size=n, dtype=np.uint8)
            assert np.array_equal(F.pack_values(c, vb), O.pack_value_codes(c, vb))
