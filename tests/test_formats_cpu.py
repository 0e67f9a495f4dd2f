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


def test_tile_value_rows_matches_the_definition():
    """The vectorised tiling (used to import codes into a tiled pool) equals
    the bit-by-bit definition, and untiling any bytes then tiling is the
    identity (every unit bit holds a code bit)."""
    rng = np.random.default_rng(1)
    for vb in (3, 4):
        codes = rng.integers(0, 2 ** vb, size=(48, 128), dtype=np.uint8)
        want = np.concatenate([_tile(codes[16 * i:16 * (i + 1)], vb) for i in range(3)])
        got = F.tile_value_rows(codes, vb)
        assert got.shape == (48, 128 * vb // 8)
        assert np.array_equal(got.reshape(-1), want)
        raw = rng.integers(0, 256, size=(32, 128 * vb // 8), dtype=np.uint8)
        assert np.array_equal(F.tile_value_rows(F.untile_value_rows(raw, vb), vb), raw)


def test_pack_values_matches_oracle_pack():
    rng = np.random.default_rng(1)
    for vb in (2, 3, 4):
        for n in (1, 8, 13, 256):
            c = rng.integers(0, 2 ** vb, size=n, dtype=np.uint8)
            assert np.array_equal(F.pack_values(c, vb), O.pack_value_codes(c, vb))


def _zero_level(packed, idx, H, S, D):
    """Stored form of reference key codes: NF4 zero level at outlier positions."""
    codes = O.unpack_key_codes(packed, H * S * D, 4).reshape(-1).copy()
    codes[idx] = F.NF4_ZERO_CODE
    return O.pack_key_codes(codes.reshape(1, H, S, D), 4).reshape(H, S, D // 2)


def test_restore_outlier_codes_matches_reference_codes(golden_dir):
    """Export restores the reference's kpacked from the zero-level storage form:
    on the reference's own group fixture and on oracle groups with ties."""
    import os
    g = np.load(os.path.join(golden_dir, "cache_k4v3_w512.npz"))
    H, D = g["k"].shape[0], g["k"].shape[2]
    S = g["g0_kpacked"].size * 2 // (H * D)
    for i in range(int(g["n_groups"])):
        idx = g[f"g{i}_oidx"].astype(np.int64)
        stored = _zero_level(g[f"g{i}_kpacked"], idx, H, S, D)
        back = F.restore_outlier_codes(stored, idx, g[f"g{i}_oval"], g[f"g{i}_nf4_scale"],
                                       g[f"g{i}_nf4_mean"])
        assert np.array_equal(back.reshape(-1), g[f"g{i}_kpacked"])
    rng = np.random.default_rng(3)
    x = (np.round(rng.standard_normal((2, 64, 128)) * 2) / 2).astype(np.float16).astype(np.float32)
    x[1, :, 7] = 0.0
    kg = O.encode_keys(x, 0.05)
    idx = kg.outlier_idx.astype(np.int64)
    stored = _zero_level(kg.packed, idx, 2, 64, 128)
    assert not np.array_equal(stored.reshape(-1), kg.packed)
    back = F.restore_outlier_codes(stored, idx, kg.outlier_val, kg.nf4_scale, kg.nf4_mean)
    assert np.array_equal(back.reshape(-1), kg.packed)


def test_nf4_zero_code_is_exact_zero():
    assert F.NF4[F.NF4_ZERO_CODE] == 0.0
    assert np.array_equal(F.NF4, O.NF4.astype(np.float32))


def test_clustered_block_table_is_a_permutation_with_adjacent_blocks():
    """Default table for 32-token pages: a bijection onto each sequence's page
    range in which block k of the 8 groups of a cluster occupy 8 adjacent pages."""
    from turboquant_pro_amd.pool import TQKVPool
    B, G = 3, 256
    nb = G // 32
    max_pages = 127 * nb
    max_pages = -(-max_pages // (8 * nb)) * (8 * nb)
    bt = TQKVPool._clustered_table(B, max_pages, 32, G)
    for b in range(B):
        row = bt[b]
        assert sorted(row.tolist()) == list(range(b * max_pages, (b + 1) * max_pages))
        for c in range(max_pages // (8 * nb)):
            for k in range(nb):
                pages = [row[(8 * c + w) * nb + k] for w in range(8)]
                assert pages == list(range(pages[0], pages[0] + 8))
    ident = TQKVPool._clustered_table(2, 10, 16, 256)
    assert np.array_equal(ident.reshape(-1), np.arange(20))


def test_uniform_outlier_codes_round_trip(golden_dir):
    """Uniform keys store code 0 at outlier positions (its level is the zero
    term the decode's bias carries); restoring puts back the reference's own
    codes there (tests/golden/perchannel_uniform.npz, written by
    PerChannelKV.compress, turboquant_pro/per_channel_kv.py:303-317)."""
    import os
    z = np.load(os.path.join(golden_dir, "perchannel_uniform.npz"))
    for tag in ("s256", "s200"):
        H, S, D = z[f"{tag}_x"].shape
        kp = z[f"{tag}_kpacked"].reshape(H, S, D // 2)
        idx = z[f"{tag}_oidx"].astype(np.int64)
        stored = F.mark_outlier_codes(kp, idx, grid="uniform")
        codes = F.unpack_keys(stored, H * S * D)
        assert np.all(codes[idx] == 0)
        back = F.restore_outlier_codes(stored, idx, z[f"{tag}_oval"], z[f"{tag}_scale"], z[f"{tag}_zero"],
                                       grid="uniform")
        assert np.array_equal(back, kp)


def test_key_rows_follow_the_chunk_layout_at_every_head_dim():
    """3- and 2-bit key rows: D / 32 chunks of 4 * bits bytes, chunk c's
    little-endian field i = code(32c + 2i) | code(32c + 2i + 1) << bits,
    checked bit by bit from that definition, and the unpack inverts it."""
    rng = np.random.default_rng(4)
    for D in (64, 128, 256):
        for bits in (2, 3, 4):
            codes = rng.integers(0, 2 ** bits, size=(5, D), dtype=np.uint8)
            rows = F.key_rows_from_codes(codes, bits)
            assert rows.shape == (5, D * bits // 8)
            assert np.array_equal(F.codes_from_key_rows(rows, bits, D), codes), (D, bits)
            if bits == 4:
                continue
            for t in range(5):
                for c in range(D // 32):
                    chunk = int.from_bytes(rows[t, 4 * bits * c:4 * bits * (c + 1)].tobytes(), "little")
                    for i in range(16):
                        f = (chunk >> (2 * bits * i)) & ((1 << 2 * bits) - 1)
                        assert f == int(codes[t, 32 * c + 2 * i]) | int(codes[t, 32 * c + 2 * i + 1]) << bits
