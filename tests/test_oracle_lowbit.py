"""3- and 2-bit uniform per-channel keys on the CPU: the oracle against the
reference-written fixtures (tests/golden/make_lowbit_golden.py: the
reference's default ``TurboQuantKVCache(bits=3)``, bits=2 with outliers, K3/V4
at hot window 512, and ``PerChannelKV`` blocks at 3 and 2 bits), bit for bit,
and the stored key-row layout (a permutation of the reference's bit stream)
against its definition."""

import hashlib
import os
import sys

import numpy as np
import pytest

from oracle import tq_oracle as O
from turboquant_pro_amd import formats as F

GOLD = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLD)
import make_lowbit_golden as LG  # noqa: E402  (case tables only; no reference import)
import make_variant_golden as MG  # noqa: E402  (input generators only)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("case", LG.CACHES, ids=[c[0] for c in LG.CACHES])
def test_uniform_lowbit_cache(case):
    name, seed, H, L, _, kw = case
    z = np.load(os.path.join(GOLD, name))
    k, v = MG.cache_inputs(seed, H, L)
    assert _sha(k) == str(z["k_sha"]) and _sha(v) == str(z["v_sha"])
    kb = kw.get("key_bits", kw["bits"])
    vb = kw.get("value_bits", kw["bits"])
    sc = O.SequenceCache(hot_window=kw["hot_window"], value_bits=vb,
                         outlier_frac=kw.get("key_outlier_frac", 0.0), seed=kw["seed"],
                         key_grid="uniform", key_bits=kb)
    sc.build(k, v, *O.rotation(kw["seed"], 128))
    assert len(sc.keys) == int(z["n_groups"])
    for i, (kg, vg) in enumerate(zip(sc.keys, sc.values)):
        assert np.array_equal(kg.packed, z[f"g{i}_kpacked"]), f"group {i} key codes"
        assert np.array_equal(kg.nf4_scale, z[f"g{i}_scale"]) and np.array_equal(kg.nf4_mean, z[f"g{i}_zero"])
        if f"g{i}_oidx" in z:
            assert np.array_equal(kg.outlier_idx, z[f"g{i}_oidx"])
            assert np.array_equal(kg.outlier_val.view(np.uint16), z[f"g{i}_oval"].view(np.uint16))
        else:
            assert kg.outlier_idx is None
        assert np.array_equal(vg.packed, z[f"g{i}_vpacked"]) and np.array_equal(vg.norms, z[f"g{i}_vnorms"])
    assert _sha(sc.get_keys()) == str(z["get_keys_sha"])
    assert _sha(sc.get_values()) == str(z["get_values_sha"])
    assert np.allclose(sc.attend(z["q"]), z["attn_out"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("case", LG.BLOCKS, ids=[c[0] for c in LG.BLOCKS])
def test_uniform_lowbit_block(case):
    tag, seed, S, fp16, bits = case
    z = np.load(os.path.join(GOLD, "perchannel_lowbit.npz"))
    x = MG.long_block_input(seed, 2, S, fp16)
    assert _sha(x) == str(z[f"{tag}_x_sha"])
    kg = O.encode_keys_uniform(x[0], 0.02, bits)
    assert np.array_equal(kg.packed, z[f"{tag}_kpacked"])
    assert np.array_equal(kg.nf4_scale, z[f"{tag}_scale"][0, :, 0, :])
    assert np.array_equal(kg.nf4_mean, z[f"{tag}_zero"][0, :, 0, :])
    assert np.array_equal(kg.outlier_idx, z[f"{tag}_oidx"])
    assert np.array_equal(kg.outlier_val.view(np.uint16), z[f"{tag}_oval"].view(np.uint16))
    assert _sha(O.decode_keys(kg)[None].astype(np.float32)) == str(z[f"{tag}_dec_sha"])


def test_uniform_closed_forms():
    """Codes of a channel spanning [mn, mn + qmax * step] are the step index; a
    constant channel takes code 0 (scale floored at 1e-8 / qmax)."""
    for bits in (2, 3):
        qmax = (1 << bits) - 1
        S = 64
        x = np.zeros((1, S, 128), np.float32)
        x[0, :, 0] = np.arange(S) % (qmax + 1) * 0.5 - 1.0
        x[0, :, 1] = 3.25
        kg = O.encode_keys_uniform(x, 0.0, bits)
        assert np.array_equal(kg.codes[0, :, 0], np.arange(S) % (qmax + 1))
        assert np.all(kg.codes[0, :, 1] == 0)
        assert kg.nf4_scale[0, 0] == np.float32(np.float32(0.5 * qmax) / qmax)
        assert kg.nf4_scale[0, 1] == np.float32(np.float32(1e-8) / qmax)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_key_pack_and_row_layout(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, size=(7, 128)).astype(np.uint8)
    # the product's reference pack equals the oracle's, and round-trips
    pk = F.pack_key_codes(codes, bits)
    assert np.array_equal(pk, O.pack_key_codes(codes, bits))
    assert np.array_equal(F.unpack_key_codes(pk, codes.size, bits).reshape(codes.shape), codes)
    rows = F.key_rows_from_codes(codes, bits)
    assert rows.shape == (7, 128 * bits // 8)
    assert np.array_equal(F.codes_from_key_rows(rows, bits), codes)
    if bits == 4:
        assert np.array_equal(rows.reshape(-1), pk)     # 4-bit rows are the reference's pack
        return
    # field i of chunk c (little-endian, 2 * bits wide) = code(32c + 2i) | code(32c + 2i + 1) << bits
    cb = 128 * bits // 32
    for r in range(7):
        for c in range(4):
            word = int.from_bytes(rows[r, c * cb:(c + 1) * cb].tobytes(), "little")
            for i in range(16):
                f = (word >> (2 * bits * i)) & ((1 << (2 * bits)) - 1)
                assert f == int(codes[r, 32 * c + 2 * i]) | (int(codes[r, 32 * c + 2 * i + 1]) << bits)
