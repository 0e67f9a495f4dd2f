"""The oracle against the reference's outputs for the variants beyond K4/V3
calibrated asym-NF4 (fixtures written by tests/golden/make_variant_golden.py):
2-bit values (the "compression" preset), the "bias" and "sparse" key zero
points through the cache cadence, whole-layer key blocks of 1000 and 2500
tokens (fp32 and fp16-valued input, all key modes), and PolarQuant values from
fp32 input.  Everything here is compared bit for bit."""

import hashlib
import os
import sys

import numpy as np
import pytest

from oracle import tq_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_variant_golden as MG  # noqa: E402  (input generators only; no reference import)


def _sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _load(golden_dir, name):
    return dict(np.load(os.path.join(golden_dir, name)))


def _check_cache(z, sc, dc=None):
    assert sc.keys and len(sc.keys) == int(z["n_groups"])
    for i, (kg, vg) in enumerate(zip(sc.keys, sc.values)):
        assert np.array_equal(kg.packed, z[f"g{i}_kpacked"]), f"group {i} key codes"
        assert np.array_equal(kg.nf4_scale, z[f"g{i}_nf4_scale"]), f"group {i} nf4_scale"
        if f"g{i}_nf4_mean" in z:
            mean = kg.nf4_mean if dc is None else kg.nf4_mean[:, dc]
            assert np.array_equal(mean, z[f"g{i}_nf4_mean"]), f"group {i} nf4_mean"
        assert np.array_equal(kg.outlier_idx, z[f"g{i}_oidx"]), f"group {i} outlier idx"
        assert np.array_equal(kg.outlier_val.view(np.uint16), z[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(vg.packed, z[f"g{i}_vpacked"]), f"group {i} value codes"
        assert np.array_equal(vg.norms, z[f"g{i}_vnorms"]), f"group {i} norms"
    keys, vals = sc.get_keys(), sc.get_values()
    assert _sha(keys) == str(z["get_keys_sha"])
    assert _sha(vals) == str(z["get_values_sha"])
    out = O.attend(z["q"], keys, vals)
    assert np.allclose(out, z["attn_out"], atol=1e-6, rtol=1e-5)


def test_k4v2_compression_preset_cache(golden_dir):
    z = _load(golden_dir, "cache_k4v2_w512.npz")
    pi, pi_t = O.rotation(0, 128)
    sc = O.SequenceCache(hot_window=512, value_bits=2, outlier_frac=0.02).build(z["k"], z["v"], pi, pi_t)
    _check_cache(z, sc)


def test_bias_zero_point_cache(golden_dir):
    """zero_point="bias": the zero point is the RoPE-averaged k_proj bias of
    each group's positions (position_start = the cold length before it); the
    reference stores no nf4_mean."""
    z = _load(golden_dir, "cache_bias_w64.npz")
    pi, pi_t = O.rotation(3, 128)
    sc = O.SequenceCache(hot_window=64, value_bits=3, outlier_frac=0.02, zero_point="bias",
                         rope_theta=float(z["rope_theta"]), k_bias=z["k_bias"]).build(z["k"], z["v"], pi, pi_t)
    assert "g0_nf4_mean" not in z and str(z["g0_zp_mode"]) == "bias"
    assert [int(z[f"g{i}_position_start"]) for i in range(int(z["n_groups"]))] == \
        [32 * i for i in range(int(z["n_groups"]))]
    _check_cache(z, sc)


def test_sparse_zero_point_cache(golden_dir):
    """zero_point="sparse": the channel mean on the DC channels of a 32-token
    window only; the reference stores the DC channels' means."""
    z = _load(golden_dir, "cache_sparse_w64.npz")
    pi, pi_t = O.rotation(3, 128)
    sc = O.SequenceCache(hot_window=64, value_bits=3, outlier_frac=0.02, zero_point="sparse",
                         rope_theta=1e4).build(z["k"], z["v"], pi, pi_t)
    dc = O.dc_channel_mask(1e4, 128, 32)
    assert 0 < dc.sum() < 128 and z["g0_nf4_mean"].shape == (2, int(dc.sum()))
    _check_cache(z, sc, dc=dc)


LONG_CASES = [
    # tag, seed, S, fp16-valued, encode keywords, position_start
    ("nf4_f32_s1000", 50, 1000, False, {}, 0),
    ("nf4_f16_s2500", 51, 2500, True, {}, 0),
    ("uni_f32_s1000", 52, 1000, False, None, 0),
    ("sparse_f32_s1000", 53, 1000, False, dict(zero_point="sparse", rope_theta=1e4), 0),
    ("bias_f32_s1000", 54, 1000, False, dict(zero_point="bias", rope_theta=1e6), 777),
]


@pytest.mark.parametrize("tag,seed,S,fp16,kw,pos", LONG_CASES, ids=[c[0] for c in LONG_CASES])
def test_long_key_blocks(golden_dir, tag, seed, S, fp16, kw, pos):
    """Whole-layer key blocks (the block store's records): one quantization
    group of S tokens, k = round(0.02 S) outliers per channel."""
    z = _load(golden_dir, "perchannel_long.npz")
    x = MG.long_block_input(seed, 2, S, fp16)
    assert _sha(x) == str(z[f"{tag}_x_sha"])
    if kw is None:
        g = O.encode_keys_uniform(x[0], 0.02)
        assert np.array_equal(g.nf4_scale, z[f"{tag}_scale"][0, :, 0, :])
        assert np.array_equal(g.nf4_mean, z[f"{tag}_zero"][0, :, 0, :])
    else:
        kw = dict(kw)
        if kw.get("zero_point") == "bias":
            kw["k_bias"] = z["k_bias"]
        g = O.encode_keys(x[0], 0.02, position_start=pos, **kw)
        assert np.array_equal(g.nf4_scale, z[f"{tag}_nf4_scale"][0])
        if f"{tag}_nf4_mean" in z:
            mean = g.nf4_mean
            if kw.get("zero_point") == "sparse":
                mean = mean[:, O.dc_channel_mask(1e4, 128, S)]
            assert np.array_equal(mean, z[f"{tag}_nf4_mean"][0])
    assert _sha(g.packed) == str(z[f"{tag}_kpacked_sha"])
    assert np.array_equal(g.outlier_idx, z[f"{tag}_oidx"])
    assert np.array_equal(g.outlier_val.view(np.uint16), z[f"{tag}_oval"].view(np.uint16))
    dec = O.decode_keys(g)
    assert _sha(dec[None].astype(np.float32)) == str(z[f"{tag}_dec_sha"])


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_polar_values_from_fp32(golden_dir, bits):
    z = _load(golden_dir, "polar_f32.npz")
    v = MG.value_input(60, 2, 300)
    assert _sha(v) == str(z["v_sha"])
    pi, pi_t = O.rotation(0, 128)
    cent, bnd = O.polar_codebook(bits, 128)
    g = O.encode_values(v[0], pi_t, bnd, bits)
    assert np.array_equal(g.packed, z[f"b{bits}_packed"])
    assert np.array_equal(g.norms, z[f"b{bits}_norms"][0])
    assert _sha(O.decode_values(g, cent, pi)[None].astype(np.float32)) == str(z[f"b{bits}_dec_sha"])


def test_zero_point_closed_forms():
    """Invariants that pin the zero-point restatements independently of the
    fixtures: a zero bias gives a zero zero point; a one-token window at
    position 0 averages nothing (cos 1, sin 0) so the zero point is the bias
    itself; the DC mask is monotone in the window and empty past the longest
    wavelength."""
    kb = np.arange(2 * 128, dtype=np.float32).reshape(2, 128) / 7
    assert not O.rope_averaged_bias(np.zeros((2, 128), np.float32), 1e6, 128, 5, 40).any()
    assert np.array_equal(O.rope_averaged_bias(kb, 1e4, 128, 0, 1), kb)
    m32, m256 = O.dc_channel_mask(1e4, 128, 32), O.dc_channel_mask(1e4, 128, 256)
    assert m256.sum() < m32.sum() and not (m256 & ~m32).any()
    assert not O.dc_channel_mask(1e4, 128, 10 ** 9).any()
    # halves of the mask are the same frequencies (rotate_half pairs j, j + 64)
    assert np.array_equal(m32[:64], m32[64:])
