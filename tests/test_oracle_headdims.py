"""The oracle at head_dim 64 and 256 against vectors the reference wrote
(tests/golden/make_hd_golden.py): rotation and codebook, every coded group of
the gemma-2-9b cache (8 kv heads x 256 channels, asym-NF4 + 2 % outliers, V3)
and of a head_dim-64 K4/V4 cache bit for bit, their reconstructions by sha256,
and the block quantizers (PerChannelKV at 256, PolarQuant values at 64)."""

import hashlib
import os

import numpy as np
import pytest

from oracle import tq_oracle as O


def _load(golden_dir, name):
    return np.load(os.path.join(golden_dir, name), allow_pickle=False)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("name,hot_window,vbits,seed,full", [
    ("cache_gemma2_9b_w64.npz", 64, 3, 6, False),
    ("cache_d64_k4v4_w32.npz", 32, 4, 7, True),
])
def test_cache_matches_reference(golden_dir, name, hot_window, vbits, seed, full):
    g = _load(golden_dir, name)
    k, v, q = g["k"], g["v"], g["q"]
    H, L, D = k.shape
    pi, pi_t = O.rotation(seed, D)
    assert np.array_equal(pi, g["pi"]) and np.array_equal(pi_t, g["pi_t"])
    assert np.allclose(pi @ pi_t, np.eye(D), atol=1e-5)
    cent, bnd = O.polar_codebook(vbits, D)
    assert np.array_equal(cent, g["vcent"]) and np.array_equal(bnd, g["vbnd"])
    assert set(g["zp_modes"]) == {"calibrated"}
    sc = O.SequenceCache(hot_window=hot_window, value_bits=vbits, outlier_frac=0.02,
                         seed=seed).build(k, v, pi, pi_t)
    assert len(sc.keys) == int(g["n_groups"]) == O.n_groups(L, hot_window)
    assert sc.hot_k.shape[1] == int(g["hot_length"])
    for i, (kg, vg) in enumerate(zip(sc.keys, sc.values)):
        assert np.array_equal(kg.packed, g[f"g{i}_kpacked"]), f"group {i} key codes"
        assert np.array_equal(kg.nf4_scale, g[f"g{i}_nf4_scale"])
        assert np.array_equal(kg.nf4_mean, g[f"g{i}_nf4_mean"])
        assert np.array_equal(kg.outlier_idx, g[f"g{i}_oidx"])
        assert np.array_equal(kg.outlier_val.view(np.uint16), g[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(vg.packed, g[f"g{i}_vpacked"]), f"group {i} value codes"
        assert np.array_equal(vg.norms, g[f"g{i}_vnorms"])
    keys, vals = sc.get_keys(), sc.get_values()
    assert _sha(keys) == str(g["get_keys_sha"]) and _sha(vals) == str(g["get_values_sha"])
    if full:
        assert np.array_equal(keys, g["get_keys"]) and np.array_equal(vals, g["get_values"])
    assert np.allclose(O.attend(q, keys, vals), g["attn_out"], atol=1e-6, rtol=1e-5)


def test_perchannel_d256(golden_dir):
    g = _load(golden_dir, "perchannel_d256.npz")
    kg = O.encode_keys(g["x"], 0.02)
    assert np.array_equal(kg.packed, g["kpacked"])
    assert np.array_equal(kg.nf4_scale, g["nf4_scale"]) and np.array_equal(kg.nf4_mean, g["nf4_mean"])
    assert np.array_equal(kg.outlier_idx, g["oidx"])
    assert np.array_equal(kg.outlier_val.view(np.uint16), g["oval"].view(np.uint16))
    assert np.array_equal(O.decode_keys(kg), g["decompressed"])


def test_polar_values_d64(golden_dir):
    g = _load(golden_dir, "polar_d64.npz")
    pi, pi_t = O.rotation(8, 64)
    assert np.array_equal(pi, g["pi"]) and np.array_equal(pi_t, g["pi_t"])
    cent, bnd = O.polar_codebook(3, 64)
    vg = O.encode_values(g["x"], pi_t, bnd, 3)
    assert np.array_equal(vg.packed, g["packed"]) and np.array_equal(vg.norms, g["norms"])
    assert np.array_equal(O.decode_values(vg, cent, pi), g["decompressed"])
