"""The oracle on fp32 tokens against the reference's own fp32 caches
(tests/golden/cache_f32.npz, written by tests/golden/make_f32_golden.py with
the settings of the reference's dispatch tests, tests/test_kv_fused_pck.py:
193-308: 4 heads of head_dim 64, hot window 16, fp32 appends with a DC
offset, fp32 query).  Every group bit for bit -- uniform, asym-NF4 + 2 %,
the "bias" zero point over eight positions, symmetric NF4 and PolarQuant
keys -- the reconstruction equal to the reference's get_keys/get_values, and
the dequantize-then-attend output equal to its truth."""

import os

import numpy as np
import pytest

from oracle import tq_oracle as O

THETA = 1e6
VARIANTS = {
    "uniform": dict(key_grid="uniform", key_bits=4, outlier_frac=0.0),
    "nf4": dict(outlier_frac=0.02),
    "bias": dict(outlier_frac=0.02, zero_point="bias", rope_theta=THETA),
    "sym": dict(outlier_frac=0.02, zero_point="symmetric"),
    "polar": dict(key_grid="polar", key_bits=4, outlier_frac=0.0),
}


@pytest.fixture(scope="module")
def z(golden_dir):
    return np.load(os.path.join(golden_dir, "cache_f32.npz"), allow_pickle=False)


def oracle_cache(z, tag):
    kw = dict(VARIANTS[tag])
    if kw.get("zero_point") == "bias":
        kw["k_bias"] = z["k_bias"]
    k, v = z[f"{tag}_k"], z[f"{tag}_v"]
    pi, pi_t = O.rotation(0, k.shape[-1])
    return O.SequenceCache(hot_window=16, value_bits=4, **kw).build(k, v, pi, pi_t)


@pytest.mark.parametrize("tag", list(VARIANTS))
def test_fp32_cache_matches_reference(z, tag):
    sc = oracle_cache(z, tag)
    assert len(sc.keys) == int(z[f"{tag}_n_groups"]) == 8
    assert sc.hot_k.shape[1] == int(z[f"{tag}_hot_length"])
    for g, (kg, vg) in enumerate(zip(sc.keys, sc.values)):
        p = f"{tag}_g{g}_"
        assert np.array_equal(kg.packed, z[p + "kpacked"]), f"{tag} group {g} keys"
        if tag == "polar":
            assert np.array_equal(kg.norms, z[p + "k_norms"][0])
        elif tag == "uniform":
            assert np.array_equal(kg.nf4_scale, z[p + "k_scale"][0, :, 0])
            assert np.array_equal(kg.nf4_mean, z[p + "k_zero"][0, :, 0])
        else:
            assert np.array_equal(kg.nf4_scale, z[p + "k_nf4_scale"][0])
            if p + "k_nf4_mean" in z.files:
                assert np.array_equal(kg.nf4_mean, z[p + "k_nf4_mean"][0])
            assert np.array_equal(kg.outlier_idx, z[p + "k_outlier_idx"])
            assert np.array_equal(kg.outlier_val.view(np.uint16), z[p + "k_outlier_val"].view(np.uint16))
        assert np.array_equal(vg.packed, z[p + "vpacked"]) and np.array_equal(vg.norms, z[p + "vnorms"])
    keys, vals = sc.get_keys(), sc.get_values()
    assert np.array_equal(keys, z[f"{tag}_get_keys"]) and np.array_equal(vals, z[f"{tag}_get_values"])
    assert np.allclose(O.attend(z[f"{tag}_q"], keys, vals), z[f"{tag}_truth"], atol=1e-6, rtol=1e-5)
    # the reference's own fused decode agrees with its truth to its test's 2e-4
    assert np.abs(z[f"{tag}_fused"] - z[f"{tag}_truth"]).max() < 2e-4
