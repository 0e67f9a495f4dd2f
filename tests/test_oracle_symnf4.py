"""Symmetric NF4 keys (``PerChannelKV(nf4=True)`` without ``nf4_asym``,
turboquant_pro/per_channel_kv.py:354-357) in the oracle, against the
reference's own outputs (tests/golden/make_sym_golden.py): a K4/V3 cache
with 2 % outliers built token by token, and a 520-token fp32 block.  The
oracle restates the branch as the asym-NF4 encode with a zero mean; the
fixtures pin that reading bit for bit, and a closed form shows the branch is
not the asym one (on channels with an offset their codes differ)."""

import hashlib
import os

import numpy as np

from oracle import tq_oracle as O


def _sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_symmetric_nf4_cache_matches_reference(golden_dir):
    z = dict(np.load(os.path.join(golden_dir, "cache_symnf4_w64.npz")))
    pi, pi_t = O.rotation(3, 128)
    sc = O.SequenceCache(hot_window=64, value_bits=3, outlier_frac=0.02,
                         zero_point="symmetric").build(z["k"], z["v"], pi, pi_t)
    assert len(sc.keys) == int(z["n_groups"]) == 8
    for i, (kg, vg) in enumerate(zip(sc.keys, sc.values)):
        assert np.array_equal(kg.packed, z[f"g{i}_kpacked"]), f"group {i} key codes"
        assert np.array_equal(kg.nf4_scale, z[f"g{i}_nf4_scale"]), f"group {i} scale"
        assert not np.any(kg.nf4_mean), "symmetric NF4 has no mean"
        assert np.array_equal(kg.outlier_idx, z[f"g{i}_oidx"])
        assert np.array_equal(kg.outlier_val.view(np.uint16), z[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(vg.packed, z[f"g{i}_vpacked"])
        assert np.array_equal(vg.norms, z[f"g{i}_vnorms"])
    keys, vals = sc.get_keys(), sc.get_values()
    assert _sha(keys) == str(z["get_keys_sha"]) and _sha(vals) == str(z["get_values_sha"])
    assert np.allclose(O.attend(z["q"], keys, vals), z["attn_out"], atol=1e-6, rtol=1e-5)


def test_symmetric_nf4_block_matches_reference(golden_dir):
    z = dict(np.load(os.path.join(golden_dir, "perchannel_symnf4.npz")))
    x = z["x"]
    H = x.shape[0]
    kg = O.encode_keys(x, 0.02, zero_point="symmetric")
    assert np.array_equal(kg.packed, z["kpacked"])
    assert np.array_equal(kg.nf4_scale, z["nf4_scale"])
    assert np.array_equal(kg.outlier_idx, z["oidx"])
    assert np.array_equal(kg.outlier_val.view(np.uint16), z["oval"].view(np.uint16))
    assert np.array_equal(O.decode_keys(kg), z["decompressed"])
    # the scale is the raw channel's abs-max (closed form), and with the
    # channel offsets of these inputs the symmetric codes are not the asym
    # ones: a restatement that kept the mean would fail here
    assert np.array_equal(kg.nf4_scale, np.maximum(np.abs(x).max(axis=1), 1e-8))
    asym = O.encode_keys(x, 0.02)
    assert not np.array_equal(asym.packed, kg.packed)
    assert H == 2
