"""Symmetric NF4 keys on the GPU (``TurboQuantKVCache(key_nf4=True)``,
``create("per_channel", nf4=True)``; turboquant_pro/per_channel_kv.py:
354-357): the asym-NF4 encode and decode with every mean zero.  The cache
rebuilt token by token as the reference built tests/golden/
cache_symnf4_w64.npz gives its groups bit for bit (no stored mean, mode
"calibrated", as the reference's containers), its reconstruction sha-equal,
and a fused decode within the bar; the plugin reproduces the reference's
fp32 block bit for bit and decompresses it back exactly."""

import hashlib
import os

import numpy as np
import pytest

from gpu_util import assert_attn_close

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_symmetric_nf4_cache_matches_reference(golden_dir):
    from turboquant_pro_amd import TurboQuantKVCache
    print("[symnf4] cache W64", flush=True)
    g = np.load(os.path.join(golden_dir, "cache_symnf4_w64.npz"))
    cache = TurboQuantKVCache(head_dim=128, n_heads=2, bits=3, key_bits=4, value_bits=3, hot_window=64,
                              seed=3, key_nf4=True, key_outlier_frac=0.02)
    k, v = g["k"], g["v"]
    for t in range(k.shape[1]):
        cache.append(k[:, t, :], v[:, t, :])
    assert cache.length == int(g["length"]) and cache.cold_length == int(g["cold_length"])
    assert cache.pool.n_groups(0) == int(g["n_groups"]) == 8
    for i in range(int(g["n_groups"])):
        e = cache.pool.export_group(0, i)
        assert e["nf4_mean"] is None and e["zp_mode"] == "calibrated"
        assert np.array_equal(e["kpacked"], g[f"g{i}_kpacked"]), f"group {i} kpacked"
        assert np.array_equal(e["nf4_scale"], g[f"g{i}_nf4_scale"])
        assert np.array_equal(e["outlier_idx"], g[f"g{i}_oidx"])
        assert np.array_equal(e["outlier_val"].view(np.uint16), g[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(e["vpacked"], g[f"g{i}_vpacked"])
        assert np.array_equal(e["vnorms"], g[f"g{i}_vnorms"])
    keys = cache.get_keys(0, cache.length)[0]
    vals = cache.get_values(0, cache.length)[0]
    assert _sha(keys) == str(g["get_keys_sha"]) and _sha(vals) == str(g["get_values_sha"])
    assert_attn_close(cache.fused_decode(g["q"]), g["attn_out"], what="symmetric NF4")


def test_symmetric_nf4_plugin_block_matches_reference(golden_dir):
    from turboquant_pro_amd import plugins
    print("[symnf4] plugin block", flush=True)
    z = np.load(os.path.join(golden_dir, "perchannel_symnf4.npz"))
    q = plugins.create("per_channel", head_dim=128, n_heads=2, bits=4, nf4=True, outlier_frac=0.02)
    c = q.compress(z["x"][None], packed=True)
    assert c.nf4_mean is None and c.zp_mode == "calibrated"
    assert np.array_equal(c.indices, z["kpacked"])
    assert np.array_equal(c.nf4_scale[0], z["nf4_scale"])
    assert np.array_equal(c.outlier_idx, z["oidx"])
    assert np.array_equal(c.outlier_val.view(np.uint16), z["oval"].view(np.uint16))
    assert np.array_equal(q.decompress(c)[0], z["decompressed"])
