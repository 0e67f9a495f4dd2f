"""The drop-in ``TurboQuantKVCache`` / ``AutoConfig.build_cache`` on the GPU,
rebuilt token by token exactly as the reference built its own caches in
``tests/golden/make_golden.py``: flush cadence and lengths equal, every coded
group bit-exact in the reference container layout, ``get_keys``/``get_values``
bit-exact (sha256 of the reference's arrays), and ``fused_decode`` within
max-abs 2e-3 / relative 1e-2 of the reference's dequantize-then-attend output.
"""

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


def _fill(cache, g, bulk_from=None):
    k, v = g["k"], g["v"]
    L = k.shape[1]
    t = 0
    while t < L:
        if bulk_from is not None and t >= bulk_from:
            cache.extend(k[:, t:], v[:, t:])      # the rest in one call
            break
        cache.append(k[:, t, :], v[:, t, :])
        t += 1


def _check(cache, g, full):
    assert cache.length == int(g["length"])
    assert cache.cold_length == int(g["cold_length"])
    assert cache.hot_length == int(g["hot_length"])
    assert cache.pool.n_groups(0) == int(g["n_groups"])
    for i in range(int(g["n_groups"])):
        e = cache.pool.export_group(0, i)
        assert np.array_equal(e["kpacked"], g[f"g{i}_kpacked"]), f"group {i} kpacked"
        assert np.array_equal(e["nf4_scale"], g[f"g{i}_nf4_scale"])
        assert np.array_equal(e["nf4_mean"], g[f"g{i}_nf4_mean"])
        assert np.array_equal(e["outlier_idx"], g[f"g{i}_oidx"])
        assert np.array_equal(e["outlier_val"].view(np.uint16), g[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(e["vpacked"], g[f"g{i}_vpacked"])
        assert np.array_equal(e["vnorms"], g[f"g{i}_vnorms"])
    keys = cache.get_keys(0, cache.length)[0]
    vals = cache.get_values(0, cache.length)[0]
    assert keys.dtype == np.float32 and keys.shape == g["k"].shape
    assert _sha(keys) == str(g["get_keys_sha"])
    assert _sha(vals) == str(g["get_values_sha"])
    if full:
        # a window straddling the cold/hot boundary
        a, b = max(0, cache.cold_length - 5), cache.length
        assert np.array_equal(cache.get_keys(a, b)[0], g["get_keys"][:, a:b])
        assert np.array_equal(cache.get_values(a, b)[0], g["get_values"][:, a:b])
    out = cache.fused_decode(g["q"])
    assert out.shape == g["q"].shape and out.dtype == np.float32
    assert_attn_close(out, g["attn_out"])


def test_autoconfig_balanced_cache_matches_reference(golden_dir):
    """AutoConfig 'balanced' K4/V3, W=512, seed 0, 770 single-token appends."""
    from turboquant_pro_amd import AutoConfig
    print("[cache api] balanced W512", flush=True)
    g = np.load(os.path.join(golden_dir, "cache_k4v3_w512.npz"))
    cfg = AutoConfig.from_dict({"head_dim": 128, "num_key_value_heads": 2,
                                "num_attention_heads": 8, "num_hidden_layers": 1},
                               target="balanced")
    cache = cfg.build_cache(hot_window=512, seed=0)
    assert (cache.key_bits, cache.value_bits, cache.hot_window) == (4, 3, 512)
    _fill(cache, g)
    _check(cache, g, full=False)


def test_robust_v4_small_window_matches_reference(golden_dir):
    """TurboQuantKVCache.robust K4/V4, W=16 (groups of 8), seed 1, DC-offset keys."""
    from turboquant_pro_amd import TurboQuantKVCache
    print("[cache api] robust W16", flush=True)
    g = np.load(os.path.join(golden_dir, "cache_k4v4_w16.npz"))
    cache = TurboQuantKVCache.robust(head_dim=128, n_heads=2, hot_window=16, seed=1)
    _fill(cache, g, bulk_from=20)
    _check(cache, g, full=True)


def test_ties_cache_matches_reference_and_grows(golden_dir):
    """K4/V3 W=64 with outlier magnitude ties, seed 2; a small initial capacity
    forces the pool to grow (re-allocate and copy) mid-sequence."""
    from turboquant_pro_amd import TurboQuantKVCache
    print("[cache api] ties W64 + grow", flush=True)
    g = np.load(os.path.join(golden_dir, "cache_k4v3_w64_ties.npz"))
    cache = TurboQuantKVCache(head_dim=128, n_heads=2, bits=3, key_bits=4, value_bits=3,
                              hot_window=64, seed=2, key_nf4_asym=True, key_outlier_frac=0.02,
                              capacity=70)
    _fill(cache, g)
    _check(cache, g, full=True)


def test_stats_clear_and_errors():
    from turboquant_pro_amd import TurboQuantKVCache
    cache = TurboQuantKVCache.robust(head_dim=128, n_heads=2, hot_window=64, seed=0)
    with pytest.raises(RuntimeError, match="empty"):
        cache.fused_decode(np.zeros((2, 128), np.float16))
    rng = np.random.default_rng(0)
    k = rng.standard_normal((2, 200, 128)).astype(np.float16)
    cache.extend(k, k)
    st = cache.memory_stats()
    assert set(st) == {"cold_bytes", "hot_bytes", "total_bytes",
                       "uncompressed_equivalent_bytes", "effective_ratio"}
    assert st["effective_ratio"] > 1.0 and st["total_bytes"] == st["cold_bytes"] + st["hot_bytes"]
    cache.clear()
    assert cache.length == 0
    with pytest.raises(ValueError):
        cache.append(np.zeros((3, 128), np.float16), np.zeros((3, 128), np.float16))
    with pytest.raises(NotImplementedError):
        # PolarQuant keys share the value codebook: unequal widths have no GPU form
        TurboQuantKVCache(head_dim=128, n_heads=2, key_bits=4, value_bits=3, per_channel_keys=False)


def test_uniform_key_cache():
    """``TurboQuantKVCache(per_channel_keys=True)`` without NF4 flags keeps the
    reference's uniform 4-bit keys (turboquant_pro/core.py:1011-1038 with
    PerChannelKV's uniform branch, per_channel_kv.py:303-317): every flushed
    group bit-exact to the oracle (itself pinned to the reference's uniform
    vectors), ``get_keys`` bit-exact, ``fused_decode`` within the bar."""
    from oracle import tq_oracle as O
    from turboquant_pro_amd import TurboQuantKVCache
    print("[cache] uniform keys", flush=True)
    H, L = 2, 1100
    k, v, q = O.synthetic_kv(91, 1, H, H, L)
    k, v, q = k[0], v[0], q[0]
    cache = TurboQuantKVCache(head_dim=128, n_heads=H, key_bits=4, value_bits=3, hot_window=512,
                              per_channel_keys=True, key_outlier_frac=0.02, seed=0)
    assert cache.key_grid == "uniform"
    cache.extend(k[:, :600], v[:, :600])
    for t in range(600, L):
        cache.append(k[:, t], v[:, t])
    pi, pi_t = O.rotation(0, 128)
    sc = O.SequenceCache(hot_window=512, value_bits=3, outlier_frac=0.02, key_grid="uniform").build(k, v, pi, pi_t)
    assert cache.length == L and cache.cold_length == len(sc.keys) * 256
    assert np.array_equal(cache.get_keys(0, L)[0], sc.get_keys())
    assert np.array_equal(cache.get_values(0, L)[0], sc.get_values())
    assert_attn_close(cache.fused_decode(q), sc.attend(q))
