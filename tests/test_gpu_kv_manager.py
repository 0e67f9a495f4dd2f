"""``TurboQuantKVManager`` / ``TurboQuantKVBackend`` over the GPU caches
(turboquant_pro/vllm_plugin.py:64-343), against the reference semantics:
token-by-token ``store`` per layer, ``load`` of any range as the reference's
``get_keys`` / ``get_values`` give it (bit-exact to the oracle's
reconstruction), ``memory_stats`` in the reference's container bytes, the
backend's initialize / store_block / load_block, and a layer's fused decode
within the parity bar.  The manager's layers are the reference's default
cache with ``bits=4`` (uniform 4-bit per-channel keys, 4-bit values)."""

import numpy as np
import pytest

from gpu_util import assert_attn_close
from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def test_manager_store_load_stats():
    from turboquant_pro_amd import TurboQuantKVManager
    print("[kv manager] 3 layers, bits=4, W=64", flush=True)
    n_layers, H, L, W = 3, 2, 150, 64
    mgr = TurboQuantKVManager(n_layers=n_layers, n_kv_heads=H, head_dim=128, bits=4, hot_window=W, seed=0)
    data = [O.synthetic_kv(40 + i, 1, H, H, L) for i in range(n_layers)]
    for t in range(L):
        for i, (k, v, _) in enumerate(data):
            mgr.store(i, k[0, :, t, :], v[0, :, t, :])
    assert mgr.n_layers == n_layers and all(mgr.length(i) == L for i in range(n_layers))
    pi, pi_t = O.rotation(0, 128)
    for i, (k, v, q) in enumerate(data):
        sc = O.SequenceCache(hot_window=W, value_bits=4, outlier_frac=0.0, key_grid="uniform").build(
            k[0], v[0], pi, pi_t)
        kk, vv = mgr.load(i)
        assert kk.shape == (1, H, L, 128) and kk.dtype == np.float32
        assert np.array_equal(kk[0], sc.get_keys()) and np.array_equal(vv[0], sc.get_values())
        k2, v2 = mgr.load(i, 20, 100)
        assert np.array_equal(k2[0], sc.get_keys()[:, 20:100])
        assert_attn_close(mgr.fused_decode(i, q[0]), sc.attend(q[0]), what=f"layer {i}")
        ls = mgr.layer_stats(i)
        ng = len(sc.keys)
        # reference container bytes: packed keys + scale + zero, values + norms
        cold = ng * (H * 32 * 64 + 2 * H * 128 * 4 + H * 32 * 64 + H * 32 * 4)
        assert (ls.length, ls.cold_length, ls.hot_length) == (L, 32 * ng, L - 32 * ng)
        assert ls.cold_bytes == cold and ls.hot_bytes == (L - 32 * ng) * H * 128 * 2 * 2
        assert ls.uncompressed_bytes == L * H * 128 * 4 * 2
    st = mgr.memory_stats()
    assert st["n_layers"] == n_layers and st["total_tokens"] == L and st["bits"] == 4
    assert st["total_bytes"] == st["cold_bytes"] + st["hot_bytes"]
    assert mgr.estimate_capacity(1.0) > W
    mgr.clear()
    assert mgr.length(0) == 0


def test_backend_blocks():
    from turboquant_pro_amd import TurboQuantKVBackend
    print("[kv manager] backend", flush=True)
    be = TurboQuantKVBackend(bits=4, hot_window=64, seed=0)
    assert be.memory_stats() == {} and not be.supports_async()
    with pytest.raises(RuntimeError):
        be.store_block(0, np.zeros((2, 128), np.float16), np.zeros((2, 128), np.float16))
    be.initialize(n_layers=2, n_kv_heads=2, head_dim=128)
    k, v, _ = O.synthetic_kv(3, 1, 2, 2, 100)
    be.store_block(1, k[0], v[0])          # (H, n, D): 100 tokens at once
    kk, vv = be.load_block(1)
    assert kk.shape == (1, 2, 100, 128) and be.memory_stats()["total_tokens"] == 100
    assert be.load_block(0)[0].shape == (1, 2, 0, 128)


def test_polar_keys_with_unequal_widths_have_no_gpu_form():
    from turboquant_pro_amd import TurboQuantKVManager
    with pytest.raises(NotImplementedError):
        TurboQuantKVManager(n_layers=1, n_kv_heads=2, key_bits=4, value_bits=3, per_channel_keys=False)
