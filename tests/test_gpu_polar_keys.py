"""PolarQuant keys (``TurboQuantKVCache(per_channel_keys=False)``, the
reference's ``TurboQuantKV.compress(kind="key")``, turboquant_pro/core.py:1028-1029)
in the fused GPU cache.

The reference codes such keys with its value encode at the key width, so a
cache fed the value tokens of a reference-written fixture as its keys must
store, per group, exactly the value groups the reference wrote for them:

* the drop-in cache at 3, 2, 4 and 3 bits (hot windows 64, 64, 16, 512; the
  MFMA kernel at 64 and 512, the VALU kernel at 16), one of them grown past
  its capacity on the way: every key group's codes and norms bit-exact to the
  fixture's value groups, ``get_keys`` bit-exact to the fixture's
  ``get_values``, ``fused_decode`` within the bar of the oracle;
* batched GQA pools on both kernels: every group bit-exact to the oracle,
  decode within the bar, export -> import into a fresh pool identical;
* ``TurboQuantKVManager(per_channel_keys=False)`` and its memory accounting.
"""

import hashlib
import os
import sys

import numpy as np
import pytest

from gpu_util import assert_attn_close
from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import test_oracle_polar_keys as PK  # noqa: E402  (fixture table and oracle builder)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("case", PK.FIXTURES, ids=[c[0] for c in PK.FIXTURES])
def test_polar_key_cache_matches_reference_groups(case):
    from turboquant_pro_amd import TurboQuantKVCache
    name, bits, W, seed, src = case
    print(f"[polar-keys] cache {name}", flush=True)
    z = dict(np.load(os.path.join(PK.GOLD, name)))
    v = src(z)
    H, L, D = v.shape
    # the 3-bit, hot-window-64 case starts small so that it grows twice
    cap = 100 if name.startswith("cache_k3v3") else 4096
    cache = TurboQuantKVCache(head_dim=D, n_heads=H, bits=bits, hot_window=W, seed=seed,
                              per_channel_keys=False, capacity=cap)
    assert cache.key_grid == "polar"
    if W == 64:
        for t in range(L):            # token by token, as the reference was fed
            cache.append(v[:, t, :], v[:, t, :])
    else:
        cache.extend(v, v)
    assert cache.pool.n_groups(0) == int(z["n_groups"])
    for i in range(int(z["n_groups"])):
        e = cache.pool.export_group(0, i)
        assert np.array_equal(e["kpacked"], z[f"g{i}_vpacked"]), f"group {i} key codes"
        assert np.array_equal(e["knorms"], z[f"g{i}_vnorms"]), f"group {i} key norms"
        assert np.array_equal(e["vpacked"], z[f"g{i}_vpacked"]), f"group {i} value codes"
        assert np.array_equal(e["vnorms"], z[f"g{i}_vnorms"])
    assert _sha(cache.get_keys(0, cache.length)[0]) == str(z["get_values_sha"])
    assert _sha(cache.get_values(0, cache.length)[0]) == str(z["get_values_sha"])
    sc = PK.polar_key_cache(v, bits, W, seed)
    q = np.random.default_rng(bits).standard_normal((H, D)).astype(np.float16)
    assert_attn_close(cache.fused_decode(q), sc.attend(q), what=name)
    st = cache.memory_stats()
    ng, G = cache.pool.n_groups(0), cache.pool.group_tokens
    assert st["cold_bytes"] == 2 * ng * (H * G * D * bits // 8 + H * G * 4)


@pytest.mark.parametrize("bits,W", [(3, 512), (2, 512), (4, 512), (4, 16), (3, 16)],
                         ids=["k3v3-mfma", "k2v2-mfma", "k4v4-mfma", "k4v4-valu", "k3v3-valu"])
def test_polar_key_pool_decode_gqa(bits, W):
    """Batched GQA pools (B=2, Hkv=2, Hq=8): every group bit-exact to the
    oracle, decode within the bar on the MFMA kernel (W=512) and the VALU
    kernel (W=16), and the exported groups imported into a fresh pool give
    the same stored rows and the same decode."""
    from turboquant_pro_amd import TQKVPool
    from turboquant_pro_amd.formats import pack_values
    print(f"[polar-keys] pool K{bits}/V{bits} W={W}", flush=True)
    B, Hkv, Hq, L = 2, 2, 8, (1400 if W == 512 else 90)
    k, v, q = O.synthetic_kv(60 + bits, B, Hkv, Hq, L)
    mk = lambda: TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, hot_window=W,  # noqa: E731
                          key_bits=bits, value_bits=bits, seed=0, key_grid="polar")
    pool = mk()
    assert pool.desc.outliers_per_channel == 0
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    pool.append(kd, vd)
    pi, pi_t = O.rotation(0, 128)
    seqs = [O.SequenceCache(hot_window=W, value_bits=bits, key_bits=bits, outlier_frac=0.0,
                            key_grid="polar").build(k[b], v[b], pi, pi_t) for b in range(B)]
    for b in range(B):
        assert pool.n_groups(b) == len(seqs[b].keys)
        for g in range(pool.n_groups(b)):
            e = pool.export_group(b, g)
            kg = seqs[b].keys[g]
            assert np.array_equal(e["kpacked"], pack_values(kg.codes, bits)), f"seq {b} group {g} keys"
            assert np.array_equal(e["knorms"], kg.norms), f"seq {b} group {g} key norms"
            assert np.array_equal(e["vpacked"], seqs[b].values[g].packed)
    got = pool.decode(qd)
    for b in range(B):
        assert_attn_close(got[b].cpu().numpy(), seqs[b].attend(q[b]), what=f"polar K{bits} W={W} seq {b}")
    other = mk()
    for b in range(B):
        exported = [pool.export_group(b, g) for g in range(pool.n_groups(b))]
        other.load_sequence(b, [(e, e) for e in exported], *pool.hot_window_tokens(b))
    assert torch.equal(other.kcodes, pool.kcodes) and torch.equal(other.knorm, pool.knorm)
    assert torch.equal(other.decode(qd), got)


def test_polar_key_manager():
    """``TurboQuantKVManager(per_channel_keys=False)``: every layer's cache
    codes its keys as PolarQuant; a layer's groups are bit-exact to the oracle
    and its decode within the bar.  Unequal key and value widths have no GPU
    form (the reference's fused decode requires them equal too)."""
    from turboquant_pro_amd import TurboQuantKVManager
    print("[polar-keys] manager", flush=True)
    H, L = 2, 200
    mgr = TurboQuantKVManager(n_layers=2, n_kv_heads=H, hot_window=64, seed=1, per_channel_keys=False)
    k, v, q = O.synthetic_kv(8, 1, H, H, L)
    for t in range(L):
        mgr.store(0, k[0, :, t], v[0, :, t])
    cache = mgr.cache(0)
    assert (cache.key_bits, cache.value_bits, cache.key_grid) == (3, 3, "polar")
    sc = O.SequenceCache(hot_window=64, value_bits=3, key_bits=3, outlier_frac=0.0,
                         key_grid="polar").build(k[0], v[0], *O.rotation(1, 128))
    for g in range(cache.pool.n_groups(0)):
        assert np.array_equal(cache.pool.export_group(0, g)["knorms"], sc.keys[g].norms)
    kk, _ = mgr.load(0)
    assert np.array_equal(np.asarray(kk)[0], sc.get_keys())
    assert_attn_close(mgr.fused_decode(0, q[0]), sc.attend(q[0]))
    assert mgr.memory_stats()["compression_ratio"] > 1.0
    with pytest.raises(NotImplementedError):
        TurboQuantKVManager(n_layers=1, n_kv_heads=2, key_bits=4, value_bits=3, per_channel_keys=False)
