"""3- and 2-bit uniform per-channel keys (the reference's default key form) on
the GPU, against the reference's own outputs
(tests/golden/make_lowbit_golden.py) and the oracle:

* the drop-in cache fed token by token as the reference was -- its default
  ``TurboQuantKVCache(bits=3)``, bits=2 with outliers, K3/V4 at hot window
  512: every coded group bit-exact in the reference container layout,
  ``get_keys`` / ``get_values`` bit-exact, ``fused_decode`` within the bar;
* the ``per_channel`` plugin at 3 and 2 bits on 256- and 1000-token blocks:
  containers and decompressions bit for bit;
* batched GQA pools with K3 and K2 keys on both decode kernels against the
  oracle, and an export -> import round trip of the stored rows;
* the default ``TurboQuantKVManager`` (bits=3).
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
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_lowbit_golden as LG  # noqa: E402  (case tables only)
import make_variant_golden as MG  # noqa: E402  (input generators only)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("case", LG.CACHES, ids=[c[0] for c in LG.CACHES])
def test_uniform_lowbit_cache_matches_reference(case):
    from turboquant_pro_amd import TurboQuantKVCache
    name, seed, H, L, _, kw = case
    print(f"[lowbit] cache {name}", flush=True)
    z = dict(np.load(os.path.join(HERE, "golden", name)))
    k, v = MG.cache_inputs(seed, H, L)
    cache = TurboQuantKVCache(head_dim=128, n_heads=H, **kw)
    assert cache.key_grid == "uniform"
    for t in range(L):
        cache.append(k[:, t, :], v[:, t, :])
    assert cache.length == int(z["length"]) and cache.pool.n_groups(0) == int(z["n_groups"])
    for i in range(int(z["n_groups"])):
        e = cache.pool.export_group(0, i)
        assert np.array_equal(e["kpacked"], z[f"g{i}_kpacked"]), f"group {i} kpacked"
        assert np.array_equal(e["nf4_scale"], z[f"g{i}_scale"]) and np.array_equal(e["nf4_mean"], z[f"g{i}_zero"])
        if f"g{i}_oidx" in z:
            assert np.array_equal(e["outlier_idx"], z[f"g{i}_oidx"])
            assert np.array_equal(e["outlier_val"].view(np.uint16), z[f"g{i}_oval"].view(np.uint16))
        else:
            assert e["outlier_idx"].size == 0
        assert np.array_equal(e["vpacked"], z[f"g{i}_vpacked"]), f"group {i} vpacked"
        assert np.array_equal(e["vnorms"], z[f"g{i}_vnorms"])
    assert _sha(cache.get_keys(0, cache.length)[0]) == str(z["get_keys_sha"])
    assert _sha(cache.get_values(0, cache.length)[0]) == str(z["get_values_sha"])
    assert_attn_close(cache.fused_decode(z["q"]), z["attn_out"], what=name)


@pytest.mark.parametrize("case", LG.BLOCKS, ids=[c[0] for c in LG.BLOCKS])
def test_per_channel_lowbit_blocks_match_reference(case):
    from turboquant_pro_amd import plugins as PL
    tag, seed, S, fp16, bits = case
    print(f"[lowbit] per_channel block {tag}", flush=True)
    z = dict(np.load(os.path.join(HERE, "golden", "perchannel_lowbit.npz")))
    x = MG.long_block_input(seed, 2, S, fp16)
    q = PL.create("per_channel", n_heads=2, bits=bits, outlier_frac=0.02)
    c = q.compress(x.astype(np.float16) if fp16 else x, packed=True)
    assert np.array_equal(c.indices, z[f"{tag}_kpacked"])
    assert np.array_equal(c.scale, z[f"{tag}_scale"]) and np.array_equal(c.zero, z[f"{tag}_zero"])
    assert np.array_equal(c.outlier_idx, z[f"{tag}_oidx"])
    assert np.array_equal(c.outlier_val.view(np.uint16), z[f"{tag}_oval"].view(np.uint16))
    dec = q.decompress(c)
    assert _sha(dec.astype(np.float32)) == str(z[f"{tag}_dec_sha"])
    cu = q.compress(x, packed=False)
    assert cu.indices.shape == (1, 2, S, 128) and int(cu.indices.max()) < (1 << bits)
    assert np.array_equal(q.decompress(cu), dec)


@pytest.mark.parametrize("kb,vb,W", [(3, 3, 512), (2, 2, 512), (3, 4, 16), (2, 3, 16)],
                         ids=["k3v3-mfma", "k2v2-mfma", "k3v4-valu", "k2v3-valu"])
def test_lowbit_pool_decode_gqa(kb, vb, W):
    """Batched GQA pools with 2 % key outliers: every group bit-exact to the
    oracle's encode, decode within the bar on the MFMA kernel (W=512) and the
    VALU kernel (W=16), and the exported groups imported into a fresh pool
    decode identically."""
    from turboquant_pro_amd import TQKVPool
    print(f"[lowbit] pool K{kb}/V{vb} W={W}", flush=True)
    B, Hkv, Hq, L = 2, 2, 8, (1400 if W == 512 else 90)
    k, v, q = O.synthetic_kv(41 + kb, B, Hkv, Hq, L)
    mk = lambda: TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, hot_window=W,  # noqa: E731
                          key_bits=kb, value_bits=vb, seed=0, key_grid="uniform")
    pool = mk()
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    pool.append(kd, vd)
    pi, pi_t = O.rotation(0, 128)
    seqs = [O.SequenceCache(hot_window=W, value_bits=vb, outlier_frac=0.02, key_grid="uniform",
                            key_bits=kb).build(k[b], v[b], pi, pi_t) for b in range(B)]
    for b in range(B):
        assert pool.n_groups(b) == len(seqs[b].keys)
        for g in range(pool.n_groups(b)):
            e = pool.export_group(b, g)
            kg = seqs[b].keys[g]
            assert np.array_equal(e["kpacked"], kg.packed), f"seq {b} group {g} keys"
            assert np.array_equal(e["nf4_scale"], kg.nf4_scale) and np.array_equal(e["nf4_mean"], kg.nf4_mean)
            assert np.array_equal(e["outlier_idx"], kg.outlier_idx)
            assert np.array_equal(e["vpacked"], seqs[b].values[g].packed)
    got = pool.decode(qd)
    for b in range(B):
        assert_attn_close(got[b].cpu().numpy(), seqs[b].attend(q[b]), what=f"K{kb}V{vb} W={W} seq {b}")
    # export -> import: the stored rows come back as they were
    other = mk()
    for b in range(B):
        exported = [pool.export_group(b, g) for g in range(pool.n_groups(b))]
        other.load_sequence(b, [(e, e) for e in exported], *pool.hot_window_tokens(b))
    assert torch.equal(other.kcodes, pool.kcodes)
    # both decode kernels sum in a fixed order: equal bit for bit
    assert torch.equal(other.decode(qd), got)


def test_default_kv_manager_runs_on_the_gpu():
    """``TurboQuantKVManager()`` with the reference's defaults (bits=3: 3-bit
    uniform keys, 3-bit values) builds GPU caches; a layer's groups are
    bit-exact to the oracle and its decode within the bar."""
    from turboquant_pro_amd import TurboQuantKVManager
    print("[lowbit] default manager", flush=True)
    H, L = 2, 200
    mgr = TurboQuantKVManager(n_layers=2, n_kv_heads=H, hot_window=64, seed=1)
    k, v, q = O.synthetic_kv(5, 1, H, H, L)
    for t in range(L):
        mgr.store(1, k[0, :, t], v[0, :, t])
    cache = mgr.cache(1)
    assert (cache.key_bits, cache.value_bits, cache.key_grid) == (3, 3, "uniform")
    sc = O.SequenceCache(hot_window=64, value_bits=3, outlier_frac=0.0, key_grid="uniform",
                         key_bits=3).build(k[0], v[0], *O.rotation(1, 128))
    for g in range(cache.pool.n_groups(0)):
        assert np.array_equal(cache.pool.export_group(0, g)["kpacked"], sc.keys[g].packed)
    kk, vv = mgr.load(1)
    assert np.array_equal(np.asarray(kk)[0], sc.get_keys())
    assert_attn_close(mgr.fused_decode(1, q[0]), sc.attend(q[0]))
    assert mgr.memory_stats()["bits"] == 3
