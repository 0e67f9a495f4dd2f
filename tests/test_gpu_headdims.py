"""head_dim 64 and 256 on the GPU (the reference's caches take any head_dim;
its registry's gemma-2-9b and gemma-4-27b-a4b are head_dim 256,
turboquant_pro/autoconfig.py:76-91).  These pools run the VALU decode and
per-token value rows.

* ``AutoConfig.from_pretrained("gemma-2-9b").build_cache(hot_window=64)``
  rebuilt token by token as the reference built tests/golden/
  cache_gemma2_9b_w64.npz: every group bit for bit, reconstruction sha-equal,
  fused decode within the bar; the same for a head_dim-64 K4/V4 cache;
* the block quantizers against the reference's head_dim-256 PerChannelKV and
  head_dim-64 PolarQuant blocks, bit for bit, and their reconstructions;
* pool decodes (GQA 1, 2, 4 and 8, ragged batches, small and default hot
  windows, heavy outliers) against the oracle's dequantize-then-attend, the
  partial state, and the no-allocation decode against the workspace one.
"""

import ctypes
import hashlib
import os

import numpy as np
import pytest

from gpu_util import assert_attn_close, compare_group, oracle_state
from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _check_cache(cache, g, full):
    assert cache.length == int(g["length"]) and cache.cold_length == int(g["cold_length"])
    assert cache.hot_length == int(g["hot_length"])
    assert cache.pool.n_groups(0) == int(g["n_groups"])
    assert not cache.pool.tiled
    for i in range(int(g["n_groups"])):
        e = cache.pool.export_group(0, i)
        assert np.array_equal(e["kpacked"], g[f"g{i}_kpacked"]), f"group {i} kpacked"
        assert np.array_equal(e["nf4_scale"], g[f"g{i}_nf4_scale"])
        assert np.array_equal(e["nf4_mean"], g[f"g{i}_nf4_mean"])
        assert np.array_equal(e["outlier_idx"], g[f"g{i}_oidx"])
        assert np.array_equal(e["outlier_val"].view(np.uint16), g[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(e["vpacked"], g[f"g{i}_vpacked"]), f"group {i} vpacked"
        assert np.array_equal(e["vnorms"], g[f"g{i}_vnorms"])
    keys = cache.get_keys(0, cache.length)[0]
    vals = cache.get_values(0, cache.length)[0]
    assert _sha(keys) == str(g["get_keys_sha"]) and _sha(vals) == str(g["get_values_sha"])
    if full:
        assert np.array_equal(keys, g["get_keys"]) and np.array_equal(vals, g["get_values"])
    out = cache.fused_decode(g["q"])
    assert out.shape == g["q"].shape and out.dtype == np.float32
    assert_attn_close(out, g["attn_out"])


def test_gemma2_9b_build_cache_matches_reference(golden_dir):
    from turboquant_pro_amd import AutoConfig
    print("[headdims] gemma-2-9b build_cache W64", flush=True)
    g = np.load(os.path.join(golden_dir, "cache_gemma2_9b_w64.npz"))
    cfg = AutoConfig.from_pretrained("gemma-2-9b")
    cache = cfg.build_cache(hot_window=64, seed=6)
    assert (cache.head_dim, cache.n_heads, cache.key_bits, cache.value_bits) == (256, 8, 4, 3)
    k, v = g["k"], g["v"]
    for t in range(k.shape[1]):
        cache.append(k[:, t, :], v[:, t, :])
    _check_cache(cache, g, full=False)


def test_head_dim_64_cache_matches_reference(golden_dir):
    from turboquant_pro_amd import TurboQuantKVCache
    print("[headdims] D64 K4/V4 W32", flush=True)
    g = np.load(os.path.join(golden_dir, "cache_d64_k4v4_w32.npz"))
    cache = TurboQuantKVCache(head_dim=64, n_heads=2, bits=4, key_bits=4, value_bits=4,
                              hot_window=32, seed=7, key_nf4_asym=True, key_outlier_frac=0.02)
    k, v = g["k"], g["v"]
    for t in range(40):
        cache.append(k[:, t, :], v[:, t, :])
    cache.extend(k[:, 40:], v[:, 40:])
    _check_cache(cache, g, full=True)


def test_block_quantizers_match_reference(golden_dir):
    from turboquant_pro_amd import plugins as PL
    print("[headdims] plugins D256 keys, D64 values", flush=True)
    z = np.load(os.path.join(golden_dir, "perchannel_d256.npz"))
    q = PL.create("per_channel", head_dim=256, n_heads=2, bits=4, nf4_asym=True, outlier_frac=0.02)
    c = q.compress(z["x"][None], packed=True)
    assert np.array_equal(c.indices, z["kpacked"])
    assert np.array_equal(c.nf4_scale[0], z["nf4_scale"]) and np.array_equal(c.nf4_mean[0], z["nf4_mean"])
    assert np.array_equal(c.outlier_idx, z["oidx"])
    assert np.array_equal(c.outlier_val.view(np.uint16), z["oval"].view(np.uint16))
    assert np.array_equal(q.decompress(c)[0], z["decompressed"])
    z = np.load(os.path.join(golden_dir, "polar_d64.npz"))
    q = PL.create("polar", head_dim=64, n_heads=2, bits=3, seed=8)
    c = q.compress(z["x"][None], packed=True, kind="value")
    assert np.array_equal(c.indices, z["packed"]) and np.array_equal(c.norms[0], z["norms"])
    assert np.array_equal(q.decompress(c)[0], z["decompressed"])


DECODE_CASES = [
    # (B, Hkv, Hq, L, vbits, hot_window, page_tokens, D)
    (2, 8, 16, 700, 3, 64, None, 256),    # gemma-2-9b heads, GQA 2
    (1, 1, 8, 1100, 3, 512, None, 256),   # gemma-4-27b-a4b heads, GQA 8
    (2, 2, 8, 1300, 4, 512, 16, 256),     # GQA 4, V4, 16-token pages
    (1, 4, 4, 600, 2, 64, None, 256),     # MHA, V2
    (2, 2, 8, 1300, 3, 512, None, 64),    # GQA 4
    (1, 4, 4, 900, 4, 64, 32, 64),        # MHA, V4, 32-token pages
    (1, 2, 16, 200, 3, 16, None, 64),     # GQA 8, groups of 8
    (2, 2, 4, 300, 3, 512, None, 64),     # hot window only
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=[str(c) for c in DECODE_CASES])
def test_decode_matches_dequant_then_attend(case):
    from turboquant_pro_amd import TQKVPool
    B, Hkv, Hq, L, vbits, W, P, D = case
    print(f"[headdims decode] {case}", flush=True)
    k, v, q = O.synthetic_kv(91 + L + D, B, Hkv, Hq, L, D=D)
    seqs, rot = oracle_state(k, v, W, vbits, seed=11)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, head_dim=D, max_batch=B, max_seq_len=L,
                    hot_window=W, value_bits=vbits, rotation=rot, page_tokens=P)
    pool.append(_dev(k), _dev(v))
    for b in range(B):
        for g in range(pool.n_groups(b)):
            compare_group(pool.export_group(b, g), seqs[b].keys[g], seqs[b].values[g],
                          what=f"D{D} seq {b} group {g}")
    got = pool.decode(_dev(q)).cpu().numpy()
    for b in range(B):
        assert_attn_close(got[b], seqs[b].attend(q[b]), what=f"case {case} seq {b}")


@pytest.mark.parametrize("D", [64, 256])
def test_decode_ragged_heavy_outliers_and_partials(D):
    """A ragged batch (hot-only, one-token and multi-group sequences) with
    10 % outliers; the partial state (m, l, acc) normalises to the output;
    the no-allocation decode equals the workspace decode; two decodes of one
    state are equal bit for bit (every sum has a fixed order)."""
    from turboquant_pro_amd import TQKVPool
    from turboquant_pro_amd import _native as N
    lens = [1000, 1, 257, 65, 513]
    B, Hkv, Hq, T = len(lens), 2, 8, max(lens)
    print(f"[headdims ragged] D={D} lens={lens}", flush=True)
    k, v, q = O.synthetic_kv(97 + D, B, Hkv, Hq, T, D=D)
    pi, pi_t = O.rotation(12, D)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, head_dim=D, max_batch=B, max_seq_len=T,
                    hot_window=128, rotation=(pi, pi_t), outlier_frac=0.1)
    pool.append(_dev(k), _dev(v), n_new=lens)
    qd = _dev(q)
    got = pool.decode(qd).cpu().numpy()
    again = pool.decode(qd).cpu().numpy()
    assert np.array_equal(got, again)
    for b, L in enumerate(lens):
        sc = O.SequenceCache(hot_window=128, value_bits=3, outlier_frac=0.1).build(
            k[b, :, :L], v[b, :, :L], pi, pi_t)
        assert_attn_close(got[b], sc.attend(q[b]), what=f"D{D} seq {b} L={L}")
    m, l_, acc = pool.decode_partials(qd)
    assert_attn_close((acc / l_[..., None]).cpu().numpy(), got, what="partials")
    out = torch.full((B, Hq, D), float("nan"), dtype=torch.float32, device=pool.device)
    N.check(N.lib().tqk_decode_noalloc(ctypes.byref(pool.desc), ctypes.byref(pool.ptrs), B,
                                       qd.contiguous().data_ptr(), pool.seq_lens.data_ptr(),
                                       max(pool.lengths), out.data_ptr(), pool._stream()),
            "tqk_decode_noalloc")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), got)


@pytest.mark.parametrize("D,kb,vb", [(256, 3, 3), (64, 2, 2), (256, 4, 4)])
def test_uniform_and_polar_keys(D, kb, vb):
    """Uniform 3-/2-bit keys (the reference's default cache mode) and
    PolarQuant keys at head_dim 64/256: groups bit for bit, decode within the
    bar, export -> import into a fresh pool decodes identically."""
    from turboquant_pro_amd import TQKVPool
    B, Hkv, Hq, L, W = 2, 2, 4, 400, 64
    for grid in ("uniform", "polar"):
        print(f"[headdims keys] D={D} K{kb}/V{vb} {grid}", flush=True)
        k, v, q = O.synthetic_kv(131 + D + kb, B, Hkv, Hq, L, D=D)
        ofrac = 0.02 if grid == "uniform" else 0.0
        mk = lambda: TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, head_dim=D, max_batch=B,  # noqa: E731
                              max_seq_len=L, hot_window=W, key_bits=kb, value_bits=vb, seed=0,
                              key_grid=grid, outlier_frac=ofrac)
        pool = mk()
        pool.append(_dev(k), _dev(v))
        pi, pi_t = O.rotation(0, D)
        seqs = [O.SequenceCache(hot_window=W, value_bits=vb, outlier_frac=ofrac, key_grid=grid,
                                key_bits=kb).build(k[b], v[b], pi, pi_t) for b in range(B)]
        for b in range(B):
            assert pool.n_groups(b) == len(seqs[b].keys)
            for g in range(pool.n_groups(b)):
                e, kg = pool.export_group(b, g), seqs[b].keys[g]
                assert np.array_equal(e["kpacked"], kg.packed), f"{grid} seq {b} group {g} keys"
                assert np.array_equal(e["vpacked"], seqs[b].values[g].packed)
        got = pool.decode(_dev(q)).cpu().numpy()
        for b in range(B):
            assert_attn_close(got[b], seqs[b].attend(q[b]), what=f"D{D} {grid} seq {b}")
        other = mk()
        for b in range(B):
            exported = [pool.export_group(b, g) for g in range(pool.n_groups(b))]
            other.load_sequence(b, [(e, e) for e in exported], *pool.hot_window_tokens(b))
        assert np.array_equal(other.decode(_dev(q)).cpu().numpy(), got)
