"""The key/value variants beyond K4/V3 calibrated asym-NF4, and whole-layer
blocks, on the GPU, against the reference's own outputs
(tests/golden/make_variant_golden.py) and the oracle:

* the "compression" preset (K4/V2) and the "bias" / "sparse" key zero points
  through the drop-in cache, fed token by token as the reference was: every
  coded group bit-exact in the reference container layout, ``get_keys`` /
  ``get_values`` bit-exact, ``fused_decode`` within the parity bar;
* the plugins' block encode on 1000- and 2500-token blocks (fp32 and
  fp16-valued input; asym-NF4 with the three zero points, uniform) and
  PolarQuant from fp32 at 2, 3 and 4 bits: containers and decompressions bit
  for bit;
* 2-bit values in a batched GQA pool on both decode kernels, against the
  oracle;
* a value norm the decode cannot carry is refused at append.
"""

import hashlib
import os
import sys

import numpy as np
import pytest

from gpu_util import assert_attn_close, oracle_state
from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_variant_golden as MG  # noqa: E402  (input generators only)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _load(name):
    return dict(np.load(os.path.join(HERE, "golden", name)))


def _fill_and_check(cache, z, mean_key=lambda e: e["nf4_mean"]):
    k, v = z["k"], z["v"]
    for t in range(k.shape[1]):
        cache.append(k[:, t, :], v[:, t, :])
    assert cache.length == int(z["length"]) and cache.cold_length == int(z["cold_length"])
    assert cache.pool.n_groups(0) == int(z["n_groups"])
    for i in range(int(z["n_groups"])):
        e = cache.pool.export_group(0, i)
        assert np.array_equal(e["kpacked"], z[f"g{i}_kpacked"]), f"group {i} kpacked"
        assert np.array_equal(e["nf4_scale"], z[f"g{i}_nf4_scale"]), f"group {i} nf4_scale"
        if f"g{i}_nf4_mean" in z:
            assert np.array_equal(mean_key(e), z[f"g{i}_nf4_mean"]), f"group {i} nf4_mean"
        else:
            assert e["nf4_mean"] is None
        assert e["position_start"] == int(z[f"g{i}_position_start"])
        assert np.array_equal(e["outlier_idx"], z[f"g{i}_oidx"])
        assert np.array_equal(e["outlier_val"].view(np.uint16), z[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(e["vpacked"], z[f"g{i}_vpacked"]), f"group {i} vpacked"
        assert np.array_equal(e["vnorms"], z[f"g{i}_vnorms"])
    assert _sha(cache.get_keys(0, cache.length)[0]) == str(z["get_keys_sha"])
    assert _sha(cache.get_values(0, cache.length)[0]) == str(z["get_values_sha"])
    assert_attn_close(cache.fused_decode(z["q"]), z["attn_out"])


def test_compression_preset_k4v2_cache():
    from turboquant_pro_amd import AutoConfig
    print("[variants] compression preset K4/V2 W512", flush=True)
    z = _load("cache_k4v2_w512.npz")
    cfg = AutoConfig.from_dict({"head_dim": 128, "num_key_value_heads": 2, "num_attention_heads": 8,
                                "num_hidden_layers": 1}, target="compression")
    cache = cfg.build_cache(hot_window=512, seed=0)
    assert (cache.key_bits, cache.value_bits) == (4, 2)
    _fill_and_check(cache, z)


def test_bias_zero_point_cache():
    from turboquant_pro_amd import TurboQuantKVCache
    print("[variants] bias zero point W64", flush=True)
    z = _load("cache_bias_w64.npz")
    cache = TurboQuantKVCache(head_dim=128, n_heads=2, bits=3, key_bits=4, value_bits=3, hot_window=64,
                              seed=3, key_nf4_asym=True, key_outlier_frac=0.02, key_zero_point="bias",
                              key_rope_theta=float(z["rope_theta"]), key_k_bias=z["k_bias"])
    _fill_and_check(cache, z)


def test_sparse_zero_point_cache():
    from turboquant_pro_amd import TurboQuantKVCache
    print("[variants] sparse zero point W64", flush=True)
    z = _load("cache_sparse_w64.npz")
    cache = TurboQuantKVCache(head_dim=128, n_heads=2, bits=3, key_bits=4, value_bits=3, hot_window=64,
                              seed=3, key_nf4_asym=True, key_outlier_frac=0.02, key_zero_point="sparse",
                              key_rope_theta=1e4)
    _fill_and_check(cache, z)


def test_qwen_build_cache_takes_the_bias_zero_point():
    """AutoConfig for a Qwen registry model with this layer's k_proj bias
    resolves the "bias" zero point (turboquant_pro/autoconfig.py:390-417) and
    builds the GPU cache, which decodes within the bar of the oracle."""
    from turboquant_pro_amd import AutoConfig
    print("[variants] qwen2.5-7b build_cache(k_bias)", flush=True)
    cfg = AutoConfig.from_pretrained("qwen2.5-7b")
    H, Hq = cfg.n_kv_heads, cfg.n_q_heads
    assert (H, Hq) == (4, 28)      # 7 query heads per kv head
    kb = (np.random.default_rng(9).standard_normal((H, 128)) * 3).astype(np.float32)
    cache = cfg.build_cache(hot_window=64, seed=1, k_bias=kb, n_q_heads=Hq)
    assert cache.key_zero_point == "bias"
    k, v, q = O.synthetic_kv(77, 1, H, Hq, 200)
    cache.extend(k[0], v[0])
    sc = O.SequenceCache(hot_window=64, value_bits=cache.value_bits, outlier_frac=0.02,
                         zero_point="bias", rope_theta=cfg.rope_theta, k_bias=kb)
    sc.build(k[0], v[0], *cache._rotation)
    for i in range(cache.pool.n_groups(0)):
        assert np.array_equal(cache.pool.export_group(0, i)["kpacked"], sc.keys[i].packed), f"group {i}"
    # GQA: q-head i reads kv-head i // (Hq / Hkv)
    assert_attn_close(cache.fused_decode(q[0]), O.attend(q[0], sc.get_keys(), sc.get_values()))


LONG_CASES = [
    ("nf4_f32_s1000", 50, 1000, False, dict(nf4_asym=True), 0),
    ("nf4_f16_s2500", 51, 2500, True, dict(nf4_asym=True), 0),
    ("uni_f32_s1000", 52, 1000, False, dict(bits=4), 0),
    ("sparse_f32_s1000", 53, 1000, False, dict(nf4_asym=True, zero_point="sparse", rope_theta=1e4), 0),
    ("bias_f32_s1000", 54, 1000, False, dict(nf4_asym=True, zero_point="bias", rope_theta=1e6), 777),
]


@pytest.mark.parametrize("tag,seed,S,fp16,kw,pos", LONG_CASES, ids=[c[0] for c in LONG_CASES])
def test_per_channel_long_blocks_match_reference(tag, seed, S, fp16, kw, pos):
    """The block store's whole-layer records: one group of S tokens per
    (b, h), fp32 input encoded as given (no fp16 rounding)."""
    from turboquant_pro_amd import plugins as PL
    print(f"[variants] per_channel block {tag}", flush=True)
    z = _load("perchannel_long.npz")
    x = MG.long_block_input(seed, 2, S, fp16)
    kw = dict(kw)
    if kw.get("zero_point") == "bias":
        kw["k_bias"] = z["k_bias"]
    q = PL.create("per_channel", n_heads=2, outlier_frac=0.02, **kw)
    c = q.compress(x if not fp16 else x.astype(np.float16), packed=True, position_start=pos)
    assert _sha(c.indices) == str(z[f"{tag}_kpacked_sha"])
    if f"{tag}_nf4_scale" in z:
        assert np.array_equal(c.nf4_scale, z[f"{tag}_nf4_scale"])
    if f"{tag}_nf4_mean" in z:
        assert np.array_equal(c.nf4_mean, z[f"{tag}_nf4_mean"])
    elif f"{tag}_scale" not in z:
        assert c.nf4_mean is None
    if f"{tag}_scale" in z:
        assert np.array_equal(c.scale, z[f"{tag}_scale"]) and np.array_equal(c.zero, z[f"{tag}_zero"])
    assert np.array_equal(c.outlier_idx, z[f"{tag}_oidx"])
    assert np.array_equal(c.outlier_val.view(np.uint16), z[f"{tag}_oval"].view(np.uint16))
    assert c.position_start == (pos if "nf4_asym" in kw else 0)
    dec = q.decompress(c)
    assert _sha(dec.astype(np.float32)) == str(z[f"{tag}_dec_sha"])
    # the unpacked container decodes the same
    cu = q.compress(x, packed=False, position_start=pos)
    assert np.array_equal(q.decompress(cu), dec)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_polar_from_fp32_matches_reference(bits):
    from turboquant_pro_amd import plugins as PL
    print(f"[variants] polar fp32 bits={bits}", flush=True)
    z = _load("polar_f32.npz")
    v = MG.value_input(60, 2, 300)
    q = PL.create("polar", n_heads=2, bits=bits, seed=0)
    c = q.compress(v, packed=True, kind="value")
    assert np.array_equal(c.indices, z[f"b{bits}_packed"])
    assert np.array_equal(c.norms, z[f"b{bits}_norms"])
    assert _sha(q.decompress(c).astype(np.float32)) == str(z[f"b{bits}_dec_sha"])


@pytest.mark.parametrize("W,P", [(512, None), (16, None)], ids=["mfma", "valu"])
def test_v2_pool_decode_gqa(W, P):
    """2-bit values in a batched GQA pool: groups bit-exact to the oracle's
    encode and decode within the bar, on the MFMA kernel (W=512) and the VALU
    kernel (W=16: 8-token groups, per-token value rows)."""
    from turboquant_pro_amd import TQKVPool
    print(f"[variants] V2 pool W={W}", flush=True)
    B, Hkv, Hq, L = 2, 2, 8, (1400 if W == 512 else 90)
    k, v, q = O.synthetic_kv(31, B, Hkv, Hq, L)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, hot_window=W,
                    value_bits=2, seed=0)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    seqs, _ = oracle_state(k, v, W, 2, 0)
    for b in range(B):
        for g in range(pool.n_groups(b)):
            e = pool.export_group(b, g)
            assert np.array_equal(e["kpacked"], seqs[b].keys[g].packed)
            assert np.array_equal(e["vpacked"], seqs[b].values[g].packed), f"seq {b} group {g}"
            assert np.array_equal(e["vnorms"], seqs[b].values[g].norms)
    got = pool.decode(torch.from_numpy(q).cuda()).cpu().numpy()
    for b in range(B):
        assert_attn_close(got[b], seqs[b].attend(q[b]), what=f"V2 W={W} seq {b}")


def test_value_norm_beyond_the_decode_range_is_refused():
    """A value vector whose norm exceeds 16376 (weight <= 4 times the norm
    must stay below fp16's 65504 in the decode) is flagged by the encode;
    the pool refuses it at its next check (the append does not wait for the
    flag), and a decode checks before it runs."""
    from turboquant_pro_amd import TQKVPool
    print("[variants] value norm overflow", flush=True)
    k, v, _ = O.synthetic_kv(5, 1, 1, 1, 600)
    v = v.astype(np.float32)
    v[0, 0, 10] = 2000.0          # norm ~ 22600 > 16376
    pool = TQKVPool(n_kv_heads=1, max_batch=1, max_seq_len=600, seed=0)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v.astype(np.float16)).cuda())
    with pytest.raises(ValueError, match="16376"):
        pool.check()
    # the same through the decode of a second pool
    other = TQKVPool(n_kv_heads=1, max_batch=1, max_seq_len=600, seed=0)
    other.append(torch.from_numpy(k).cuda(), torch.from_numpy(v.astype(np.float16)).cuda())
    with pytest.raises(ValueError, match="16376"):
        other.decode(torch.zeros((1, 1, 128), dtype=torch.float16, device="cuda"))
    # the error is sticky: the offending codes stay, so a second decode (and
    # an export) raise too, until reset() drops the contents
    with pytest.raises(ValueError, match="16376"):
        other.decode(torch.zeros((1, 1, 128), dtype=torch.float16, device="cuda"))
    with pytest.raises(ValueError, match="16376"):
        other.export_group(0, 0)
    other.reset()
    other.check()
    # a pool with in-range norms has nothing pending after its checks
    _, v0, _ = O.synthetic_kv(5, 1, 1, 1, 600)
    ok = TQKVPool(n_kv_heads=1, max_batch=1, max_seq_len=600, seed=0)
    ok.append(torch.from_numpy(k).cuda(), torch.from_numpy(v0).cuda())
    ok.check()
    assert ok._pending == []


def test_side_list_beyond_its_cap_is_refused():
    """A group whose side-list needs more entries than ``outlier_cap`` sets
    the encode's flag; the pool's next check raises, and so does a decode."""
    from turboquant_pro_amd import TQKVPool
    print("[variants] side-list beyond outlier_cap", flush=True)
    k, v, _ = O.synthetic_kv(6, 1, 1, 1, 600)
    mk = lambda: TQKVPool(n_kv_heads=1, max_batch=1, max_seq_len=600, seed=0,  # noqa: E731
                          outlier_frac=0.1, outlier_cap=64)
    pool = mk()
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    with pytest.raises(RuntimeError, match="outlier_cap"):
        pool.check()
    other = mk()
    other.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    with pytest.raises(RuntimeError, match="outlier_cap"):
        other.decode(torch.zeros((1, 1, 128), dtype=torch.float16, device="cuda"))
    with pytest.raises(RuntimeError, match="outlier_cap"):
        other.decode(torch.zeros((1, 1, 128), dtype=torch.float16, device="cuda"))


def test_pool_grows_with_its_codes():
    """``TQKVPool.grown`` moves pages, group slots and hot rings through both
    clustered block tables (batch 2): the grown pool exports the same groups
    and decodes bit-identically, and further appends give the codes a pool of
    that size from the start gets."""
    from turboquant_pro_amd import TQKVPool
    print("[variants] pool growth", flush=True)
    B, Hkv, Hq = 2, 2, 8
    k, v, q = O.synthetic_kv(21, B, Hkv, Hq, 5000)
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    small = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=1500, seed=0)
    small.append(kd[:, :, :1400], vd[:, :, :1400], n_new=[1400, 1100])
    big = small.grown(5000)
    assert big.max_seq_len == 5000 and big.lengths == small.lengths
    for b in range(B):
        for g in range(small.n_groups(b)):
            a, c = small.export_group(b, g), big.export_group(b, g)
            for key in ("kpacked", "vpacked", "vnorms", "outlier_idx", "nf4_scale", "nf4_mean"):
                assert np.array_equal(np.asarray(a[key]), np.asarray(c[key])), f"seq {b} group {g} {key}"
    assert torch.equal(big.decode(qd), small.decode(qd))
    ref = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=5000, seed=0)
    ref.append(kd[:, :, :1400], vd[:, :, :1400], n_new=[1400, 1100])
    for p in (big, ref):
        p.append(kd[:, :, 1400:4900], vd[:, :, 1400:4900], n_new=[3500, 3500])
    for b in range(B):
        for g in range(ref.n_groups(b)):
            assert np.array_equal(big.export_group(b, g)["kpacked"], ref.export_group(b, g)["kpacked"])
            assert np.array_equal(big.export_group(b, g)["vpacked"], ref.export_group(b, g)["vpacked"])
    assert torch.equal(big.decode(qd), ref.decode(qd))


def test_hf_layer_grows_on_demand():
    """A TurboQuantLayer starts at 4096 tokens per sequence and doubles when a
    chunk needs more, up to max_cache_len."""
    from turboquant_pro_amd.hf_cache import TurboQuantLayer
    print("[variants] hf layer growth", flush=True)
    k, v, _ = O.synthetic_kv(23, 1, 2, 2, 5200)
    kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    layer = TurboQuantLayer(hot_window=512, value_bits=3, max_cache_len=6000)
    layer.update(kd[:, :, :100], vd[:, :, :100])
    assert layer.pool.max_seq_len == 4096
    kk, vv = layer.update(kd[:, :, 100:5000], vd[:, :, 100:5000])
    assert layer.pool.max_seq_len == 6000 and layer.get_seq_length() == 5000 and kk.shape[2] == 5000
    with pytest.raises(ValueError, match="max_cache_len"):
        layer.update(kd[:, :, :1100], vd[:, :, :1100])
