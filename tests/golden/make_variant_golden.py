"""Write the golden vectors for the key/value variants beyond K4/V3
asym-NF4 and for the stateless block quantizers.

Run once, in the build container only (the reference tree does not exist on
the GPU box):

    python tests/golden/make_variant_golden.py /path/to/reference

The reference pins none of these with committed arrays, so this script drives
its public API on seeded inputs and stores inputs (or the seeds that
regenerate them, with a SHA-256 of the regenerated array) and outputs only:

* ``cache_k4v2_w512.npz``: the ``"compression"`` preset (K4/V2 asym-NF4 + 2 %
  outliers, turboquant_pro/autoconfig.py:158-163) built by
  ``AutoConfig.build_cache`` and fed token by token;
* ``cache_bias_w64.npz`` / ``cache_sparse_w64.npz``: ``TurboQuantKVCache``
  with ``key_zero_point="bias"`` (a k_proj bias, RoPE theta 1e6) and
  ``"sparse"`` (theta 1e4) (turboquant_pro/per_channel_kv.py:234-267,327-345,
  506-524);
* ``perchannel_long.npz``: ``PerChannelKV.compress`` / ``decompress`` on
  blocks of 1000 and 2500 tokens (fp32 and fp16-valued inputs; asym-NF4 with
  the three zero-point modes, uniform 4-bit), the block store's shape;
* ``polar_f32.npz``: ``TurboQuantKV.compress(kind="value")`` of fp32 inputs at
  2, 3 and 4 bits, packed, and its decompress.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
D = 128


def _sha(a: np.ndarray) -> np.ndarray:
    return np.array(hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest())


def long_block_input(seed: int, H: int, S: int, fp16: bool) -> np.ndarray:
    """(1, H, S, D) fp32 keys: N(0,1) x per-channel lognormal scale, 3 x10
    channels per head, a per-channel offset; rounded through fp16 if asked.
    Regenerated identically by the tests from the seed."""
    rng = np.random.default_rng(seed)
    scale = rng.lognormal(0.0, 1.0, size=(H, 1, D)).astype(np.float32)
    for h in range(H):
        scale[h, 0, rng.choice(D, size=3, replace=False)] *= 10.0
    x = rng.standard_normal((H, S, D)).astype(np.float32) * scale
    x = x + rng.uniform(-2, 2, size=(H, 1, D)).astype(np.float32)
    if fp16:
        x = x.astype(np.float16).astype(np.float32)
    return x[None]


def value_input(seed: int, H: int, S: int) -> np.ndarray:
    """(1, H, S, D) fp32 values, N(0,1) x a per-token scale (not fp16-exact)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((H, S, D)) * rng.uniform(0.1, 3.0, size=(H, S, 1)))[None].astype(np.float32)


def cache_inputs(seed: int, H: int, L: int):
    rng = np.random.default_rng(seed)
    scale = rng.lognormal(0.0, 1.0, size=(H, 1, D)).astype(np.float32)
    k = rng.standard_normal((H, L, D)).astype(np.float32) * scale
    k = k + 2.0 * rng.uniform(-1, 1, size=(H, 1, D)).astype(np.float32)
    v = rng.standard_normal((H, L, D)).astype(np.float32)
    return k.astype(np.float16), v.astype(np.float16)


def dump_cache(cache, k, v, q, path: Path) -> None:
    H, L, _ = k.shape
    for t in range(L):
        cache.append(k[:, t, :], v[:, t, :])
    out = {"k": k, "v": v, "q": q, "length": np.int64(cache.length),
           "cold_length": np.int64(cache.cold_length), "n_groups": np.int64(len(cache._cold_keys))}
    for i, (ck, cv) in enumerate(zip(cache._cold_keys, cache._cold_values)):
        out[f"g{i}_kpacked"] = ck.indices
        out[f"g{i}_nf4_scale"] = ck.nf4_scale[0]
        if ck.nf4_mean is not None:
            out[f"g{i}_nf4_mean"] = ck.nf4_mean[0]
        out[f"g{i}_oidx"] = ck.outlier_idx
        out[f"g{i}_oval"] = ck.outlier_val
        out[f"g{i}_vpacked"] = cv.indices
        out[f"g{i}_vnorms"] = cv.norms[0]
        out[f"g{i}_position_start"] = np.int64(ck.position_start)
        out[f"g{i}_zp_mode"] = np.array(ck.zp_mode)
    keys = np.asarray(cache.get_keys(0, cache.length))[0]
    vals = np.asarray(cache.get_values(0, cache.length))[0]
    out["get_keys_sha"], out["get_values_sha"] = _sha(keys), _sha(vals)
    out["get_keys_rows"], out["get_values_rows"] = keys[:, ::37], vals[:, ::37]
    sc = np.einsum("hd,hsd->hs", q.astype(np.float32), keys) / np.sqrt(D)
    p = np.exp(sc - sc.max(axis=-1, keepdims=True))
    out["attn_out"] = np.einsum("hs,hsd->hd", p / p.sum(axis=-1, keepdims=True), vals)
    np.savez_compressed(path, **out)
    print("wrote", path.name, int(out["n_groups"]), "groups")


def main(ref: str) -> None:
    sys.path.insert(0, ref)
    from turboquant_pro.autoconfig import AutoConfig
    from turboquant_pro.core import TurboQuantKV, TurboQuantKVCache
    from turboquant_pro.per_channel_kv import PerChannelKV

    # --- the "compression" preset: K4/V2 ------------------------------------
    cfg = AutoConfig.from_dict({"head_dim": D, "num_key_value_heads": 2, "num_attention_heads": 8,
                                "num_hidden_layers": 1}, target="compression")
    assert (cfg.key_bits, cfg.value_bits) == (4, 2)
    k, v = cache_inputs(40, 2, 770)
    q = np.random.default_rng(140).standard_normal((2, D)).astype(np.float16)
    dump_cache(cfg.build_cache(hot_window=512, use_gpu=False, seed=0), k, v, q, HERE / "cache_k4v2_w512.npz")

    # --- zero-point modes through the cache (position_start = cold length) --
    kb = (np.random.default_rng(41).standard_normal((2, D)) * 2.0).astype(np.float32)
    k, v = cache_inputs(42, 2, 300)
    q = np.random.default_rng(142).standard_normal((2, D)).astype(np.float16)
    cache = TurboQuantKVCache(head_dim=D, n_heads=2, bits=3, key_bits=4, value_bits=3, hot_window=64,
                              use_gpu=False, seed=3, key_nf4_asym=True, key_outlier_frac=0.02,
                              key_zero_point="bias", key_rope_theta=1e6, key_k_bias=kb)
    dump_cache(cache, k, v, q, HERE / "cache_bias_w64.npz")
    with np.load(HERE / "cache_bias_w64.npz") as z:
        data = dict(z)
    data["k_bias"], data["rope_theta"] = kb, np.float64(1e6)
    np.savez_compressed(HERE / "cache_bias_w64.npz", **data)
    cache = TurboQuantKVCache(head_dim=D, n_heads=2, bits=3, key_bits=4, value_bits=3, hot_window=64,
                              use_gpu=False, seed=3, key_nf4_asym=True, key_outlier_frac=0.02,
                              key_zero_point="sparse", key_rope_theta=1e4)
    dump_cache(cache, k, v, q, HERE / "cache_sparse_w64.npz")

    # --- PerChannelKV on long blocks (the block store's whole-layer records) -
    out = {}
    cases = [
        # tag, seed, S, fp16-valued, quantizer keywords, position_start
        ("nf4_f32_s1000", 50, 1000, False, dict(nf4_asym=True, outlier_frac=0.02), 0),
        ("nf4_f16_s2500", 51, 2500, True, dict(nf4_asym=True, outlier_frac=0.02), 0),
        ("uni_f32_s1000", 52, 1000, False, dict(outlier_frac=0.02), 0),
        ("sparse_f32_s1000", 53, 1000, False,
         dict(nf4_asym=True, outlier_frac=0.02, zero_point="sparse", rope_theta=1e4), 0),
        ("bias_f32_s1000", 54, 1000, False,
         dict(nf4_asym=True, outlier_frac=0.02, zero_point="bias", rope_theta=1e6, k_bias=kb), 777),
    ]
    for tag, seed, S, fp16, kw, pos in cases:
        x = long_block_input(seed, 2, S, fp16)
        pk = PerChannelKV(head_dim=D, n_heads=2, bits=4, **kw)
        c = pk.compress(x, packed=True, position_start=pos)
        dec = pk.decompress(c)
        out[f"{tag}_x_sha"] = _sha(x)
        out[f"{tag}_kpacked_sha"] = _sha(c.indices)
        out[f"{tag}_kpacked_head"] = c.indices[:4096]
        if c.nf4_scale is not None:
            out[f"{tag}_nf4_scale"] = c.nf4_scale
        if c.nf4_mean is not None:
            out[f"{tag}_nf4_mean"] = c.nf4_mean
        if c.scale is not None:
            out[f"{tag}_scale"], out[f"{tag}_zero"] = c.scale, c.zero
        out[f"{tag}_oidx"] = c.outlier_idx
        out[f"{tag}_oval"] = c.outlier_val
        out[f"{tag}_dec_sha"] = _sha(dec.astype(np.float32))
        out[f"{tag}_dec_rows"] = dec[0, :, :3].astype(np.float32)
        print(tag, c.indices.shape, c.outlier_idx.shape)
    out["k_bias"] = kb
    np.savez_compressed(HERE / "perchannel_long.npz", **out)

    # --- PolarQuant values from fp32 -----------------------------------------
    out = {}
    v = value_input(60, 2, 300)
    out["v_sha"] = _sha(v)
    for b in (2, 3, 4):
        tq = TurboQuantKV(head_dim=D, n_heads=2, bits=b, use_gpu=False, seed=0)
        c = tq.compress(v, packed=True, kind="value")
        out[f"b{b}_packed"] = c.indices
        out[f"b{b}_norms"] = c.norms
        dec = tq.decompress(c)
        out[f"b{b}_dec_sha"] = _sha(dec.astype(np.float32))
        out[f"b{b}_dec_rows"] = dec[0, :, :3].astype(np.float32)
    np.savez_compressed(HERE / "polar_f32.npz", **out)
    print("done")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
