"""Write the golden vectors for 3- and 2-bit uniform per-channel keys, the
reference's default key form (``TurboQuantKVCache(bits=3)``,
turboquant_pro/core.py:886-950, and ``PerChannelKV(bits=...)``,
turboquant_pro/per_channel_kv.py:285-317,497-539).

Run once, in the build container only (the reference tree does not exist on
the GPU box):

    python tests/golden/make_lowbit_golden.py /path/to/reference

Inputs are regenerated from seeds by the tests (``cache_inputs`` /
``long_block_input`` of make_variant_golden.py); the files hold a SHA-256 of
each input and the reference's outputs:

* ``cache_k3v3_default_w64.npz``: the reference's default cache (3-bit uniform
  keys without outliers, 3-bit PolarQuant values), hot window 64, fed token by
  token;
* ``cache_k2v2_w64.npz``: bits=2 with 2 % key outliers;
* ``cache_k3v4_w512.npz``: 3-bit uniform keys with 2 % outliers, 4-bit
  values, hot window 512;
* ``perchannel_lowbit.npz``: ``PerChannelKV`` compress / decompress at 3 and 2
  bits (2 % outliers) of 256-token fp16-valued and 1000-token fp32 blocks.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import make_variant_golden as MG  # noqa: E402

D = 128

# (file, seed, H, L, query seed, constructor keywords)
CACHES = [
    ("cache_k3v3_default_w64.npz", 70, 2, 300, 170, dict(bits=3, hot_window=64, seed=5)),
    ("cache_k2v2_w64.npz", 71, 2, 300, 171, dict(bits=2, hot_window=64, seed=6, key_outlier_frac=0.02)),
    ("cache_k3v4_w512.npz", 72, 2, 800, 172,
     dict(bits=3, key_bits=3, value_bits=4, hot_window=512, seed=7, key_outlier_frac=0.02)),
]
# (tag, seed, S, fp16-valued, bits)
BLOCKS = [
    ("k3_f16_s256", 80, 256, True, 3),
    ("k2_f16_s256", 81, 256, True, 2),
    ("k3_f32_s1000", 82, 1000, False, 3),
    ("k2_f32_s1000", 83, 1000, False, 2),
]


def dump_uniform_cache(cache, k, v, q, path: Path) -> None:
    H, L, _ = k.shape
    for t in range(L):
        cache.append(k[:, t, :], v[:, t, :])
    out = {"k_sha": MG._sha(k), "v_sha": MG._sha(v), "q": q, "length": np.int64(cache.length),
           "n_groups": np.int64(len(cache._cold_keys))}
    for i, (ck, cv) in enumerate(zip(cache._cold_keys, cache._cold_values)):
        out[f"g{i}_kpacked"] = ck.indices
        out[f"g{i}_scale"] = ck.scale[0, :, 0, :]
        out[f"g{i}_zero"] = ck.zero[0, :, 0, :]
        if ck.outlier_idx is not None:
            out[f"g{i}_oidx"] = ck.outlier_idx
            out[f"g{i}_oval"] = ck.outlier_val
        out[f"g{i}_vpacked"] = cv.indices
        out[f"g{i}_vnorms"] = cv.norms[0]
    keys = np.asarray(cache.get_keys(0, cache.length))[0]
    vals = np.asarray(cache.get_values(0, cache.length))[0]
    out["get_keys_sha"], out["get_values_sha"] = MG._sha(keys), MG._sha(vals)
    out["get_keys_rows"], out["get_values_rows"] = keys[:, ::37], vals[:, ::37]
    sc = np.einsum("hd,hsd->hs", q.astype(np.float32), keys) / np.sqrt(D)
    p = np.exp(sc - sc.max(axis=-1, keepdims=True))
    out["attn_out"] = np.einsum("hs,hsd->hd", p / p.sum(axis=-1, keepdims=True), vals)
    np.savez_compressed(path, **out)
    print("wrote", path.name, int(out["n_groups"]), "groups")


def main(ref: str) -> None:
    sys.path.insert(0, ref)
    from turboquant_pro.core import TurboQuantKVCache
    from turboquant_pro.per_channel_kv import PerChannelKV

    for name, seed, H, L, qseed, kw in CACHES:
        k, v = MG.cache_inputs(seed, H, L)
        q = np.random.default_rng(qseed).standard_normal((H, D)).astype(np.float16)
        cache = TurboQuantKVCache(head_dim=D, n_heads=H, use_gpu=False, **kw)
        assert cache.per_channel_keys and cache._kq is not None
        dump_uniform_cache(cache, k, v, q, HERE / name)

    out = {}
    for tag, seed, S, fp16, bits in BLOCKS:
        x = MG.long_block_input(seed, 2, S, fp16)
        pk = PerChannelKV(head_dim=D, n_heads=2, bits=bits, outlier_frac=0.02)
        c = pk.compress(x, packed=True)
        dec = pk.decompress(c)
        out[f"{tag}_x_sha"] = MG._sha(x)
        out[f"{tag}_kpacked"] = c.indices
        out[f"{tag}_scale"], out[f"{tag}_zero"] = c.scale, c.zero
        out[f"{tag}_oidx"] = c.outlier_idx
        out[f"{tag}_oval"] = c.outlier_val
        out[f"{tag}_dec_sha"] = MG._sha(dec.astype(np.float32))
        out[f"{tag}_dec_rows"] = dec[0, :, :3].astype(np.float32)
        print(tag, c.indices.shape, c.outlier_idx.shape)
    np.savez_compressed(HERE / "perchannel_lowbit.npz", **out)
    print("done")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
