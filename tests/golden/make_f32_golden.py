"""Write the golden vectors of the reference's fp32 caches.

Run once, in the build container only (the reference tree does not exist on
the GPU box):

    python tests/golden/make_f32_golden.py /path/to/reference

The reference's caches take fp32 tokens as they are; its own dispatch tests
(tests/test_kv_fused_pck.py:193-308) append fp32 keys with a per-channel DC
offset, 4 heads of head_dim 64, hot window 16, and query in fp32.  This script
builds those caches through the reference's public ``TurboQuantKVCache`` with
the same settings and seeded fp32 inputs, and stores inputs and outputs as
``.npz`` data, nothing else (``cache_f32.npz``, one set of arrays per variant
``<tag>_...``):

* ``uniform``: per-channel uniform 4-bit keys (the cache's default mode);
* ``nf4``: asym-NF4 keys with 2 % outliers;
* ``bias``: asym-NF4 + 2 % with the "bias" zero point (rope theta 1e6, a
  seeded k_proj bias), several groups at different positions;
* ``sym``: symmetric NF4 keys with 2 % outliers;
* ``polar``: PolarQuant keys (per_channel_keys=False), K4/V4.

Per variant: the appended ``k``/``v`` (H, L, D) fp32 and ``q`` (H, D) fp32,
every coded group's container arrays, ``get_keys``/``get_values`` over the
whole cache, the reference's ``fused_decode`` output and its
dequantize-then-attend truth (the reference test's ``_cache_truth``).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

H, D, L, W = 4, 64, 80, 16
THETA = 1e6


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from turboquant_pro.core import TurboQuantKVCache

    rng = np.random.default_rng(42)
    bias = rng.uniform(-2, 2, size=(H, D)).astype(np.float32)
    variants = {
        "uniform": dict(),
        "nf4": dict(key_nf4_asym=True, key_outlier_frac=0.02),
        "bias": dict(key_nf4_asym=True, key_outlier_frac=0.02, key_zero_point="bias",
                     key_rope_theta=THETA, key_k_bias=bias),
        "sym": dict(key_nf4=True, key_outlier_frac=0.02),
        "polar": dict(per_channel_keys=False),
    }
    out = {"k_bias": bias}
    for i, (tag, kw) in enumerate(variants.items()):
        r = np.random.default_rng(100 + i)
        per_channel = kw.pop("per_channel_keys", True)
        cache = TurboQuantKVCache(head_dim=D, n_heads=H, bits=4, hot_window=W, use_gpu=False, seed=0,
                                  per_channel_keys=per_channel, **kw)
        off = r.uniform(-4.0, 4.0, size=(H, D)).astype(np.float32)
        k = np.stack([(off + r.standard_normal((H, D))).astype(np.float32) for _ in range(L)], axis=1)
        v = r.standard_normal((H, L, D)).astype(np.float32)
        for t in range(L):
            cache.append(k[:, t], v[:, t])
        q = r.standard_normal((H, D)).astype(np.float32)
        out[f"{tag}_k"], out[f"{tag}_v"], out[f"{tag}_q"] = k, v, q
        out[f"{tag}_n_groups"] = np.int64(len(cache._cold_keys))
        out[f"{tag}_hot_length"] = np.int64(cache.length - cache.cold_length)
        for g, (ck, cv) in enumerate(zip(cache._cold_keys, cache._cold_values)):
            p = f"{tag}_g{g}_"
            out[p + "kpacked"] = ck.indices
            for name in ("nf4_scale", "nf4_mean", "outlier_idx", "outlier_val", "scale", "zero", "norms"):
                val = getattr(ck, name, None)
                if val is not None:
                    out[p + "k_" + name] = np.asarray(val)
            out[p + "vpacked"] = cv.indices
            out[p + "vnorms"] = cv.norms[0]
        keys = np.asarray(cache.get_keys(0, cache.length))[0]
        vals = np.asarray(cache.get_values(0, cache.length))[0]
        out[f"{tag}_get_keys"], out[f"{tag}_get_values"] = keys, vals
        sc = np.einsum("hd,hsd->hs", q, keys) / np.sqrt(D)
        sc = sc - sc.max(axis=-1, keepdims=True)
        p_ = np.exp(sc)
        p_ = p_ / p_.sum(axis=-1, keepdims=True)
        out[f"{tag}_truth"] = np.einsum("hs,hsd->hd", p_, vals)
        out[f"{tag}_fused"] = np.asarray(cache.fused_decode(q), np.float32)
        print(tag, "groups", len(cache._cold_keys), "max |fused - truth|",
              float(np.abs(out[f"{tag}_fused"] - out[f"{tag}_truth"]).max()))
    np.savez_compressed(HERE / "cache_f32.npz", **out)
    print("wrote cache_f32.npz")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
