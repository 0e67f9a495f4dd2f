"""Write the golden vectors of the reference at head_dim 64 and 256.

Run once, in the build container only (the reference tree does not exist on
the GPU box):

    python tests/golden/make_hd_golden.py /path/to/reference

The reference's caches and quantizers take any head_dim (its fused kernel
any d % 32 == 0 up to 512, turboquant_pro/kv_kernel.py:334-335; its registry
holds two head_dim-256 models, turboquant_pro/autoconfig.py:76-91).  This
script drives the reference's public API on seeded inputs and stores inputs
and outputs as ``.npz`` data, nothing else:

* ``cache_gemma2_9b_w64.npz``: ``AutoConfig.from_pretrained("gemma-2-9b")
  .build_cache(hot_window=64)`` -- 8 kv heads of head_dim 256, asym-NF4 keys
  with 2 % outliers and 3-bit values -- after 150 fp16 tokens appended one by
  one, with the cache's rotation and codebook;
* ``cache_d64_k4v4_w32.npz``: a K4/V4 asym-NF4 + 2 % cache of head_dim 64,
  hot window 32, 120 tokens;
* ``perchannel_d256.npz`` / ``polar_d64.npz``: ``PerChannelKV`` (asym-NF4,
  2 % outliers) on a 300-token fp32 block of head_dim 256 and
  ``TurboQuantKV.compress(kind="value")`` on a 3-bit fp32 block of head_dim 64,
  each with its decompress.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

from make_golden import _dump_cache, _inputs  # noqa: E402


def _with_rotation(path: Path, cache) -> None:
    z = dict(np.load(path))
    tq = cache._tq
    z["pi"], z["pi_t"] = tq._Pi, tq._Pi_T
    c, bnd = tq._codebooks[cache.value_bits]
    z["vcent"], z["vbnd"] = c, bnd
    z["zp_modes"] = np.array([ck.zp_mode for ck in cache._cold_keys])
    np.savez_compressed(path, **z)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from turboquant_pro.autoconfig import AutoConfig
    from turboquant_pro.core import TurboQuantKV, TurboQuantKVCache
    from turboquant_pro.per_channel_kv import PerChannelKV

    cfg = AutoConfig.from_pretrained("gemma-2-9b")
    cache = cfg.build_cache(hot_window=64, use_gpu=False, seed=6)
    assert cache.head_dim == 256 and cache.n_heads == 8
    k, v = _inputs(20, 8, 150, 256, dc=2.0)
    q = np.random.default_rng(120).standard_normal((8, 256)).astype(np.float16)
    path = HERE / "cache_gemma2_9b_w64.npz"
    _dump_cache(cache, k, v, q, path, store_full=False)
    _with_rotation(path, cache)

    cache = TurboQuantKVCache(head_dim=64, n_heads=2, bits=4, key_bits=4, value_bits=4,
                              hot_window=32, use_gpu=False, seed=7, key_nf4_asym=True,
                              key_outlier_frac=0.02)
    k, v = _inputs(21, 2, 120, 64, dc=3.0)
    q = np.random.default_rng(121).standard_normal((2, 64)).astype(np.float16)
    path = HERE / "cache_d64_k4v4_w32.npz"
    _dump_cache(cache, k, v, q, path, store_full=True)
    _with_rotation(path, cache)

    pk = PerChannelKV(head_dim=256, n_heads=2, bits=4, nf4_asym=True, outlier_frac=0.02)
    x = _inputs(22, 2, 300, 256, dc=2.0)[0].astype(np.float32)
    x = x + np.random.default_rng(23).standard_normal(x.shape).astype(np.float32) * 1e-3
    c = pk.compress(x[None], packed=True)
    np.savez_compressed(HERE / "perchannel_d256.npz", x=x, kpacked=c.indices,
                        nf4_scale=c.nf4_scale[0], nf4_mean=c.nf4_mean[0], oidx=c.outlier_idx,
                        oval=c.outlier_val, decompressed=pk.decompress(c)[0])

    tq = TurboQuantKV(head_dim=64, n_heads=2, bits=3, use_gpu=False, seed=8)
    xv = np.random.default_rng(24).standard_normal((1, 2, 200, 64)).astype(np.float32) * 2
    cv = tq.compress(xv, packed=True, kind="value")
    np.savez_compressed(HERE / "polar_d64.npz", x=xv[0], packed=cv.indices, norms=cv.norms[0],
                        pi=tq._Pi, pi_t=tq._Pi_T, decompressed=tq.decompress(cv)[0])
    print("done")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
