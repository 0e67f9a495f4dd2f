"""Write the golden vectors of the reference's symmetric-NF4 keys.

Run once, in the build container only (the reference tree does not exist on
the GPU box):

    python tests/golden/make_sym_golden.py /path/to/reference

Symmetric NF4 (``PerChannelKV(nf4=True)`` without ``nf4_asym``,
turboquant_pro/per_channel_kv.py:354-357; ``TurboQuantKVCache(key_nf4=True)``)
is its own branch of the reference's encode: the per-channel abs-max of the
raw channel scales the NF4 grid, no mean is taken or stored
(``nf4_mean is None``, ``zp_mode == "calibrated"``), and the decompress adds
none (:503-524).  This script drives the reference's public API on seeded
inputs with per-channel offsets (where symmetric and asymmetric codes differ)
and stores inputs and outputs as ``.npz`` data, nothing else:

* ``cache_symnf4_w64.npz``: a K4/V3 ``TurboQuantKVCache`` with symmetric-NF4
  keys and 2 % outliers, hot window 64, 300 fp16 tokens appended one by one:
  every group's containers, ``get_keys``/``get_values`` digests and the
  dequantize-then-attend output for an fp16 query;
* ``perchannel_symnf4.npz``: ``PerChannelKV(nf4=True, outlier_frac=0.02)`` on
  a 520-token fp32 block of 2 heads: packed codes, scales, outliers and the
  decompress.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

from make_golden import _inputs, _sha  # noqa: E402


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from turboquant_pro.core import TurboQuantKVCache
    from turboquant_pro.per_channel_kv import PerChannelKV

    D = 128
    cache = TurboQuantKVCache(head_dim=D, n_heads=2, bits=3, key_bits=4, value_bits=3,
                              hot_window=64, use_gpu=False, seed=3, key_nf4=True,
                              key_outlier_frac=0.02)
    k, v = _inputs(7, 2, 300, D, dc=3.0)
    q = np.random.default_rng(107).standard_normal((2, D)).astype(np.float16)
    for t in range(k.shape[1]):
        cache.append(k[:, t, :], v[:, t, :])
    out = {"k": k, "v": v, "q": q, "length": np.int64(cache.length),
           "cold_length": np.int64(cache.cold_length), "n_groups": np.int64(len(cache._cold_keys))}
    for i, (ck, cv) in enumerate(zip(cache._cold_keys, cache._cold_values)):
        assert ck.nf4_mean is None and ck.zp_mode == "calibrated"
        out[f"g{i}_kpacked"] = ck.indices
        out[f"g{i}_nf4_scale"] = ck.nf4_scale[0]
        out[f"g{i}_oidx"] = ck.outlier_idx
        out[f"g{i}_oval"] = ck.outlier_val
        out[f"g{i}_vpacked"] = cv.indices
        out[f"g{i}_vnorms"] = cv.norms[0]
    keys = np.asarray(cache.get_keys(0, cache.length))[0]
    vals = np.asarray(cache.get_values(0, cache.length))[0]
    out["get_keys_sha"] = np.array(_sha(keys))
    out["get_values_sha"] = np.array(_sha(vals))
    sc = np.einsum("hd,hsd->hs", q.astype(np.float32), keys) / np.sqrt(D)
    sc = sc - sc.max(axis=-1, keepdims=True)
    p = np.exp(sc)
    p = p / p.sum(axis=-1, keepdims=True)
    out["attn_out"] = np.einsum("hs,hsd->hd", p, vals)
    np.savez_compressed(HERE / "cache_symnf4_w64.npz", **out)
    print("wrote cache_symnf4_w64.npz groups", len(cache._cold_keys))

    pk = PerChannelKV(head_dim=D, n_heads=2, bits=4, nf4=True, outlier_frac=0.02)
    x = _inputs(8, 2, 520, D, dc=2.0)[0].astype(np.float32)
    x = x + np.random.default_rng(9).standard_normal(x.shape).astype(np.float32) * 1e-3  # fp32-valued
    c = pk.compress(x[None], packed=True)
    assert c.nf4_mean is None
    np.savez_compressed(HERE / "perchannel_symnf4.npz", x=x, kpacked=c.indices,
                        nf4_scale=c.nf4_scale[0], oidx=c.outlier_idx, oval=c.outlier_val,
                        decompressed=pk.decompress(c)[0])
    print("wrote perchannel_symnf4.npz")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
