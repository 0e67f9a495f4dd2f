"""Write the golden vectors that pin the oracle to the reference implementation.

Run once, in the build container only (the reference tree does not exist on
the GPU box):

    python tests/golden/make_golden.py /path/to/reference

The reference ships no golden arrays for its KV path (all its KV tests are
tolerance or self-consistency based), so this script drives the reference's
own public API -- ``TurboQuantKVCache`` (turboquant_pro/core.py:818-1307),
``PerChannelKV`` (turboquant_pro/per_channel_kv.py:145-539) and
``TurboQuantKV`` (turboquant_pro/core.py:139-810) -- on small seeded inputs and
stores inputs and outputs as ``.npz`` data.  Nothing from the reference is
stored except these input/output arrays.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _inputs(seed: int, H: int, L: int, D: int, dc: float = 0.0):
    """Seeded fp16 keys with a per-channel lognormal scale, a few x10 channels,
    an optional DC offset, and N(0,1) values."""
    rng = np.random.default_rng(seed)
    scale = rng.lognormal(0.0, 1.0, size=(H, 1, D)).astype(np.float32)
    for h in range(H):
        scale[h, 0, rng.choice(D, size=3, replace=False)] *= 10.0
    k = rng.standard_normal((H, L, D)).astype(np.float32) * scale
    k = k + dc * rng.uniform(-1, 1, size=(H, 1, D)).astype(np.float32)
    v = rng.standard_normal((H, L, D)).astype(np.float32)
    return k.astype(np.float16), v.astype(np.float16)


def _dump_cache(cache, k, v, q, path: Path, store_full: bool) -> None:
    H, L, D = k.shape
    for t in range(L):
        cache.append(k[:, t, :], v[:, t, :])
    out = {"k": k, "v": v, "q": q,
           "length": np.int64(cache.length), "cold_length": np.int64(cache.cold_length),
           "hot_length": np.int64(cache.hot_length),
           "n_groups": np.int64(len(cache._cold_keys))}
    for i, (ck, cv) in enumerate(zip(cache._cold_keys, cache._cold_values)):
        out[f"g{i}_kpacked"] = ck.indices
        out[f"g{i}_nf4_scale"] = ck.nf4_scale[0]
        out[f"g{i}_nf4_mean"] = ck.nf4_mean[0]
        out[f"g{i}_oidx"] = ck.outlier_idx
        out[f"g{i}_oval"] = ck.outlier_val
        out[f"g{i}_vpacked"] = cv.indices
        out[f"g{i}_vnorms"] = cv.norms[0]
        out[f"g{i}_position_start"] = np.int64(ck.position_start)
    keys = np.asarray(cache.get_keys(0, cache.length))[0]
    vals = np.asarray(cache.get_values(0, cache.length))[0]
    if store_full:
        out["get_keys"], out["get_values"] = keys, vals
    out["get_keys_sha"] = np.array(_sha(keys))
    out["get_values_sha"] = np.array(_sha(vals))
    # attention over the reconstruction (tests/test_kv_fused_pck.py:202-208 formula)
    sc = np.einsum("hd,hsd->hs", q.astype(np.float32), keys) / np.sqrt(D)
    sc = sc - sc.max(axis=-1, keepdims=True)
    p = np.exp(sc)
    p = p / p.sum(axis=-1, keepdims=True)
    out["attn_out"] = np.einsum("hs,hsd->hd", p, vals)
    np.savez_compressed(path, **out)
    print("wrote", path.name, {k_: getattr(v_, "shape", None) for k_, v_ in out.items()
                               if k_.startswith("g0_") or k_ in ("k",)})


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from turboquant_pro.autoconfig import AutoConfig
    from turboquant_pro.core import TurboQuantKV, TurboQuantKVCache
    from turboquant_pro.per_channel_kv import PerChannelKV, _pack_indices

    D = 128
    # --- rotation + codebooks (seed 0, d=128) -------------------------------
    tq = TurboQuantKV(head_dim=D, n_heads=2, bits=3, use_gpu=False, seed=0)
    books = {}
    for b in (2, 3, 4):
        c, bnd = TurboQuantKV(head_dim=D, bits=b, use_gpu=False, seed=0)._codebooks[b]
        books[f"cent{b}"], books[f"bnd{b}"] = c, bnd
    np.savez_compressed(HERE / "rotation_d128_seed0.npz", pi=tq._Pi, pi_t=tq._Pi_T, **books)

    # --- pack known answers (both layouts, 2/3/4-bit, ragged lengths) --------
    rng = np.random.default_rng(5)
    packs = {}
    for b in (2, 3, 4):
        for n in (1, 7, 13, 64, 257):
            codes = rng.integers(0, 2 ** b, size=n, dtype=np.uint8)
            packs[f"codes_b{b}_n{n}"] = codes
            packs[f"vpack_b{b}_n{n}"] = TurboQuantKV(head_dim=64, bits=b, use_gpu=False,
                                                     seed=0)._pack_bits(codes)
            packs[f"kpack_b{b}_n{n}"] = _pack_indices(codes, b)
    np.savez_compressed(HERE / "pack_kat.npz", **packs)

    # --- the north-star cache: AutoConfig "balanced" = K4/V3 asym-NF4 + 2% ----
    cfg = AutoConfig.from_dict({"head_dim": D, "num_key_value_heads": 2,
                                "num_attention_heads": 8, "num_hidden_layers": 1},
                               target="balanced")
    cache = cfg.build_cache(hot_window=512, use_gpu=False, seed=0)
    k, v = _inputs(0, 2, 770, D)
    q = np.random.default_rng(100).standard_normal((2, D)).astype(np.float16)
    _dump_cache(cache, k, v, q, HERE / "cache_k4v3_w512.npz", store_full=False)

    # --- robust() = K4/V4, small hot window (group of 8), full reconstructions
    cache = TurboQuantKVCache.robust(head_dim=D, n_heads=2, hot_window=16,
                                     use_gpu=False, seed=1)
    k, v = _inputs(1, 2, 45, D, dc=4.0)
    q = np.random.default_rng(101).standard_normal((2, D)).astype(np.float16)
    _dump_cache(cache, k, v, q, HERE / "cache_k4v4_w16.npz", store_full=True)

    # --- K4/V3 with a small window and coarse keys (outlier magnitude ties) ---
    cache = TurboQuantKVCache(head_dim=D, n_heads=2, bits=3, key_bits=4, value_bits=3,
                              hot_window=64, use_gpu=False, seed=2, key_nf4_asym=True,
                              key_outlier_frac=0.02)
    k, v = _inputs(2, 2, 150, D)
    k = (np.round(k.astype(np.float32) * 2.0) / 2.0).astype(np.float16)  # many |x| ties
    k[1, :, 7] = 0.0                     # a constant channel: every token ties
    q = np.random.default_rng(102).standard_normal((2, D)).astype(np.float16)
    _dump_cache(cache, k, v, q, HERE / "cache_k4v3_w64_ties.npz", store_full=True)

    # --- PerChannelKV.compress directly on an odd group length ---------------
    pk = PerChannelKV(head_dim=D, n_heads=3, bits=4, nf4_asym=True, outlier_frac=0.02)
    x = _inputs(3, 3, 200, D, dc=2.0)[0].astype(np.float32)[None]
    c = pk.compress(x, packed=True)
    np.savez_compressed(HERE / "perchannel_s200.npz", x=x[0], kpacked=c.indices,
                        nf4_scale=c.nf4_scale[0], nf4_mean=c.nf4_mean[0],
                        oidx=c.outlier_idx, oval=c.outlier_val,
                        decompressed=pk.decompress(c)[0])
    print("done")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
