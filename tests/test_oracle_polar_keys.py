"""PolarQuant keys (``TurboQuantKVCache(per_channel_keys=False)``) on the CPU.

The reference flushes such keys with ``TurboQuantKV.compress(kind="key")``
(turboquant_pro/core.py:1028-1029): the very encode it runs on values
(core.py:542-617), with the codebook of ``key_bits`` (``_resolve_bits``,
core.py:534-540).  With ``key_bits == value_bits`` a key group of tokens X is
therefore the value group the reference wrote for the same tokens X, so the
reference-written value groups of four fixture caches (3-, 2-, 4- and 3-bit,
hot windows 64, 64, 16 and 512) pin the oracle's key groups bit for bit when
a cache is fed those values as its keys.  The decode's on-codes score
``|k| * (q @ Pi_T) . cent[code]`` (turboquant_pro/kv_fused.py:83-98) is pinned
against ``q . k`` of the dequantised keys, and a transposed rotation fails it.
"""

import hashlib
import os
import sys

import numpy as np
import pytest

from oracle import tq_oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLD)
import make_variant_golden as MG  # noqa: E402  (input generators only)

# (fixture, bits, hot window, rotation seed, value input): every fixture's
# value groups are the reference's PolarQuant encode of its values
FIXTURES = [
    ("cache_k3v3_default_w64.npz", 3, 64, 5, lambda z: MG.cache_inputs(70, 2, 300)[1]),
    ("cache_k2v2_w64.npz", 2, 64, 6, lambda z: MG.cache_inputs(71, 2, 300)[1]),
    ("cache_k4v4_w16.npz", 4, 16, 1, lambda z: z["v"]),
    ("cache_k4v3_w512.npz", 3, 512, 0, lambda z: z["v"]),
]


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def polar_key_cache(v, bits, W, seed):
    """Oracle cache whose keys and values are both ``v`` (H, L, D)."""
    return O.SequenceCache(hot_window=W, value_bits=bits, key_bits=bits, outlier_frac=0.0,
                           key_grid="polar", seed=seed).build(v, v, *O.rotation(seed, 128))


@pytest.mark.parametrize("case", FIXTURES, ids=[c[0] for c in FIXTURES])
def test_polar_key_groups_match_reference_value_groups(case):
    name, bits, W, seed, src = case
    z = np.load(os.path.join(GOLD, name))
    v = src(z)
    sc = polar_key_cache(v, bits, W, seed)
    assert len(sc.keys) == int(z["n_groups"])
    for i, kg in enumerate(sc.keys):
        assert isinstance(kg, O.ValueGroup) and kg.bits == bits
        assert np.array_equal(kg.packed, z[f"g{i}_vpacked"]), f"group {i} key codes"
        assert np.array_equal(kg.norms, z[f"g{i}_vnorms"]), f"group {i} key norms"
    # get_keys of the coded keys = the reference's get_values of the same tokens
    assert _sha(sc.get_keys()) == str(z["get_values_sha"])


def test_on_codes_score_equals_dequantised_dot():
    """``|k| * (q @ Pi_T) . cent[code]`` == ``q . ((cent[code] @ Pi) * |k|)``
    to fp32 rounding, per token; the same formula with ``Pi`` in place of
    ``Pi_T`` (a transposed operand) is far off."""
    bits, seed = 3, 5
    v = MG.cache_inputs(70, 2, 300)[1]
    sc = polar_key_cache(v, bits, 64, seed)
    pi, pi_t = O.rotation(seed, 128)
    cent, _ = O.polar_codebook(bits, 128)
    q = np.random.default_rng(9).standard_normal((2, 128)).astype(np.float32)
    for kg in sc.keys:
        deq = O.decode_values(kg, cent, pi)                          # (H, S, D)
        want = np.einsum("hsd,hd->hs", deq.astype(np.float64), q.astype(np.float64))
        y = cent[kg.codes].astype(np.float64)                        # (H, S, D)
        got = kg.norms * np.einsum("hsd,hd->hs", y, q @ pi_t.astype(np.float64))
        assert np.allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
        wrong = kg.norms * np.einsum("hsd,hd->hs", y, q @ pi.astype(np.float64))
        assert not np.allclose(wrong, want, rtol=1e-2, atol=1e-2 * np.abs(want).max())


def test_polar_keys_attend_is_dense_attention_of_the_dequantised_cache():
    v = MG.cache_inputs(71, 2, 300)[1]
    sc = polar_key_cache(v, 2, 64, 6)
    q = np.random.default_rng(3).standard_normal((4, 128)).astype(np.float16)   # GQA 2
    k, vv = sc.get_keys(), sc.get_values()
    assert np.array_equal(k, vv)            # keys and values were the same tokens
    out = sc.attend(q)
    s = np.einsum("hd,hsd->hs", q.astype(np.float32), np.repeat(k, 2, axis=0)) / np.sqrt(128)
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = np.einsum("hs,hsd->hd", p / p.sum(-1, keepdims=True), np.repeat(vv, 2, axis=0))
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_polar_keys_need_equal_widths():
    v = MG.cache_inputs(70, 2, 100)[1]
    with pytest.raises(ValueError):
        O.SequenceCache(hot_window=16, value_bits=3, key_bits=4, outlier_frac=0.0,
                        key_grid="polar").build(v, v, *O.rotation(0, 128))
