"""Pin the CPU oracle against the reference's own outputs (golden vectors
written by tests/golden/make_golden.py) and against closed forms.

These run on any machine (no GPU).  A plausible restatement mistake -- a wrong
pack bit order, a dropped tie in the outlier threshold, a wrong flush cadence,
the wrong value codebook -- fails at least one of them.
"""

import hashlib
import os

import numpy as np
import pytest

from oracle import tq_oracle as O


def _load(golden_dir, name):
    return np.load(os.path.join(golden_dir, name), allow_pickle=False)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ------------------------------------------------------------------ tables --

def test_rotation_and_codebooks_match_reference(golden_dir):
    g = _load(golden_dir, "rotation_d128_seed0.npz")
    pi, pi_t = O.rotation(0, 128)
    assert np.array_equal(pi, g["pi"]) and np.array_equal(pi_t, g["pi_t"])
    for b in (2, 3, 4):
        c, bnd = O.polar_codebook(b, 128)
        assert np.array_equal(c, g[f"cent{b}"]) and np.array_equal(bnd, g[f"bnd{b}"])
    # orthogonality (a transposed operand would still pass the equality above
    # only if the fixture were transposed too; this pins what Pi means)
    assert np.allclose(pi @ pi_t, np.eye(128), atol=1e-5)


def test_nf4_table_is_monotone_and_symmetric_ends():
    assert np.all(np.diff(O.NF4) > 0) and O.NF4[0] == -1.0 and O.NF4[-1] == 1.0 and O.NF4[7] == 0.0


# ------------------------------------------------------------------ packing --

def test_pack_known_answers(golden_dir):
    g = _load(golden_dir, "pack_kat.npz")
    for b in (2, 3, 4):
        for n in (1, 7, 13, 64, 257):
            codes = g[f"codes_b{b}_n{n}"]
            vp = O.pack_value_codes(codes, b)
            kp = O.pack_key_codes(codes, b)
            assert np.array_equal(vp, g[f"vpack_b{b}_n{n}"]), (b, n)
            assert np.array_equal(kp, g[f"kpack_b{b}_n{n}"]), (b, n)
            assert np.array_equal(O.unpack_value_codes(vp, n, b), codes)
            assert np.array_equal(O.unpack_key_codes(kp, n, b), codes)


def test_pack_3bit_closed_form():
    # tests/test_core.py:228-256: codes 0..7 -> one 24-bit little-endian word
    w = sum(i << (3 * i) for i in range(8))
    got = O.pack_value_codes(np.arange(8, dtype=np.uint8), 3)
    assert list(got) == [w & 0xFF, (w >> 8) & 0xFF, (w >> 16) & 0xFF]


def test_pack_4bit_key_is_bit_reversed_nibbles():
    # turboquant_pro/volta_kernels.py:270-280: byte -> (even code, odd code)
    def rev4(x):
        return int(f"{x:04b}"[::-1], 2)
    for a in range(16):
        for b in range(16):
            byte = O.pack_key_codes(np.array([a, b], np.uint8), 4)[0]
            assert byte == (rev4(a) << 4) | rev4(b)


# ------------------------------------------------------------- cache golds --

def _check_cache(g, hot_window, vbits, seed, full):
    k, v, q = g["k"], g["v"], g["q"]
    H, L, D = k.shape
    pi, pi_t = O.rotation(seed, D)
    sc = O.SequenceCache(hot_window=hot_window, value_bits=vbits, outlier_frac=0.02).build(k, v, pi, pi_t)
    assert len(sc.keys) == int(g["n_groups"]) == O.n_groups(L, hot_window)
    assert sc.hot_k.shape[1] == int(g["hot_length"])
    Gt = O.group_tokens(hot_window)
    for i, (kg, vg) in enumerate(zip(sc.keys, sc.values)):
        assert int(g[f"g{i}_position_start"]) == i * Gt
        assert np.array_equal(kg.packed, g[f"g{i}_kpacked"]), f"group {i} key codes"
        assert np.array_equal(kg.nf4_scale, g[f"g{i}_nf4_scale"])
        assert np.array_equal(kg.nf4_mean, g[f"g{i}_nf4_mean"])
        assert np.array_equal(kg.outlier_idx, g[f"g{i}_oidx"]), f"group {i} outlier idx"
        assert np.array_equal(kg.outlier_val.view(np.uint16), g[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(vg.packed, g[f"g{i}_vpacked"]), f"group {i} value codes"
        assert np.array_equal(vg.norms, g[f"g{i}_vnorms"])
    keys, vals = sc.get_keys(), sc.get_values()
    assert _sha(keys) == str(g["get_keys_sha"])
    assert _sha(vals) == str(g["get_values_sha"])
    if full:
        assert np.array_equal(keys, g["get_keys"]) and np.array_equal(vals, g["get_values"])
    out = O.attend(q, keys, vals)
    assert np.allclose(out, g["attn_out"], atol=1e-6, rtol=1e-5)


def test_cache_k4v3_w512_balanced(golden_dir):
    _check_cache(_load(golden_dir, "cache_k4v3_w512.npz"), 512, 3, 0, False)


def test_cache_k4v4_w16_robust(golden_dir):
    # robust() is K4/V4 with bits=3: decompress must use the value_bits codebook
    _check_cache(_load(golden_dir, "cache_k4v4_w16.npz"), 16, 4, 1, True)


def test_cache_k4v3_w64_outlier_ties(golden_dir):
    g = _load(golden_dir, "cache_k4v3_w64_ties.npz")
    # ties at the threshold must add entries beyond k per channel
    k_nominal = O.outlier_count_per_channel(32, 0.02) * 2 * 128
    assert g["g0_oidx"].size > k_nominal
    _check_cache(g, 64, 3, 2, True)


def test_perchannel_odd_group_length(golden_dir):
    g = _load(golden_dir, "perchannel_s200.npz")
    kg = O.encode_keys(g["x"], 0.02)
    assert np.array_equal(kg.packed, g["kpacked"])
    assert np.array_equal(kg.nf4_scale, g["nf4_scale"]) and np.array_equal(kg.nf4_mean, g["nf4_mean"])
    assert np.array_equal(kg.outlier_idx, g["oidx"])
    assert np.array_equal(kg.outlier_val.view(np.uint16), g["oval"].view(np.uint16))
    assert np.array_equal(O.decode_keys(kg), g["decompressed"])


# ------------------------------------------------------- closed-form attend --

def test_attend_uniform_scores_is_mean_of_values():
    rng = np.random.default_rng(0)
    k = np.ones((2, 50, 128), np.float32)
    v = rng.standard_normal((2, 50, 128)).astype(np.float32)
    q = np.zeros((8, 128), np.float32)
    out = O.attend(q, k, v)
    # GQA: q-heads 0..3 read kv-head 0, 4..7 read kv-head 1
    assert np.allclose(out[:4], v[0].mean(0), atol=1e-6)
    assert np.allclose(out[4:], v[1].mean(0), atol=1e-6)


def test_attend_one_hot_picks_a_row():
    k = np.zeros((1, 10, 128), np.float32)
    k[0, 3, 0] = 1000.0
    v = np.arange(10 * 128, dtype=np.float32).reshape(1, 10, 128)
    q = np.zeros((1, 128), np.float32)
    q[0, 0] = 1.0
    assert np.allclose(O.attend(q, k, v)[0], v[0, 3])


def test_merge_partials_equals_single_pass():
    rng = np.random.default_rng(1)
    s = rng.standard_normal((4, 30)).astype(np.float32) * 3
    vv = rng.standard_normal((4, 30, 16)).astype(np.float32)

    def part(a, b):
        m = s[:, a:b].max(1)
        e = np.exp(s[:, a:b] - m[:, None])
        return m, e.sum(1), np.einsum("hs,hsd->hd", e, vv[:, a:b])

    p = O.softmax_rows(s)
    want = np.einsum("hs,hsd->hd", p, vv)
    got = O.merge_partials([part(0, 7), part(7, 19), part(19, 30)])
    assert np.allclose(got, want, atol=1e-5)


def test_n_groups_cadence():
    # hot length is 512 for every power-of-two L >= 1024 at W=512
    for L in (1024, 2048, 32768, 131072):
        assert L - 256 * O.n_groups(L, 512) == 512
    assert O.n_groups(512, 512) == 0 and O.n_groups(513, 512) == 1 and O.n_groups(769, 512) == 2
    assert O.n_groups(768, 512) == 1


def test_decode_step_bytes_headline():
    b = O.decode_step_bytes([32768] * 16, 8, 32)
    assert abs(b / 1e6 - 591.2) < 0.5


@pytest.mark.parametrize("tag", ["s256", "s200"])
def test_uniform_keys_match_reference(golden_dir, tag):
    """Uniform per-channel keys (turboquant_pro/per_channel_kv.py:303-317,
    529-530) against the reference's own container and decompress
    (tests/golden/perchannel_uniform.npz): packed codes, scale, zero,
    outliers and the reconstruction, bit for bit."""
    import os
    z = np.load(os.path.join(golden_dir, "perchannel_uniform.npz"))
    g = O.encode_keys_uniform(z[f"{tag}_x"], 0.02)
    assert np.array_equal(g.packed, z[f"{tag}_kpacked"])
    assert np.array_equal(g.nf4_scale, z[f"{tag}_scale"]) and np.array_equal(g.nf4_mean, z[f"{tag}_zero"])
    assert np.array_equal(g.outlier_idx, z[f"{tag}_oidx"])
    assert np.array_equal(g.outlier_val.view(np.uint16), z[f"{tag}_oval"].view(np.uint16))
    assert np.array_equal(O.decode_keys(g), z[f"{tag}_decompressed"])
    # codes are in range and the grid's ends are hit
    assert g.codes.max() == 15 and g.codes.min() == 0
