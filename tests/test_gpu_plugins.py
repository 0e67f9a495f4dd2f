"""The plugin formats on the GPU (turboquant_pro/plugins.py:300-360):

* ``create("per_channel", nf4_asym=True, outlier_frac=0.02).compress`` of the
  reference's own S=200 block (tests/golden/perchannel_s200.npz, written by
  ``PerChannelKV.compress``) reproduces its container bit for bit, packed and
  unpacked; ``decompress`` reproduces the reference's ``decompress`` bit for
  bit; batches of two round-trip bit-exact against the oracle.
* ``create("polar", bits=3, seed=0).compress(v, kind="value", packed=True)``
  of the first flushed group of the reference cache fixture reproduces that
  group's value bytes and norms; ``decompress`` equals the oracle's
  ``decode_values`` bit for bit, and a 300-token block (two encode groups)
  round-trips the same way.
"""

import os

import numpy as np
import pytest

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _pl():
    from turboquant_pro_amd import plugins
    return plugins


def test_per_channel_compress_matches_reference_container():
    print("[plugins] per_channel S=200 compress", flush=True)
    PL = _pl()
    z = np.load(os.path.join(GOLD, "perchannel_s200.npz"), allow_pickle=False)
    x = z["x"][None]
    q = PL.create("per_channel", n_heads=3, nf4_asym=True, outlier_frac=0.02)
    c = q.compress(x, packed=True)
    assert c.shape == x.shape and c.packed and c.bits == 4 and c.zp_mode == "calibrated"
    assert np.array_equal(c.indices, z["kpacked"])
    assert np.array_equal(c.nf4_scale[0], z["nf4_scale"])
    assert np.array_equal(c.nf4_mean[0], z["nf4_mean"])
    assert np.array_equal(c.outlier_idx, z["oidx"]) and c.outlier_idx.dtype == np.int32
    assert np.array_equal(c.outlier_val.view(np.uint16), z["oval"].view(np.uint16))
    cu = q.compress(x, packed=False)
    assert np.array_equal(cu.indices, q.codes(c))
    print("[plugins] per_channel S=200 decompress", flush=True)
    assert np.array_equal(q.decompress(c), z["decompressed"][None])
    assert np.array_equal(q.decompress(cu), z["decompressed"][None])


def test_per_channel_round_trip_batch_against_oracle():
    print("[plugins] per_channel B=2 S=256 round trip", flush=True)
    PL = _pl()
    k, _, _ = O.synthetic_kv(77, 2, 2, 2, 256)            # (B, H, S, D) fp16
    q = PL.create("per_channel", n_heads=2, nf4_asym=True, outlier_frac=0.02)
    c = q.compress(k.astype(np.float32), packed=True)
    dec = q.decompress(c)
    HSD = 2 * 256 * 128
    for b in range(2):
        g = O.encode_keys(k[b].astype(np.float32), 0.02)
        assert np.array_equal(c.indices[b * HSD // 2:(b + 1) * HSD // 2], g.packed)
        assert np.array_equal(c.nf4_scale[b], g.nf4_scale) and np.array_equal(c.nf4_mean[b], g.nf4_mean)
        m = (c.outlier_idx // HSD) == b
        assert np.array_equal(c.outlier_idx[m] - b * HSD, g.outlier_idx)
        assert np.array_equal(c.outlier_val[m].view(np.uint16), g.outlier_val.view(np.uint16))
        assert np.array_equal(dec[b], O.decode_keys(g))
    # without a side-list
    q0 = PL.create("per_channel", n_heads=2, nf4_asym=True)
    c0 = q0.compress(k.astype(np.float32))
    assert c0.outlier_idx is None and c0.outlier_val is None
    g0 = O.encode_keys(k[0].astype(np.float32), 0.0)
    assert np.array_equal(q0.decompress(c0)[0], O.decode_keys(g0))


def test_polar_matches_reference_cache_group():
    print("[plugins] polar V3 group 0 of the reference cache", flush=True)
    PL = _pl()
    z = np.load(os.path.join(GOLD, "cache_k4v3_w512.npz"), allow_pickle=False)
    v = z["v"][:, :256][None].astype(np.float32)             # (1, H, 256, D)
    q = PL.create("polar", n_heads=2, bits=3, seed=0)
    c = q.compress(v, packed=True, kind="value")
    assert c.packed and c.bits == 3 and c.shape == v.shape and c.n_values == v.size
    assert np.array_equal(c.indices, z["g0_vpacked"])
    assert np.array_equal(c.norms[0], z["g0_vnorms"])
    r = np.load(os.path.join(GOLD, "rotation_d128_seed0.npz"), allow_pickle=False)
    cent, _ = O.polar_codebook(3, 128)
    g = O.ValueGroup(codes=None, packed=z["g0_vpacked"], norms=z["g0_vnorms"], bits=3)
    assert np.array_equal(q.decompress(c)[0], O.decode_values(g, cent, r["pi"]))


def test_polar_round_trip_across_groups():
    print("[plugins] polar V4 S=300 round trip", flush=True)
    PL = _pl()
    _, v, _ = O.synthetic_kv(78, 1, 2, 2, 300)
    q = PL.create("polar", n_heads=2, bits=3, value_bits=4, seed=3)
    c = q.compress(v.astype(np.float32), kind="value")
    assert not c.packed and c.indices.shape == v.shape and c.norms.shape == v.shape[:3]
    pi, pi_t = O.rotation(3, 128)
    cent, bnd = O.polar_codebook(4, 128)
    for t0, n in ((0, 256), (256, 44)):
        g = O.encode_values(v[0][:, t0:t0 + n].astype(np.float32), pi_t, bnd, 4)
        assert np.array_equal(c.indices[0][:, t0:t0 + n], g.codes)
        assert np.array_equal(c.norms[0][:, t0:t0 + n], g.norms)
    dec = q.decompress(c)
    g_all = O.encode_values(v[0].astype(np.float32), pi_t, bnd, 4)
    assert np.array_equal(dec[0], O.decode_values(g_all, cent, pi))
    cp = q.compress(v.astype(np.float32), packed=True, kind="value")
    assert np.array_equal(q.decompress(cp), dec)


@pytest.mark.parametrize("tag", ["s256", "s200"])
def test_per_channel_uniform_matches_reference(tag):
    """``create("per_channel", bits=4)`` -- the reference's default, uniform
    mode (turboquant_pro/per_channel_kv.py:303-317) -- on the GPU: the
    container (packed codes, (1, H, 1, D) scale and zero, outliers) and the
    decompress equal the reference's for the same block
    (tests/golden/perchannel_uniform.npz), packed and unpacked."""
    print(f"[plugins] per_channel uniform {tag}", flush=True)
    PL = _pl()
    z = np.load(os.path.join(GOLD, "perchannel_uniform.npz"), allow_pickle=False)
    x = z[f"{tag}_x"][None]
    q = PL.create("per_channel", n_heads=2, bits=4, outlier_frac=0.02)
    c = q.compress(x, packed=True)
    assert c.nf4_scale is None and c.nf4_mean is None and c.scale.shape == (1, 2, 1, 128)
    assert np.array_equal(c.indices, z[f"{tag}_kpacked"])
    assert np.array_equal(c.scale[0, :, 0], z[f"{tag}_scale"]) and np.array_equal(c.zero[0, :, 0], z[f"{tag}_zero"])
    assert np.array_equal(c.outlier_idx, z[f"{tag}_oidx"])
    assert np.array_equal(c.outlier_val.view(np.uint16), z[f"{tag}_oval"].view(np.uint16))
    assert np.array_equal(q.decompress(c), z[f"{tag}_decompressed"][None])
    cu = q.compress(x)
    assert np.array_equal(q.decompress(cu), z[f"{tag}_decompressed"][None])
    mu, w, grid = PL.affine_params(q, c)
    assert np.array_equal(grid, np.arange(16, dtype=np.float32)) and np.array_equal(mu, z[f"{tag}_zero"])


def test_polar_unseeded_rotation_is_the_instances():
    """``create("polar")`` with no seed (the reference's default,
    turboquant_pro/core.py:178-228) draws one random rotation per instance:
    compress and decompress of that instance -- across two groups -- equal
    the oracle under ``q.rotation``."""
    print("[plugins] polar seed=None", flush=True)
    PL = _pl()
    _, v, _ = O.synthetic_kv(79, 1, 2, 2, 300)
    q = PL.create("polar", n_heads=2, bits=3)
    assert q.seed is None
    pi, pi_t = q.rotation
    cent, bnd = O.polar_codebook(3, 128)
    c = q.compress(v.astype(np.float32), packed=True, kind="value")
    g = O.encode_values(v[0].astype(np.float32), pi_t, bnd, 3)
    assert np.array_equal(c.norms[0], g.norms)
    assert np.array_equal(q.decompress(c)[0], O.decode_values(g, cent, pi))


def test_per_channel_uniform_without_outliers():
    """``create("per_channel")`` with no arguments -- the reference's default:
    uniform 4-bit keys, ``outlier_frac=0`` (turboquant_pro/per_channel_kv.py:
    183-200,303-317) -- on the GPU equals the oracle's uniform encode (pinned
    to the reference's uniform vectors) and its decode, with no side-list."""
    print("[plugins] per_channel default (uniform, no outliers)", flush=True)
    PL = _pl()
    z = np.load(os.path.join(GOLD, "perchannel_uniform.npz"), allow_pickle=False)
    for tag in ("s256", "s200"):
        x = z[f"{tag}_x"]
        q = PL.create("per_channel", n_heads=2)
        c = q.compress(x[None], packed=True)
        g = O.encode_keys_uniform(x, 0.0)
        assert c.outlier_idx is None and g.outlier_idx is None
        assert np.array_equal(c.indices.reshape(-1), g.packed.reshape(-1))
        assert np.array_equal(c.scale[0, :, 0], g.nf4_scale) and np.array_equal(c.zero[0, :, 0], g.nf4_mean)
        assert np.array_equal(q.decompress(c)[0], O.decode_keys(g))
