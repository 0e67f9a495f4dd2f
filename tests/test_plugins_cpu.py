"""Plugin surface on the CPU: the registry's behaviour
(turboquant_pro/plugins.py:60-200), constructor validation and the
no-gfx950-form signal, and the affine capability of the "per_channel" format
(turboquant_pro/kv_fused_pck.py:47-127) on a container holding the
reference's own bytes (tests/golden/perchannel_s200.npz, written by
``PerChannelKV.compress``), checked against the oracle's unpack and decode
and against the overlay identity: dense dequant + CSR deltas = the
outlier-overwritten dequant (turboquant_pro tests/test_kv_fused_pck.py:159-176)."""

import os

import numpy as np
import pytest

from oracle import tq_oracle as O
from turboquant_pro_amd import plugins as PL

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _s200_container():
    z = np.load(os.path.join(GOLD, "perchannel_s200.npz"), allow_pickle=False)
    H, S, D = z["x"].shape
    c = PL.CompressedPerChannelKV(
        z["kpacked"], None, None, 4, (1, H, S, D), True,
        nf4_scale=z["nf4_scale"][None], nf4_mean=z["nf4_mean"][None],
        outlier_idx=z["oidx"], outlier_val=z["oval"])
    return z, c


def test_registry_lists_in_tree_formats():
    names = PL.available_plugins()
    assert {"per_channel", "polar"} <= set(names)
    assert set(PL.available_plugins(target=PL.TARGET_KV_KEY)) >= {"per_channel"}
    assert "per_channel" not in PL.available_plugins(target=PL.TARGET_KV_VALUE)
    assert "polar" in PL.available_plugins(target=PL.TARGET_KV_VALUE)
    assert PL.get_plugin("polar").tier == "stable"


def test_registry_errors():
    with pytest.raises(KeyError, match="no quantizer plugin"):
        PL.get_plugin("does_not_exist")
    spec = PL.get_plugin("per_channel")
    with pytest.raises(ValueError, match="already registered"):
        PL.register(spec)
    PL.register(spec, overwrite=True)
    for bad in (dict(name="", factory=dict, targets=frozenset()),
                dict(name="a/b", factory=dict, targets=frozenset()),
                dict(name="x", factory=dict, targets=frozenset({"nope"})),
                dict(name="x", factory=dict, targets=frozenset(), tier="gold")):
        with pytest.raises(ValueError):
            PL.PluginSpec(**bad)
    PL.register(PL.PluginSpec(name="not_a_quantizer", factory=lambda **kw: object(),
                              targets=frozenset({PL.TARGET_WEIGHT})), overwrite=True)
    with pytest.raises(TypeError, match="compress/decompress"):
        PL.create("not_a_quantizer")


def test_per_channel_constructor_validation():
    ok = PL.create("per_channel", nf4_asym=True, outlier_frac=0.02)
    assert isinstance(ok, PL.Quantizer) and PL.native_dtype(ok) is None
    for cfg in (dict(bits=5), dict(nf4=True, bits=3), dict(outlier_frac=1.0),
                dict(zero_point="nope"), dict(zero_point="sparse", rope_theta=1e4),
                dict(nf4_asym=True, zero_point="sparse"),
                dict(nf4_asym=True, zero_point="bias", rope_theta=1e4)):
        with pytest.raises(ValueError):
            PL.create("per_channel", **cfg)
    # valid reference configurations without a gfx950 encode
    uni = PL.create("per_channel", bits=4, outlier_frac=0.02)      # the reference's default mode
    assert uni.uniform and uni.key_grid == "uniform"
    for cfg in (dict(nuq=True), dict(nf4_asym=True, head_dim=96)):
        with pytest.raises(NotImplementedError):
            PL.create("per_channel", **cfg)
    for D in (64, 256):                                               # head dims of the kernels
        assert PL.create("per_channel", nf4_asym=True, head_dim=D).head_dim == D
    sym = PL.create("per_channel", nf4=True)                         # symmetric NF4
    assert sym.symmetric and sym.key_grid == "nf4_asym" and not sym.uniform
    for b in (2, 3):                                                  # uniform 3- and 2-bit keys
        low = PL.create("per_channel", bits=b, outlier_frac=0.02)
        assert low.uniform and low.bits == b
    # every asym-NF4 zero point has a gfx950 encode
    sp = PL.create("per_channel", nf4_asym=True, zero_point="sparse", rope_theta=1e4)
    bi = PL.create("per_channel", nf4_asym=True, zero_point="bias", rope_theta=1e6,
                   k_bias=np.ones((32, 128), np.float32), n_heads=32)
    assert sp.zero_point == "sparse" and bi.k_bias.shape == (32, 128)


def test_polar_constructor_validation():
    q = PL.create("polar", bits=3, seed=0)
    with pytest.raises(ValueError):
        PL.create("polar", bits=5)
    with pytest.raises(ValueError):
        PL.create("polar", value_bits=1)
    with pytest.raises(NotImplementedError):
        PL.create("polar", head_dim=96)
    # widths per kind, as TurboQuantKV._resolve_bits (turboquant_pro/core.py:528-540)
    kv = PL.create("polar", bits=3, key_bits=4, value_bits=2, seed=0)
    assert (kv._width(None), kv._width("key"), kv._width("value")) == (3, 4, 2)
    with pytest.raises(ValueError):
        kv._width("query")
    assert PL.affine_params(q, None) is None and PL.outlier_csr(q, None) is None


def test_affine_codes_and_grid_on_reference_container():
    z, c = _s200_container()
    q = PL.create("per_channel", nf4_asym=True, outlier_frac=0.02)
    H, S, D = z["x"].shape
    codes = PL.affine_codes(q, c)
    assert codes.shape == (1, H, S, D) and codes.dtype == np.uint8
    assert np.array_equal(codes.reshape(-1), O.unpack_key_codes(z["kpacked"], H * S * D, 4))
    mu, w, grid = PL.affine_params(q, c)
    assert np.array_equal(mu, z["nf4_mean"]) and np.array_equal(w, z["nf4_scale"])
    assert np.array_equal(grid, O.NF4.astype(np.float32))
    # the unpacked container gives the same codes
    c2 = PL.CompressedPerChannelKV(codes, None, None, 4, c.shape, False, nf4_scale=c.nf4_scale,
                                   nf4_mean=c.nf4_mean)
    assert np.array_equal(q.codes(c2), codes)


def test_outlier_csr_overlay_identity():
    z, c = _s200_container()
    q = PL.create("per_channel", nf4_asym=True, outlier_frac=0.02)
    H, S, D = z["x"].shape
    row_ptr, cols, deltas = PL.outlier_csr(q, c)
    nnz = z["oidx"].size
    assert row_ptr.shape == (H * S + 1,) and row_ptr[0] == 0 and row_ptr[-1] == nnz
    assert np.all(np.diff(row_ptr) >= 0) and cols.dtype == np.uint16 and deltas.dtype == np.float32
    # dense dequant without the overlay, plus the deltas at (row, col), is the
    # overwritten dequant the reference returns (to fp32 rounding of the add)
    mu, w, grid = q.grid_params(c)
    codes = q.codes(c)[0]
    dense = (mu[:, None, :] + w[:, None, :] * grid[codes]).astype(np.float32)
    applied = dense.copy().reshape(H * S, D)
    for r in range(H * S):
        for e in range(row_ptr[r], row_ptr[r + 1]):
            applied[r, cols[e]] += deltas[e]
    applied = applied.reshape(H, S, D)
    ref = z["decompressed"]
    assert np.allclose(applied, ref, rtol=0, atol=1e-5 * np.abs(ref).max())
    changed = np.argwhere(applied != dense)
    assert changed.shape[0] <= nnz
    # every overlay position carries its fp16 value
    flat = z["oidx"].astype(np.int64)
    h, s, j = flat // (S * D), (flat // D) % S, flat % D
    assert np.allclose(applied[h, s, j], z["oval"].astype(np.float32), rtol=1e-6, atol=0)
    # no outliers -> no CSR
    c.outlier_idx = None
    assert PL.outlier_csr(q, c) is None
