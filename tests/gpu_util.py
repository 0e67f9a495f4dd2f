"""Helpers shared by the GPU parity tests (imported by test modules only)."""

import numpy as np

from oracle import tq_oracle as O

ATOL = 2e-3    # max-abs tolerance on attention outputs
RTOL = 1e-2    # relative tolerance: ||got - want|| / ||want||


def assert_attn_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert err.max() <= atol, f"{what} max-abs {err.max():.3e} > {atol}"
    assert rel <= rtol, f"{what} rel {rel:.3e} > {rtol}"
    return float(err.max()), float(rel)


def oracle_state(k, v, hot_window, vbits, seed, outlier_frac=0.02):
    """Per-sequence oracle caches for fp16 k, v (B, Hkv, L, D)."""
    D = k.shape[-1]
    pi, pi_t = O.rotation(seed, D)
    return [O.SequenceCache(hot_window=hot_window, value_bits=vbits, outlier_frac=outlier_frac)
            .build(k[b], v[b], pi, pi_t) for b in range(k.shape[0])], (pi, pi_t)


def compare_group(exp, kg, vg, what=""):
    """Exported GPU group vs oracle KeyGroup/ValueGroup, bit for bit."""
    assert np.array_equal(exp["kpacked"], kg.packed), f"{what}: key codes differ"
    assert np.array_equal(exp["nf4_scale"], kg.nf4_scale), f"{what}: nf4_scale differs"
    assert np.array_equal(exp["nf4_mean"], kg.nf4_mean), f"{what}: nf4_mean differs"
    assert np.array_equal(exp["outlier_idx"], kg.outlier_idx), f"{what}: outlier idx differ"
    assert np.array_equal(exp["outlier_val"].view(np.uint16), kg.outlier_val.view(np.uint16)), \
        f"{what}: outlier values differ"
    assert np.array_equal(exp["vpacked"], vg.packed), f"{what}: value codes differ"
    assert np.array_equal(exp["vnorms"], vg.norms), f"{what}: value norms differ"
