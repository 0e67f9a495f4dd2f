"""The scalar C restatement (oracle/tqk_oracle.c) reproduces the NumPy oracle
bit for bit.  This pins the floating-point operation order -- sequential
channel mean, 8-lane pairwise norm, sequential non-fused rotation, first-index
argmin, ">= k-th largest" outliers -- that the gfx950 encode kernel follows.
"""

import ctypes
import os
import subprocess

import numpy as np
import pytest

from oracle import tq_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "_build", "libtqk_oracle.so")


@pytest.fixture(scope="module")
def clib():
    if not os.path.exists(LIB):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True,
                       stdout=subprocess.DEVNULL)
    lib = ctypes.CDLL(LIB)
    lib.tqo_encode_keys.restype = ctypes.c_int
    return lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c_keys(lib, x, k_out):
    H, S, D = x.shape
    x = np.ascontiguousarray(x, np.float32)
    codes = np.zeros((H, S, D), np.uint8)
    scale = np.zeros((H, D), np.float32)
    mean = np.zeros((H, D), np.float32)
    oidx = np.zeros(H * S * D, np.int32)
    n = lib.tqo_encode_keys(_p(x), H, S, D, k_out, _p(codes), _p(scale), _p(mean), _p(oidx))
    return codes, scale, mean, oidx[:n]


@pytest.mark.parametrize("S,seed", [(256, 0), (256, 1), (8, 2), (200, 3), (32, 4)])
def test_keys_c_equals_numpy(clib, S, seed):
    k, _, _ = O.synthetic_kv(seed, 1, 2, 2, S)
    x = k[0].astype(np.float32)
    want = O.encode_keys(x, 0.02)
    codes, scale, mean, oidx = _c_keys(clib, x, O.outlier_count_per_channel(S, 0.02))
    assert np.array_equal(scale, want.nf4_scale) and np.array_equal(mean, want.nf4_mean)
    assert np.array_equal(codes, want.codes)
    assert np.array_equal(oidx, want.outlier_idx)


def test_keys_c_equals_numpy_with_ties(clib):
    rng = np.random.default_rng(9)
    x = np.round(rng.standard_normal((2, 64, 128)) * 2) / 2
    x[0, :, 3] = 1.5
    x = x.astype(np.float32)
    want = O.encode_keys(x, 0.02)
    codes, scale, mean, oidx = _c_keys(clib, x, O.outlier_count_per_channel(64, 0.02))
    assert np.array_equal(codes, want.codes) and np.array_equal(oidx, want.outlier_idx)


@pytest.mark.parametrize("bits", [3, 4])
def test_values_c_equals_numpy(clib, bits):
    _, v, _ = O.synthetic_kv(5, 1, 2, 2, 256)
    x = v[0].astype(np.float32)
    pi, pi_t = O.rotation(0, 128)
    cent, bnd = O.polar_codebook(bits, 128)
    want = O.encode_values(x, pi_t, bnd, bits)
    rows = np.ascontiguousarray(x.reshape(-1, 128))
    codes = np.zeros(rows.shape, np.uint8)
    norms = np.zeros(rows.shape[0], np.float32)
    clib.tqo_encode_values(_p(rows), rows.shape[0], 128, _p(pi_t), _p(bnd), bnd.size,
                           _p(codes), _p(norms))
    assert np.array_equal(norms, want.norms.reshape(-1))
    assert np.array_equal(codes, want.codes.reshape(-1, 128))


def test_fma_order_would_be_caught(clib):
    """A fused multiply-add rotation differs from NumPy on many elements: the
    bit-exact test above is sensitive to the operation order it pins."""
    _, v, _ = O.synthetic_kv(6, 1, 1, 1, 256)
    x = v[0, 0].astype(np.float32)
    _, pi_t = O.rotation(0, 128)
    u = x / np.linalg.norm(x, axis=-1, keepdims=True)
    seq = np.einsum("sd,de->se", u, pi_t)
    fused = (u.astype(np.float64) @ pi_t.astype(np.float64)).astype(np.float32)
    assert np.count_nonzero(seq != fused) > 0
