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


@pytest.mark.parametrize("bits,D", [(3, 128), (4, 128), (3, 64), (2, 64), (3, 256), (4, 256)])
def test_values_c_equals_numpy(clib, bits, D):
    _, v, _ = O.synthetic_kv(5, 1, 2, 2, 256, D=D)
    x = v[0].astype(np.float32)
    pi, pi_t = O.rotation(0, D)
    cent, bnd = O.polar_codebook(bits, D)
    want = O.encode_values(x, pi_t, bnd, bits)
    rows = np.ascontiguousarray(x.reshape(-1, D))
    codes = np.zeros(rows.shape, np.uint8)
    norms = np.zeros(rows.shape[0], np.float32)
    clib.tqo_encode_values(_p(rows), rows.shape[0], D, _p(pi_t), _p(bnd), bnd.size,
                           _p(codes), _p(norms))
    assert np.array_equal(norms, want.norms.reshape(-1))
    assert np.array_equal(codes, want.codes.reshape(-1, D))


@pytest.mark.parametrize("D", [64, 256])
def test_keys_c_equals_numpy_head_dims(clib, D):
    k, _, _ = O.synthetic_kv(11, 1, 2, 2, 256, D=D)
    x = k[0].astype(np.float32)
    want = O.encode_keys(x, 0.02)
    codes, scale, mean, oidx = _c_keys(clib, x, O.outlier_count_per_channel(256, 0.02))
    assert np.array_equal(scale, want.nf4_scale) and np.array_equal(mean, want.nf4_mean)
    assert np.array_equal(codes, want.codes) and np.array_equal(oidx, want.outlier_idx)


def _blocked8(sq):
    """Eight strided accumulators over the whole row, one tree: NumPy's order
    for rows of at most 128 values only."""
    r = sq[:, :8].copy()
    for i in range(8, sq.shape[1], 8):
        r = r + sq[:, i:i + 8]
    return ((r[:, 0] + r[:, 1]) + (r[:, 2] + r[:, 3])) + ((r[:, 4] + r[:, 5]) + (r[:, 6] + r[:, 7]))


def test_norm_split_at_256_is_pinned():
    """At D = 256 NumPy sums the two 128-channel halves apart: one 8-way
    block over all 256 values differs from np.linalg.norm's sum on some rows,
    so the half split the C oracle (and the kernels) use is what the bit-exact
    norm tests above pin."""
    rows = np.random.default_rng(3).standard_normal((4096, 256)).astype(np.float32) * 3
    sq = rows * rows
    ref = np.add.reduce(sq, axis=-1)
    halves = _blocked8(sq[:, :128]) + _blocked8(sq[:, 128:])
    assert np.array_equal(halves, ref)
    assert np.count_nonzero(_blocked8(sq) != ref) > 0


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
