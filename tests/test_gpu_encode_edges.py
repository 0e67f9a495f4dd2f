"""Key channels at the edges of the encode's fast paths, bit for bit against
the oracle: in odd groups, channel offsets from 0 to 6e4 (fp16's range) with
noise from 0 to 10, so that channels' NF4 levels are crowded or collapsed
onto one value by rounding (a large mean with a tiny amax) and the group
takes the compare-and-select argmin, constant channels the 1e-8 amax floor;
in even groups every channel's levels are spread far enough apart for the
argmin to be a count of strict distance decreases.  Every group's codes,
scales, means and side-list must equal the oracle's, which runs NumPy's own
argmin."""

import numpy as np
import pytest

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def edge_keys(seed, H, L, G, D=128):
    """Odd groups: channel offsets from 0 to fp16's range with noise from 0
    to 10 (crowded and collapsed levels among them); even groups: offsets
    within a few noise scales (every channel's levels well spread)."""
    rng = np.random.default_rng(seed)
    offsets = np.array([0.0, 0.5, 10.0, 100.0, 1000.0, 2000.0, 3.0e4, 6.0e4, -1000.0, -3.0e4])
    scales = np.array([0.0, 1e-3, 1e-2, 0.1, 1.0, 10.0])
    k = rng.standard_normal((H, L, D)).astype(np.float32)
    for j in range(D):
        off = offsets[j % len(offsets)]
        sc = scales[(j // len(offsets)) % len(scales)]
        for g in range((L + G - 1) // G):
            sl = slice(g * G, (g + 1) * G)
            if g % 2:
                k[:, sl, j] = off + sc * k[:, sl, j]
            else:
                s2 = 0.05 + j / 16.0
                k[:, sl, j] = s2 * (k[:, sl, j] + (j % 5) - 2)
    return np.clip(k, -65504, 65504).astype(np.float16)


@pytest.mark.parametrize("W", [64, 512])
def test_edge_channels_encode_matches_oracle(W):
    from turboquant_pro_amd import TQKVPool
    print(f"[encode edges] W={W}", flush=True)
    H = 2
    G = (W + 1) // 2
    L = W + 1 + 3 * G
    k = edge_keys(W, H, L, G)
    v = np.random.default_rng(1).standard_normal((H, L, 128)).astype(np.float16)
    # constant channels tie every token at the top: room for whole groups of outliers
    pool = TQKVPool(n_kv_heads=H, max_batch=1, max_seq_len=L, hot_window=W, key_bits=4,
                    value_bits=3, outlier_frac=0.02, seed=0, outlier_cap=G * 128)
    pool.append(torch.from_numpy(k[None]).cuda(), torch.from_numpy(v[None]).cuda())
    pi, pi_t = O.rotation(0, 128)
    seq = O.SequenceCache(hot_window=W, value_bits=3, outlier_frac=0.02).build(k, v, pi, pi_t)
    assert pool.n_groups(0) == len(seq.keys) == 4
    for g, kg in enumerate(seq.keys):
        e = pool.export_group(0, g)
        assert np.array_equal(e["kpacked"], kg.packed), f"group {g} key codes"
        assert np.array_equal(e["nf4_scale"].view(np.uint32), kg.nf4_scale.view(np.uint32))
        assert np.array_equal(e["nf4_mean"].view(np.uint32), kg.nf4_mean.view(np.uint32))
        assert np.array_equal(e["outlier_idx"], kg.outlier_idx)
        # channels whose levels are not spread enough for the counting argmin
        lv = kg.nf4_mean[..., None] + kg.nf4_scale[..., None] * O.NF4.astype(np.float32)
        gaps = np.diff(lv.astype(np.float32), axis=-1).min(axis=-1)
        bound = (np.abs(kg.nf4_mean) + kg.nf4_scale) * np.float32(2.0 ** -18)
        crowded = int((gaps < bound).sum())
        # both argmin paths run: every channel of an even group is spread
        # (the counting argmin), odd groups have crowded channels
        assert (crowded == 0) if g % 2 == 0 else (crowded > 0), (g, crowded)
