"""Non-finite inputs through the GPU group encode, bit for bit against the
oracle, which evaluates the reference's NumPy expressions and so inherits
NumPy's NaN and inf behaviour (turboquant_pro/per_channel_kv.py:269-401,
turboquant_pro/core.py:542-617):

* a NaN key makes its channel's mean, amax and every level NaN, and every
  code of the channel 0 (``argmin`` returns the first NaN);
* +inf and -inf in one channel make its mean NaN (inf - inf);
* an inf magnitude is the largest non-NaN one in the outlier threshold
  search (``np.partition``), NaN patterns order above it, and the side-list's
  test ``|x| >= t`` is false for a NaN magnitude or a NaN threshold;
* a NaN value makes its token's norm NaN, every rotated coordinate NaN, and
  every code 2^vb - 1 (``searchsorted`` places NaN after all boundaries).
"""

import numpy as np
import pytest

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _bits(a, dt):
    return np.ascontiguousarray(a).view(dt)


@pytest.mark.parametrize("W,frac", [(64, 0.02), (64, 0.1), (512, 0.02)], ids=["w64", "w64-10pct", "w512"])
def test_nonfinite_encode_matches_oracle(W, frac):
    from turboquant_pro_amd import TQKVPool
    print(f"[nonfinite] W={W} outlier_frac={frac}", flush=True)
    H = 2
    L = W + 1 + 4 * ((W + 1) // 2)            # five coded groups
    k, v, _ = O.synthetic_kv(77, 1, H, H, L)
    G = (W + 1) // 2
    nan, inf = np.float16(np.nan), np.float16(np.inf)
    k[0, 0, 5, 10] = nan                      # group 0: a NaN channel
    k[0, 1, G + 8, 3] = inf                   # group 1: an inf magnitude ...
    k[0, 1, G + 9, 3] = inf                   # ... tied with another
    k[0, 0, 2 * G + 1, 20] = -inf             # group 2: mean inf - inf = NaN
    k[0, 0, 2 * G + 2, 20] = inf
    k[0, 1, 3 * G + 4, 50] = nan              # group 3: NaN patterns above every magnitude
    k[0, 1, 3 * G + 6, 50] = nan
    k[0, 0, 4 * G + 3, 77] = -inf             # group 4: a -inf magnitude
    v[0, 0, 7, 2] = nan                       # a NaN value token in group 0
    v[0, 1, 3 * G + 1, 100] = nan             # and one in group 3
    pool = TQKVPool(n_kv_heads=H, max_batch=1, max_seq_len=L, hot_window=W, key_bits=4,
                    value_bits=3, outlier_frac=frac, seed=0)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    pi, pi_t = O.rotation(0, 128)
    seq = O.SequenceCache(hot_window=W, value_bits=3, outlier_frac=frac).build(k[0], v[0], pi, pi_t)
    assert pool.n_groups(0) == len(seq.keys) == 5
    for g in range(5):
        e, kg, vg = pool.export_group(0, g), seq.keys[g], seq.values[g]
        what = f"group {g}"
        assert np.array_equal(e["kpacked"], kg.packed), f"{what}: key codes"
        assert np.array_equal(_bits(e["nf4_scale"], np.uint32), _bits(kg.nf4_scale, np.uint32)), f"{what}: amax"
        assert np.array_equal(_bits(e["nf4_mean"], np.uint32), _bits(kg.nf4_mean, np.uint32)), f"{what}: mean"
        assert np.array_equal(e["outlier_idx"], kg.outlier_idx), f"{what}: outlier positions"
        assert np.array_equal(_bits(e["outlier_val"], np.uint16), _bits(kg.outlier_val, np.uint16))
        assert np.array_equal(e["vpacked"], vg.packed), f"{what}: value codes"
        assert np.array_equal(_bits(e["vnorms"], np.uint32), _bits(vg.norms, np.uint32)), f"{what}: norms"
    # the planted cases did what the docstring says
    g0 = seq.keys[0]
    assert np.isnan(g0.nf4_mean[0, 10]) and not g0.codes[0, :, 10].any()
    assert np.isnan(seq.keys[2].nf4_mean[0, 20])
    assert np.isnan(seq.values[0].norms[0, 7]) and np.all(seq.values[0].codes[0, 7] == 7)
    if frac == 0.02:
        # k = 1 for G = 32: the NaN patterns are the top of channel 50, the
        # threshold is NaN and no entry of that channel is kept
        ch50 = (seq.keys[3].outlier_idx % 128 == 50) & (seq.keys[3].outlier_idx // (G * 128) == 1)
        assert W != 64 or not ch50.any()
