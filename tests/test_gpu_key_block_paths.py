"""The key-block encode's two outlier-threshold paths agree.

With ``outlier_cap`` of at least head_dim, ``tqk_encode_key_block`` finds the
thresholds in ``tqk_key_block_thresholds`` (a lane per channel, waves over
the tokens, two magnitude bits a pass) and hands them to ``tqk_key_block``
through the side-list row; with a smaller cap ``tqk_key_block`` searches one
bit a pass in one thread per channel.  Both find the threshold of
turboquant_pro/per_channel_kv.py:274-280 (np.partition's k-th largest
magnitude, every magnitude at or above it an entry).  The same block must
give the same codes, scale, zero point and side-list count both ways, the
small cap's entries being the first ones of the large cap's: fp16 and fp32
input, asym-NF4 and uniform 4-bit keys, lognormal channel scales, magnitude
ties at the threshold and a NaN.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _encode(x, uniform, k, cap):
    from turboquant_pro_amd import _native as N
    from turboquant_pro_amd.plugins import _block_desc
    B, H, S, D = x.shape
    dev = x.device
    kp = torch.zeros(B * H * S * D // 2, dtype=torch.uint8, device=dev)
    scale = torch.zeros((B, H, D), dtype=torch.float32, device=dev)
    zero = torch.zeros_like(scale)
    count = torch.zeros(B * H, dtype=torch.int32, device=dev)
    pos = torch.zeros((B * H, cap), dtype=torch.int32, device=dev)
    val = torch.zeros((B * H, cap), dtype=torch.float16, device=dev)
    d = _block_desc(x.shape, 4, int(uniform), 0, k, cap, int(x.dtype == torch.float32), None)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    N.check(N.lib().tqk_encode_key_block(ctypes.byref(d), x.data_ptr(), None, kp.data_ptr(),
                                         scale.data_ptr(), zero.data_ptr(), pos.data_ptr(),
                                         val.data_ptr(), count.data_ptr(), st), "tqk_encode_key_block")
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (kp, scale, zero, count, pos, val)]


@pytest.mark.parametrize("dtype", ["float16", "float32"])
@pytest.mark.parametrize("uniform", [False, True], ids=["nf4_asym", "uniform4"])
@pytest.mark.parametrize("S", [300, 1000])
def test_threshold_paths_agree(dtype, uniform, S):
    from turboquant_pro_amd.codebooks import outliers_per_channel
    B, H, D = 1, 2, 128
    print(f"[key-block] threshold paths dtype={dtype} uniform={uniform} S={S}", flush=True)
    rng = np.random.default_rng(S + 7 * uniform)
    x = rng.standard_normal((B, H, S, D)).astype(np.float32)
    x *= np.exp(0.7 * rng.standard_normal((1, H, 1, D))).astype(np.float32)
    x[0, 0, :, 5] = 0.1 * rng.standard_normal(S)
    x[0, 0, : S // 4, 5] = 3.0          # the channel's largest magnitude, S / 2 times,
    x[0, 0, S // 4: S // 2, 5] = -3.0   # of both signs: ties at its threshold
    x[0, 1, 17, 9] = np.nan             # a NaN orders above every magnitude
    xt = torch.from_numpy(x).to(getattr(torch, dtype)).cuda()
    k = outliers_per_channel(S, 0.02)
    big = _encode(xt, uniform, k, 4 * k * D)   # thresholds over the chip
    small = _encode(xt, uniform, k, D // 2)    # one thread per channel
    for name, a, b in zip(("codes", "scale", "zero", "count"), big[:4], small[:4]):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name
    cnt = big[3]
    assert cnt[0] >= (D - 1) * k + S // 2   # the ties keep every equal magnitude
    for i in range(B * H):
        n = min(int(cnt[i]), D // 2)
        assert np.array_equal(big[4][i, :n], small[4][i, :n]), f"positions of (b, h) {i}"
        assert np.array_equal(big[5][i, :n].view(np.uint16), small[5][i, :n].view(np.uint16)), \
            f"values of (b, h) {i}"
