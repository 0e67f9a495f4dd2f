"""Decode numerics at the edges of the kernel's fp16 operands and of its lazy
running max, against the oracle's dequantize-then-attend:

* value norms up to 16000, just inside the 16376 the decode carries (softmax
  weights stay <= 4, and weight * norm is an fp16 hi/lo pair, largest 65504);
* queries scaled 20x and 0.01x: near one-hot attention, where the running
  max is exceeded and the accumulators rescaled again and again, and nearly
  uniform attention, where it never is.
"""

import numpy as np
import pytest

from gpu_util import assert_attn_close
from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _decode_vs_oracle(k, v, q, W, what):
    from turboquant_pro_amd import TQKVPool
    B, Hkv, L, _ = k.shape
    Hq = q.shape[1]
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, hot_window=W, seed=0)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    pool.check()
    got = pool.decode(torch.from_numpy(q).cuda()).cpu().numpy()
    pi, pi_t = O.rotation(0, 128)
    for b in range(B):
        sc = O.SequenceCache(hot_window=W, value_bits=3, outlier_frac=0.02).build(k[b], v[b], pi, pi_t)
        want = sc.attend(q[b])
        assert np.isfinite(got[b]).all(), what
        # the bar is 2e-3 of the output's largest magnitude; the absolute
        # error is printed beside it (run with -s to see it)
        scale = float(np.abs(want).max())
        print(f"[numerics] {what} seq {b}: max |out| {scale:.4g}, max abs err "
              f"{float(np.abs(got[b] - want).max()):.4g}", flush=True)
        assert_attn_close(got[b] / scale, want / scale, what=f"{what} seq {b}")


@pytest.mark.parametrize("W", [512, 64])
def test_value_norms_up_to_the_decode_limit(W):
    print(f"[numerics] value norms up to 16000, W={W}", flush=True)
    B, Hkv, Hq, L = 2, 2, 8, 1300
    k, v, q = O.synthetic_kv(91, B, Hkv, Hq, L)
    rng = np.random.default_rng(3)
    v = v.astype(np.float32)
    # every 7th token of every head scaled to a norm in [8000, 16000]
    nrm = np.linalg.norm(v, axis=-1, keepdims=True)
    target = rng.uniform(8000.0, 16000.0, size=nrm.shape).astype(np.float32)
    sel = (np.arange(L) % 7 == 0)[None, None, :, None]
    v = np.where(sel, v / nrm * target, v)
    assert float(np.linalg.norm(v.astype(np.float16).astype(np.float32), axis=-1).max()) < 16376
    _decode_vs_oracle(k, v.astype(np.float16), q, W, f"large norms W={W}")


@pytest.mark.parametrize("scale", [20.0, 0.01], ids=["sharp", "flat"])
def test_query_scale_extremes(scale):
    print(f"[numerics] query scale {scale}", flush=True)
    B, Hkv, Hq, L = 2, 2, 8, 1300
    k, v, q = O.synthetic_kv(92, B, Hkv, Hq, L)
    q = (q.astype(np.float32) * scale).astype(np.float16)
    _decode_vs_oracle(k, v, q, 512, f"query x{scale}")
