"""tqk_decode_noalloc (the decode that allocates nothing: split partials and
arrival counters in the library's device scratch array) against tqk_decode
with a caller workspace, through the C ABI, on consecutive calls of shrinking
size that share the scratch."""

import ctypes

import numpy as np
import pytest

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu


def _pool_with(torch, B, Hkv, Hq, lens, hot_window=512, seed=0):
    from turboquant_pro_amd import TQKVPool
    L = max(lens)
    k, v, q = O.synthetic_kv(seed, B, Hkv, Hq, L)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, hot_window=hot_window,
                    seed=seed)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), n_new=lens)
    return pool, torch.from_numpy(q).cuda()


def _both(torch, pool, q):
    """(tqk_decode output, tqk_decode_noalloc output) for one step."""
    from turboquant_pro_amd import _native as N
    lib = N.lib()
    B = pool.max_batch
    ref = pool.decode(q).cpu().numpy()
    out = torch.full((B, pool.n_q_heads, pool.head_dim), float("nan"), dtype=torch.float32,
                     device=pool.device)
    N.check(lib.tqk_decode_noalloc(ctypes.byref(pool.desc), ctypes.byref(pool.ptrs), B,
                                   q.contiguous().data_ptr(), pool.seq_lens.data_ptr(),
                                   max(pool.lengths), out.data_ptr(), pool._stream()),
            "tqk_decode_noalloc")
    torch.cuda.synchronize()
    return ref, out.cpu().numpy()


def test_noalloc_matches_workspace_decode_on_shrinking_calls():
    import torch
    cases = [
        # (B, Hkv, Hq, lengths, hot_window): MFMA kernel with its in-kernel merge
        (4, 2, 8, [3100, 1800, 2600, 700], 512),
        # a smaller call right after: fewer sequences and splits
        (2, 2, 8, [1300, 900], 512),
        # the VALU kernel + separate merge (groups not whole 32-token blocks)
        (2, 2, 4, [150, 90], 16),
    ]
    for i, (B, Hkv, Hq, lens, W) in enumerate(cases):
        print(f"[noalloc] call {i}: B={B} Hkv={Hkv} Hq={Hq} lens={lens} W={W}", flush=True)
        pool, q = _pool_with(torch, B, Hkv, Hq, lens, hot_window=W, seed=10 + i)
        ref, got = _both(torch, pool, q)
        assert np.isfinite(got).all()
        # both decode kernels are deterministic: the same kernels over the
        # same data give identical outputs
        assert np.array_equal(ref, got), f"call {i}: max diff {np.abs(ref - got).max():.3e}"
