"""The in-kernel merge of ``tqk_decode`` against the separate merge kernel.

``tqk_decode`` lets the last of a (sequence, kv head)'s split workgroups
combine the partials (flash-combine of turboquant_pro/kv_kernel.py:377-381,
merge_partials of turboquant_pro/kv_fused.py:139-153) and rotate the coded
part back.  ``tqk_decode_splits`` + ``tqk_decode_merge`` compute the same
partials and combine them in ``tqk_merge``.  Both run the same arithmetic in
the same order, so the outputs agree bit for bit; the arrival counters
return to zero after every call, so call after call agrees too, also when
a longer cache changes the number of splits.  The output is also checked
against dequantize-then-attend.
"""

import ctypes

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


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _two_phase(pool, q):
    """tqk_decode_splits then tqk_decode_merge on the pool's own workspace."""
    from turboquant_pro_amd import _native as N
    lib = N.lib()
    B, max_len = pool.max_batch, max(pool.lengths)
    out = torch.empty((B, pool.n_q_heads, pool.head_dim), dtype=torch.float32, device=q.device)
    ws, need = pool.workspace(B, max_len)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    N.check(lib.tqk_decode_splits(ctypes.byref(pool.desc), ctypes.byref(pool.ptrs), B, q.data_ptr(),
                                  pool.seq_lens.data_ptr(), max_len, ws.data_ptr(), need, st),
            "tqk_decode_splits")
    N.check(lib.tqk_decode_merge(ctypes.byref(pool.desc), ctypes.byref(pool.ptrs), B, max_len,
                                 out.data_ptr(), ws.data_ptr(), need, st), "tqk_decode_merge")
    return out


@pytest.mark.parametrize("gq,vbits", [(4, 3), (8, 4), (1, 3)])
def test_in_kernel_merge_equals_merge_kernel(gq, vbits):
    from turboquant_pro_amd import TQKVPool
    B, Hkv = 3, 2
    Hq = Hkv * gq
    L1, L2 = 4700, 9100           # 3 coded splits per (seq, kv head), then more
    lens1 = [L1, 2600, 700]
    print(f"[merge] gq={gq} vbits={vbits} lens={lens1} then +{L2 - L1}", flush=True)
    k, v, q = O.synthetic_kv(90 + gq, B, Hkv, Hq, L2)
    pi, pi_t = O.rotation(5, 128)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L2, value_bits=vbits,
                    rotation=(pi, pi_t))
    pool.append(_dev(k[:, :, :L1]), _dev(v[:, :, :L1]), n_new=lens1)
    qd = _dev(q)
    fused = [pool.decode(qd) for _ in range(3)]
    ref = _two_phase(pool, qd)
    torch.cuda.synchronize()
    for i, f in enumerate(fused):
        assert torch.equal(f, ref), f"call {i}: in-kernel merge differs from tqk_merge"
    got = fused[0].cpu().numpy()
    for b, L in enumerate(lens1):
        sc = O.SequenceCache(hot_window=512, value_bits=vbits, outlier_frac=0.02).build(
            k[b, :, :L], v[b, :, :L], pi, pi_t)
        assert_attn_close(got[b], sc.attend(q[b]), what=f"seq {b} L={L}")
    # a longer cache: more groups per sequence, another split plan
    print("[merge] after appending", flush=True)
    lens2 = [L2 - L1, 3000, 0]
    pool.append(_dev(k[:, :, L1:]), _dev(v[:, :, L1:]), n_new=lens2)
    f2 = pool.decode(qd)
    r2 = _two_phase(pool, qd)
    f3 = pool.decode(qd)
    torch.cuda.synchronize()
    assert torch.equal(f2, r2) and torch.equal(f3, r2)


def test_in_kernel_merge_many_splits():
    """A long single sequence over two kv heads: the planner gives each kv head
    dozens of short coded splits (77 groups, few (seq, kv head) pairs for 256
    CUs), so both merges take their chunked form over several rounds of 16
    partials (the in-kernel one skipping the hot partials past the hot
    window's blocks); still bit for bit equal, and within the bar of
    dequantize-then-attend."""
    from turboquant_pro_amd import TQKVPool
    B, Hkv, Hq, L = 1, 2, 8, 20000
    print(f"[merge] long context L={L}", flush=True)
    k, v, q = O.synthetic_kv(97, B, Hkv, Hq, L)
    pi, pi_t = O.rotation(6, 128)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, rotation=(pi, pi_t))
    pool.append(_dev(k), _dev(v))
    qd = _dev(q)
    fused = [pool.decode(qd) for _ in range(2)]
    ref = _two_phase(pool, qd)
    torch.cuda.synchronize()
    assert all(torch.equal(f, ref) for f in fused)
    sc = O.SequenceCache(hot_window=512, value_bits=3, outlier_frac=0.02).build(k[0], v[0], pi, pi_t)
    assert_attn_close(fused[0][0].cpu().numpy(), sc.attend(q[0]), what="L=20000")


def test_in_kernel_merge_after_the_plan_shrinks():
    """The pool keeps its workspace when a later decode needs fewer splits
    (a shorter cache after ``reset``): the arrival counters must not sit where
    the earlier, larger plan wrote partials."""
    from turboquant_pro_amd import TQKVPool
    B, Hkv, Hq = 2, 2, 8
    print("[merge] plan shrinks: L=9000 then L=1500 on the same workspace", flush=True)
    k, v, q = O.synthetic_kv(98, B, Hkv, Hq, 9000)
    pi, pi_t = O.rotation(7, 128)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=9000, rotation=(pi, pi_t))
    qd = _dev(q)
    pool.append(_dev(k), _dev(v))
    big = pool.decode(qd)
    torch.cuda.synchronize()
    assert torch.equal(big, _two_phase(pool, qd))
    pool.reset()
    pool.append(_dev(k[:, :, :1500]), _dev(v[:, :, :1500]))
    small = [pool.decode(qd) for _ in range(2)]
    ref = _two_phase(pool, qd)
    torch.cuda.synchronize()
    assert all(torch.equal(s, ref) for s in small)
    for b in range(B):
        sc = O.SequenceCache(hot_window=512, value_bits=3, outlier_frac=0.02).build(
            k[b, :, :1500], v[b, :, :1500], pi, pi_t)
        assert_attn_close(small[0][b].cpu().numpy(), sc.attend(q[b]), what=f"seq {b}")
