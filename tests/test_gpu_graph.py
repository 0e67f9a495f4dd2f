"""tqk_decode captured in a HIP graph, the way serving loops launch their
decode steps: the graph is replayed several times, with eager work and
synchronisations between the replays, and every replay must equal the eager
decode bit for bit (both decode kernels sum in a fixed order, and the
workspace's arrival counters are back at zero after every call).  A new query
written into the captured buffer is seen by the next replay.  Nothing the
decode records is a memset: the workspace is zero-filled once, eagerly."""

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


@pytest.mark.parametrize("W", [512, 16], ids=["mfma", "valu"])
def test_decode_replays_in_a_graph_equal_the_eager_decode(W):
    from turboquant_pro_amd import TQKVPool
    print(f"[graph] hot window {W}", flush=True)
    B, Hkv, Hq, L = 2, 2, 8, (1400 if W == 512 else 90)
    k, v, q = O.synthetic_kv(31, B, Hkv, Hq, L)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, hot_window=W, seed=0)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    qd = torch.from_numpy(q).cuda()
    # eager first: allocates and zero-fills the workspace, reads the CU count,
    # and reads the encode's flags (no host wait may happen under capture)
    eager = pool.decode(qd).clone()
    pool.check()
    torch.cuda.synchronize()

    def same(a, b):
        return torch.equal(a, b)

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = pool.decode(qd)
    for r in range(4):
        # eager work between the replays, on the same pool and workspace
        x = torch.randn((1 << 20,), device="cuda")
        y = (x * 2.0).sum()
        again = pool.decode(qd)
        torch.cuda.synchronize()
        assert same(again, eager) and torch.isfinite(y)
        g.replay()
        torch.cuda.synchronize()
        assert same(out, eager), f"replay {r}"
    # a new query in the captured buffer
    q2 = np.random.default_rng(5).standard_normal(q.shape).astype(np.float16)
    qd.copy_(torch.from_numpy(q2).cuda())
    g.replay()
    torch.cuda.synchronize()
    want = pool.decode(qd)
    torch.cuda.synchronize()
    assert same(out, want)
    pi, pi_t = O.rotation(0, 128)
    for b in range(B):
        sc = O.SequenceCache(hot_window=W, value_bits=3, outlier_frac=0.02).build(k[b], v[b], pi, pi_t)
        assert_attn_close(out[b].cpu().numpy(), sc.attend(q2[b]), what=f"graph W={W} seq {b}")


def test_capture_with_unread_encode_flags_is_refused():
    """An append leaves its encode flags unread (it does not wait for them); a
    decode captured right after it would need a host wait, which capture
    forbids, so the pool raises before launching anything.  After
    ``pool.check()`` the same capture works."""
    from turboquant_pro_amd import TQKVPool
    print("[graph] capture after an unchecked append", flush=True)
    B, Hkv, Hq = 1, 2, 8
    k, v, q = O.synthetic_kv(32, B, Hkv, Hq, 1700)
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=1700, seed=0)
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    pool.append(kd[:, :, :1400], vd[:, :, :1400])
    eager = pool.decode(qd).clone()      # workspace allocated, flags read
    pool.append(kd[:, :, 1400:], vd[:, :, 1400:])   # flushes a group: flags pending
    assert pool._pending
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="pool.check"):
        with torch.cuda.graph(g):
            pool.decode(qd)
    torch.cuda.synchronize()
    pool.check()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        out = pool.decode(qd)
    g2.replay()
    torch.cuda.synchronize()
    want = pool.decode(qd)
    torch.cuda.synchronize()
    assert torch.equal(out, want) and not torch.equal(out, eager)
