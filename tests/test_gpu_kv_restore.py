"""The connector's live load path: a request's saved prefix goes back into the
gfx950 paged pool as codes (the reference's ``start_load_kv`` is a no-op,
turboquant_pro/connectors/vllm_v1.py:773-775).

Two requests (1100 and 700 tokens, GQA 8:2) are appended to a pool, saved
through ``save_kv_layer`` in the pool's group cadence, and restored with
``start_load_kv`` into the two slots of a fresh pool.  Every coded group of
the restored pool is bit-identical to the original's (imported as codes,
including the MFMA-tiled value order, no re-encode) and so is the hot window
(kept as fp16): the restored pool decodes exactly as the original does, and
within the north-star bar of dequantize-then-attend over its own contents;
after the same further appends both pools hold the same codes and decode
alike.  The scheduler side reports the stored tokens and a finished request
is evicted.  A pool of another key grid refuses the records.
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


def _pool():
    from turboquant_pro_amd import TQKVPool
    return TQKVPool(n_kv_heads=2, n_q_heads=8, max_batch=2, max_seq_len=2048, value_bits=3, seed=0)


def _dense(pool, b):
    """fp32 (H, L, D) keys and values of sequence b: coded groups through the
    GPU dequant, then the hot window."""
    ng, G = pool.n_groups(b), pool.group_tokens
    parts_k, parts_v = [], []
    if ng:
        kk, vv = pool.dequant_groups([(b, g) for g in range(ng)])
        H, D = pool.n_kv_heads, pool.head_dim
        parts_k.append(kk.permute(1, 0, 2, 3).reshape(H, ng * G, D))
        parts_v.append(vv.permute(1, 0, 2, 3).reshape(H, ng * G, D))
    hk, hv = pool.hot_window_tokens(b)
    parts_k.append(hk.float())
    parts_v.append(hv.float())
    return torch.cat(parts_k, 1), torch.cat(parts_v, 1)


def _attend(q, k, v):
    """q (Hq, D) over k, v (Hkv, L, D), fp32 softmax attention."""
    g = q.shape[0] // k.shape[0]
    kk, vv = k.repeat_interleave(g, 0), v.repeat_interleave(g, 0)
    s = torch.einsum("hd,hld->hl", q.float(), kk) / 128 ** 0.5
    return torch.einsum("hl,hld->hd", torch.softmax(s, -1), vv)


def _check_decode(pool, q):
    out = pool.decode(q)
    for b in range(2):
        k, v = _dense(pool, b)
        assert_attn_close(out[b].cpu().numpy(), _attend(q[b], k, v).cpu().numpy(), what=f"seq {b}")


def test_start_load_kv_restores_codes():
    from turboquant_pro_amd.connectors import TurboQuantKVConnector
    lens = [1100, 700]
    print(f"[restore] lens={lens}", flush=True)
    k, v, q = O.synthetic_kv(55, 2, 2, 8, 1400)
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    src = _pool()
    src.append(kd[:, :, :1100], vd[:, :, :1100], n_new=lens)
    conn = TurboQuantKVConnector()
    conn.bind_pool("layers.0.attn", src)
    for rid, b, L in (("reqA", 0, 1100), ("reqB", 1, 700)):
        conn.save_kv_layer("layers.0.attn", (kd[b, :, :L], vd[b, :, :L]), request_id=rid)
    assert conn.get_num_new_matched_tokens(type("R", (), {"request_id": "reqA"})(), 0) == (1100, False)
    assert conn.get_num_new_matched_tokens(type("R", (), {"request_id": "reqB"})(), 300) == (400, False)
    dst = _pool()
    conn.bind_pool("layers.0.attn", dst)
    # vLLM's flow: the scheduler-side instance takes the allocations of the
    # requests that load and hands them over as connector metadata; the
    # worker is bound to it and restores each request into its slot
    from turboquant_pro_amd.connectors.vllm import KVConnectorRole
    sched = TurboQuantKVConnector(role=KVConnectorRole.SCHEDULER, store=conn.store)
    for rid in ("reqA", "reqB", "missing"):
        req = type("R", (), {"request_id": rid})()
        n, _ = sched.get_num_new_matched_tokens(req, 0)
        sched.update_state_after_alloc(req, [], n)
    meta = sched.build_connector_meta()
    assert meta.loads == [("reqA", 0, 1100), ("reqB", 1, 700)]
    conn.bind_connector_metadata(meta)
    assert conn.start_load_kv(None) == 1800
    conn.clear_connector_metadata()
    assert conn.get_metrics()["hits"] >= 2
    assert dst.lengths == lens
    for b in range(2):
        assert dst.n_groups(b) == src.n_groups(b)
        for g in range(src.n_groups(b)):
            a, c = src.export_group(b, g), dst.export_group(b, g)
            for key in a:
                assert np.array_equal(np.asarray(a[key]), np.asarray(c[key])), f"seq {b} group {g} {key}"
        for x_s, x_d in zip(src.hot_window_tokens(b), dst.hot_window_tokens(b)):
            assert torch.equal(x_s, x_d)                                      # kept as fp16
    assert torch.equal(dst.decode(qd), src.decode(qd))
    _check_decode(dst, qd)
    # decoding continues on the restored pool: more tokens, a flush in each
    # sequence, the same codes as the original pool gets from the same tokens
    dst.append(kd[:, :, 1100:1400], vd[:, :, 1100:1400], n_new=[300, 300])
    src.append(kd[:, :, 1100:1400], vd[:, :, 1100:1400], n_new=[300, 300])
    assert dst.n_groups(0) == src.n_groups(0) and dst.n_groups(1) == src.n_groups(1)
    for b in range(2):
        for g in range(src.n_groups(b)):
            a, c = src.export_group(b, g), dst.export_group(b, g)
            for key in ("kpacked", "vpacked", "vnorms", "outlier_idx"):
                assert np.array_equal(np.asarray(a[key]), np.asarray(c[key])), f"seq {b} group {g} {key}"
    assert torch.equal(dst.decode(qd), src.decode(qd))
    _check_decode(dst, qd)
    # a pool of another key grid refuses the records
    from turboquant_pro_amd import TQKVPool
    uni = TQKVPool(n_kv_heads=2, n_q_heads=8, max_batch=2, max_seq_len=2048, value_bits=3, seed=0,
                   key_grid="uniform")
    with pytest.raises(ValueError, match="asym-NF4"):
        conn.store.load_into_pool("reqA", "layers.0.attn", uni, 0)
    conn.get_finished({"reqA"})
    assert conn.store.matched_tokens("reqA") == 0 and conn.store.matched_tokens("reqB") == 700


def test_bias_zero_point_groups_restore_with_their_positions():
    """Keys with the RoPE-averaged ``bias`` zero point (per_channel_kv.py:
    245-267): each group's zero point depends on its first position, so the
    live-path save records group g at position g * G; restored into a pool of
    the same rope_theta and k_bias, every group is bit-identical to the pool
    that encoded the tokens itself.  A pool with another rope_theta refuses
    the records (its zero points would be another function)."""
    from turboquant_pro_amd import TQKVPool
    from turboquant_pro_amd.connectors import TurboQuantBlockStore
    print("[restore] bias zero point", flush=True)
    k, v, q = O.synthetic_kv(57, 1, 2, 8, 1100)
    kbias = np.random.default_rng(3).standard_normal((2, 128)).astype(np.float32)
    kw = dict(n_kv_heads=2, n_q_heads=8, max_batch=1, max_seq_len=2048, value_bits=3, seed=0,
              zero_point="bias", rope_theta=10000.0, k_bias=kbias)
    kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    src = TQKVPool(**kw)
    src.append(kd, vd)
    store = TurboQuantBlockStore(
        key_config={"nf4_asym": True, "outlier_frac": 0.02, "zero_point": "bias",
                    "rope_theta": 10000.0, "k_bias": kbias},
        value_config={"bits": 3, "seed": 0})
    ng = store.save_sequence("r", "l0", kd[0], vd[0], src.group_tokens, src.hot_window)
    assert ng == src.n_groups(0) == 3
    dst = TQKVPool(**kw)
    assert store.load_into_pool("r", "l0", dst, 0) == 1100
    for g in range(ng):
        a, c = src.export_group(0, g), dst.export_group(0, g)
        for key in a:
            assert np.array_equal(np.asarray(a[key]), np.asarray(c[key])), f"group {g} {key}"
    qd = torch.from_numpy(q).cuda()
    assert torch.equal(dst.decode(qd), src.decode(qd))
    other = TQKVPool(**dict(kw, rope_theta=500000.0))
    with pytest.raises(ValueError, match="rope_theta"):
        store.load_into_pool("r", "l0", other, 0)
    assert store.metrics.to_dict()["misses_incompatible"] == 1
