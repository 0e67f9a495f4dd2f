"""Parity at the BASELINE configurations, at their full sizes.

* config 0 (the reference's CPU-runnable case: robust() K4/V4, MHA 32 heads,
  4096 tokens, seed 0): every group bit-exact against the oracle and the decode
  against the oracle's dequantize-then-attend.
* configs 1-4 (too large for the NumPy oracle as a whole): the GPU encode is
  checked bit-exact against the oracle on sampled groups (first, middle, last;
  several sequences), and the fused decode of every sequence against a torch
  fp32 dequantize-then-attend over the same cache, whose dequantisation is the
  tqk_dequant_groups kernel (bit-exact to the reference's decompress in
  test_gpu_parity.py).  Tolerance: max-abs 2e-3 and relative 1e-2.
"""

import numpy as np
import pytest

from gpu_util import (assert_attn_close, check_groups_vs_oracle, compare_group, oracle_state,
                      ref_attend_gpu, synth_gpu)
from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _pool(**kw):
    from turboquant_pro_amd import TQKVPool
    return TQKVPool(**kw)


def _append_chunks(pool, k, v, lens=None, chunk=4096):
    B, _, T, _ = k.shape
    lens = [T] * B if lens is None else lens
    for t in range(0, T, chunk):
        n = min(chunk, T - t)
        pool.append(k[:, :, t:t + n], v[:, :, t:t + n],
                    n_new=[max(0, min(n, L - t)) for L in lens])


def _decode_vs_reference(pool, q, lens, what, every=1):
    got = pool.decode(q)
    torch.cuda.synchronize()
    for b in range(0, len(lens), every):
        want = ref_attend_gpu(torch, pool, q, b)
        assert_attn_close(got[b].cpu().numpy(), want.cpu().numpy(), what=f"{what} seq {b} L={lens[b]}")


def test_config0_robust_mha_4k_full_oracle():
    """robust(head_dim=128, n_heads=32, hot_window=512), 4096 tokens, seed 0."""
    print("[config0] B1 H32 L4096 V4", flush=True)
    k, v, q = O.synthetic_kv(0, 1, 32, 32, 4096)
    seqs, rot = oracle_state(k, v, 512, 4, seed=0)
    pool = _pool(n_kv_heads=32, max_batch=1, max_seq_len=4096, value_bits=4, rotation=rot)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    sc = seqs[0]
    assert pool.n_groups(0) == len(sc.keys) == 14
    for g, (kg, vg) in enumerate(zip(sc.keys, sc.values)):
        compare_group(pool.export_group(0, g), kg, vg, what=f"config0 group {g}")
    got = pool.decode(torch.from_numpy(q).cuda()).cpu().numpy()[0]
    assert_attn_close(got, sc.attend(q[0]), what="config0")


def test_config1_gqa_b16_8k():
    """B16, 32 q-heads / 8 kv-heads, 8192 tokens, K4/V3."""
    print("[config1] B16 Hkv8 Hq32 L8192", flush=True)
    B, Hkv, Hq, L = 16, 8, 32, 8192
    k, v = synth_gpu(torch, 1, B, Hkv, L)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, seed=0)
    _append_chunks(pool, k, v)
    ng = pool.n_groups(0)
    assert ng == O.n_groups(L, 512)
    pi_t = pool.pi_t.cpu().numpy()
    for b in (0, 9, 15):
        check_groups_vs_oracle(pool, k, v, b, (0, ng // 2, ng - 1), pi_t, 3, what="config1")
    q = torch.randn((B, Hq, 128), generator=torch.Generator(device="cuda").manual_seed(11),
                    device="cuda").half()
    _decode_vs_reference(pool, q, [L] * B, "config1")


def test_config2_long_context_128k():
    """B1, 131072 tokens, 32 q-heads / 8 kv-heads (many splits per sequence)."""
    print("[config2] B1 Hkv8 Hq32 L131072", flush=True)
    B, Hkv, Hq, L = 1, 8, 32, 131072
    k, v = synth_gpu(torch, 2, B, Hkv, L)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, seed=0)
    _append_chunks(pool, k, v)
    ng = pool.n_groups(0)
    assert ng == O.n_groups(L, 512) == 510
    check_groups_vs_oracle(pool, k, v, 0, (0, 1, 255, ng - 1), pool.pi_t.cpu().numpy(), 3,
                           what="config2")
    q = torch.randn((B, Hq, 128), generator=torch.Generator(device="cuda").manual_seed(12),
                    device="cuda").half()
    _decode_vs_reference(pool, q, [L], "config2")


def test_config3_paged_ragged_b64():
    """B64, lengths ~ U[1024, 32768] (seeded), 16-token pages, block table a
    seeded permutation of the physical pages, 32 q / 8 kv heads, K4/V3."""
    print("[config3] B64 ragged P16 permuted pages", flush=True)
    B, Hkv, Hq, T = 64, 8, 32, 32768
    lens = [int(x) for x in np.random.default_rng(3).integers(1024, 32769, size=B)]
    from turboquant_pro_amd.codebooks import n_groups_for
    max_pages = n_groups_for(T, 512) * 256 // 16
    bt = np.random.default_rng(4).permutation(B * max_pages).astype(np.int32)
    k, v = synth_gpu(torch, 3, B, Hkv, T)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=T, seed=0,
                 page_tokens=16, block_table=bt)
    _append_chunks(pool, k, v, lens=lens)
    assert pool.lengths == lens
    pi_t = pool.pi_t.cpu().numpy()
    for b in (0, 17, 63):
        ng = pool.n_groups(b)
        check_groups_vs_oracle(pool, k, v, b, sorted({0, ng // 2, ng - 1}), pi_t, 3, what="config3")
    q = torch.randn((B, Hq, 128), generator=torch.Generator(device="cuda").manual_seed(13),
                    device="cuda").half()
    _decode_vs_reference(pool, q, lens, "config3")


def test_config4_70b_append_chunks_and_decode():
    """B32, 64 q-heads / 8 kv-heads (GQA 8), prefill appended in 4096-token
    chunks up to 32768, then one decode step."""
    print("[config4] B32 Hkv8 Hq64 L32768 in 4096 chunks", flush=True)
    B, Hkv, Hq, L = 32, 8, 64, 32768
    k, v = synth_gpu(torch, 4, B, Hkv, L)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, seed=0)
    _append_chunks(pool, k, v, chunk=4096)
    ng = pool.n_groups(0)
    pi_t = pool.pi_t.cpu().numpy()
    # groups that straddle chunk boundaries read tokens back from the hot ring
    for b in (0, 31):
        check_groups_vs_oracle(pool, k, v, b, (0, 15, 16, ng - 1), pi_t, 3, what="config4")
    q = torch.randn((B, Hq, 128), generator=torch.Generator(device="cuda").manual_seed(14),
                    device="cuda").half()
    _decode_vs_reference(pool, q, [L] * B, "config4", every=3)


def test_headline_timed_shape_b16_32k():
    """The shape bench.py times (its "headline" config): B16 x 32768 tokens,
    32 q-heads / 8 kv-heads, the default pool (32-token pages in the clustered
    block table, K4 asym-NF4 + 2 % outliers, V3, hot window 512), filled in
    4096-token chunks as bench.build_pool fills it, with the measurement
    spec's synthetic data.  Sampled groups bit-exact against the oracle and
    every sequence's decode against the fp32 dequantize-then-attend, on the
    kernel plan the benchmark's number comes from."""
    import bench
    print("[headline] B16 Hkv8 Hq32 L32768, bench pool", flush=True)
    cfg = bench.CONFIGS["headline"]
    B, Hkv, Hq, L = cfg["B"], cfg["Hkv"], cfg["Hq"], cfg["L"]
    k, v = synth_gpu(torch, 5, B, Hkv, L)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, value_bits=cfg["vbits"],
                 seed=1000)
    assert pool.page_tokens == 32 and pool.tiled
    _append_chunks(pool, k, v, chunk=4096)
    ng = pool.n_groups(0)
    assert ng == 126
    pi_t = pool.pi_t.cpu().numpy()
    for b in (0, 7, 15):
        check_groups_vs_oracle(pool, k, v, b, (0, 63, ng - 1), pi_t, 3, what="headline")
    q = torch.randn((B, Hq, 128), generator=torch.Generator(device="cuda").manual_seed(7),
                    device="cuda").half()
    _decode_vs_reference(pool, q, [L] * B, "headline")
