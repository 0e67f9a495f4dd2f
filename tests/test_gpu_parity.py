"""GPU parity: the gfx950 kernels against the CPU oracle.

* Encode: packed key/value codes, norms, NF4 scale/mean and the outlier
  side-list are bit-exact (every group, every head), including chunked appends
  that read tokens back from the hot ring, page_tokens=16 with a permuted
  block table, small groups, V4 and magnitude ties.
* Decode: the fused split-K output matches dequantize-then-attend within
  max-abs 2e-3 and relative 1e-2 (MHA, GQA 4 and 8, batch > 1, hot-only,
  exactly-at-flush lengths, ragged batches).
"""

import numpy as np
import pytest

from gpu_util import assert_attn_close, compare_group, oracle_state
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


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _fill(pool, k, v, chunks=None, n_new=None):
    if chunks is None:
        pool.append(_dev(k), _dev(v), n_new=n_new)
        return
    t = 0
    for c in chunks:
        pool.append(_dev(k[:, :, t:t + c]), _dev(v[:, :, t:t + c]))
        t += c
    assert t == k.shape[2]


def _check_codes(pool, seqs, B):
    for b in range(B):
        sc = seqs[b]
        assert pool.n_groups(b) == len(sc.keys)
        for g, (kg, vg) in enumerate(zip(sc.keys, sc.values)):
            compare_group(pool.export_group(b, g), kg, vg, what=f"seq {b} group {g}")
        hk, hv = pool.hot_window_tokens(b)
        assert np.array_equal(hk.cpu().numpy(), sc.hot_k)
        assert np.array_equal(hv.cpu().numpy(), sc.hot_v)


@pytest.mark.parametrize("vbits", [3, 4])
def test_encode_bit_exact_bulk(vbits):
    B, Hkv, L = 2, 2, 1100
    print(f"[encode bulk] vbits={vbits} B={B} Hkv={Hkv} L={L}", flush=True)
    k, v, _ = O.synthetic_kv(11 + vbits, B, Hkv, Hkv, L)
    seqs, rot = oracle_state(k, v, 512, vbits, seed=0)
    pool = _pool(n_kv_heads=Hkv, max_batch=B, max_seq_len=L, value_bits=vbits, rotation=rot)
    _fill(pool, k, v)
    _check_codes(pool, seqs, B)


def test_encode_bit_exact_chunked_appends():
    B, Hkv, L = 1, 2, 1400
    print("[encode chunked] L=1400 chunks 1/7/300/513/...", flush=True)
    k, v, _ = O.synthetic_kv(21, B, Hkv, Hkv, L)
    seqs, rot = oracle_state(k, v, 512, 3, seed=3)
    pool = _pool(n_kv_heads=Hkv, max_batch=B, max_seq_len=L, rotation=rot)
    chunks = [1, 7, 300, 205, 1, 256, 255, 257, 118]
    _fill(pool, k, v, chunks=chunks)
    _check_codes(pool, seqs, B)


def test_encode_paged_permuted_block_table():
    B, Hkv, L = 3, 2, 1300
    print("[encode paged] P=16 permuted block table", flush=True)
    k, v, _ = O.synthetic_kv(31, B, Hkv, Hkv, L)
    seqs, rot = oracle_state(k, v, 512, 3, seed=4)
    from turboquant_pro_amd.codebooks import n_groups_for
    max_pages = n_groups_for(L, 512) * 256 // 16
    bt = np.random.default_rng(7).permutation(B * max_pages).astype(np.int32)
    pool = _pool(n_kv_heads=Hkv, max_batch=B, max_seq_len=L, rotation=rot, page_tokens=16,
                 block_table=bt)
    _fill(pool, k, v)
    _check_codes(pool, seqs, B)


def test_encode_small_window_v4_and_ties():
    """hot_window=16 (groups of 8 tokens), V4, and coarse keys with many |x| ties."""
    B, Hkv, L = 1, 2, 150
    print("[encode small window + ties]", flush=True)
    k, v, _ = O.synthetic_kv(41, B, Hkv, Hkv, L)
    k = (np.round(k.astype(np.float32) * 2) / 2).astype(np.float16)
    k[0, 1, :, 5] = 0.0
    seqs, rot = oracle_state(k, v, 16, 4, seed=5)
    pool = _pool(n_kv_heads=Hkv, max_batch=B, max_seq_len=L, hot_window=16, value_bits=4,
                 rotation=rot, outlier_cap=8 * 128)
    _fill(pool, k, v, chunks=[3, 40, 1, 100, 6])
    _check_codes(pool, seqs, B)


def test_dequant_groups_bit_exact():
    B, Hkv, L = 1, 2, 1030
    k, v, _ = O.synthetic_kv(51, B, Hkv, Hkv, L)
    seqs, rot = oracle_state(k, v, 512, 3, seed=6)
    pool = _pool(n_kv_heads=Hkv, max_batch=B, max_seq_len=L, rotation=rot)
    _fill(pool, k, v)
    kout, vout = pool.dequant_groups([(0, g) for g in range(pool.n_groups(0))])
    cent, _ = O.polar_codebook(3, 128)
    for g in range(pool.n_groups(0)):
        assert np.array_equal(kout[g].cpu().numpy(), O.decode_keys(seqs[0].keys[g]))
        assert np.array_equal(vout[g].cpu().numpy(), O.decode_values(seqs[0].values[g], cent, rot[0]))


DECODE_CASES = [
    # (B, Hkv, Hq, L, vbits, hot_window, page_tokens)
    (1, 4, 4, 1100, 4, 512, None),     # MHA, V4 (robust-style)
    (2, 2, 8, 1300, 3, 512, None),     # GQA 4, K4/V3
    (1, 2, 16, 2100, 3, 512, None),    # GQA 8
    (2, 2, 4, 300, 3, 512, None),      # hot window only
    (1, 2, 8, 513, 3, 512, None),      # exactly one flush
    (3, 2, 8, 1537, 3, 512, 16),       # paged 16-token pages
    (1, 2, 2, 90, 3, 16, None),        # small window: groups of 8 (per-token value rows)
    (1, 2, 8, 200, 3, 64, None),       # groups of 32 (one block), hot ring of 64
    (2, 2, 4, 777, 3, 512, 32),        # 32-token pages, partial hot block
    (1, 8, 8, 1500, 3, 512, None),     # MHA with V3
    # query heads per kv head that are not powers of two (padded heads in the
    # kernel): 3, 5, and 7 (Qwen2.5-7B's 28 / 4), on both decode kernels
    (1, 2, 6, 900, 3, 512, None),
    (2, 2, 10, 1100, 3, 512, 32),
    (1, 4, 28, 1300, 3, 512, None),
    (1, 2, 14, 90, 3, 16, None),
    (1, 2, 6, 200, 4, 64, None),
    # other page sizes: 64- and 256-token pages (a page per group), and
    # 8-token pages (not a whole MFMA tile: the VALU kernel)
    (2, 2, 8, 1300, 3, 512, 64),
    (1, 2, 8, 1300, 3, 512, 256),
    (1, 2, 8, 900, 3, 512, 8),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=[str(c) for c in DECODE_CASES])
def test_decode_matches_dequant_then_attend(case):
    B, Hkv, Hq, L, vbits, W, P = case
    print(f"[decode] {case}", flush=True)
    k, v, q = O.synthetic_kv(61 + L, B, Hkv, Hq, L)
    seqs, rot = oracle_state(k, v, W, vbits, seed=7)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, hot_window=W,
                 value_bits=vbits, rotation=rot, page_tokens=P)
    _fill(pool, k, v)
    if P not in (None, 16, 32):
        # page sizes the encode tests do not cover: its codes too, bit for bit
        _check_codes(pool, seqs, B)
    got = pool.decode(_dev(q)).cpu().numpy()
    for b in range(B):
        assert_attn_close(got[b], seqs[b].attend(q[b]), what=f"case {case} seq {b}")


def test_decode_ragged_batch():
    B, Hkv, Hq, T = 4, 2, 8, 1500
    lens = [1500, 700, 513, 40]
    print(f"[decode ragged] lens={lens}", flush=True)
    k, v, q = O.synthetic_kv(71, B, Hkv, Hq, T)
    pi, pi_t = O.rotation(8, 128)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=T, rotation=(pi, pi_t),
                 page_tokens=16)
    _fill(pool, k, v, n_new=lens)
    got = pool.decode(_dev(q)).cpu().numpy()
    for b, L in enumerate(lens):
        sc = O.SequenceCache(hot_window=512, value_bits=3, outlier_frac=0.02).build(
            k[b, :, :L], v[b, :, :L], pi, pi_t)
        assert_attn_close(got[b], sc.attend(q[b]), what=f"ragged seq {b} L={L}")


def test_decode_edge_lengths():
    """One batch with sequences of 1, 2, 31, 32, 33, 511, 512, 513, 768, 769,
    1024 and 1025 tokens: hot-only windows of one token, whole and partial
    32-token hot blocks, exactly at the first flush and one past it, and
    one token either side of the next group boundaries; GQA 4 on the MFMA
    kernel, whose item order is reranked for batches (longest first)."""
    lens = [1, 2, 31, 32, 33, 511, 512, 513, 768, 769, 1024, 1025]
    B, Hkv, Hq, T = len(lens), 2, 8, max(lens)
    print(f"[decode edge lengths] lens={lens}", flush=True)
    k, v, q = O.synthetic_kv(73, B, Hkv, Hq, T)
    pi, pi_t = O.rotation(9, 128)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=T, rotation=(pi, pi_t))
    _fill(pool, k, v, n_new=lens)
    got = pool.decode(_dev(q)).cpu().numpy()
    for b, L in enumerate(lens):
        sc = O.SequenceCache(hot_window=512, value_bits=3, outlier_frac=0.02).build(
            k[b, :, :L], v[b, :, :L], pi, pi_t)
        assert_attn_close(got[b], sc.attend(q[b]), what=f"seq {b} L={L}")


def test_decode_partials_merge():
    B, Hkv, Hq, L = 1, 2, 8, 1200
    k, v, q = O.synthetic_kv(81, B, Hkv, Hq, L)
    seqs, rot = oracle_state(k, v, 512, 3, seed=9)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, rotation=rot)
    _fill(pool, k, v)
    m, l_, acc = pool.decode_partials(_dev(q))
    out = (acc / l_[..., None]).cpu().numpy()
    assert_attn_close(out[0], seqs[0].attend(q[0]))
    # merging the cache's state with an extra (m, l, acc) part equals the
    # single-pass result over the union (turboquant_pro/kv_fused.py:139-153)
    ek = np.random.default_rng(1).standard_normal((Hq, 5, 128)).astype(np.float32)
    ev = np.random.default_rng(2).standard_normal((Hq, 5, 128)).astype(np.float32)
    qf = q[0].astype(np.float32)
    sc = np.einsum("hd,hsd->hs", qf, ek) / np.sqrt(128)
    mx = sc.max(1)
    e = np.exp(sc - mx[:, None])
    extra = (mx, e.sum(1), np.einsum("hs,hsd->hd", e, ev))
    merged = O.merge_partials([(m[0].cpu().numpy(), l_[0].cpu().numpy(), acc[0].cpu().numpy()), extra])
    K = np.concatenate([np.repeat(seqs[0].get_keys(), Hq // Hkv, 0), ek], 1)
    V = np.concatenate([np.repeat(seqs[0].get_values(), Hq // Hkv, 0), ev], 1)
    p = O.softmax_rows(np.einsum("hd,hsd->hs", qf, K) / np.sqrt(128))
    assert_attn_close(merged, np.einsum("hs,hsd->hd", p, V))


def test_golden_fixture_k4v3(golden_dir):
    """The reference's own cache (AutoConfig 'balanced' build_cache, seed 0)."""
    import os
    g = np.load(os.path.join(golden_dir, "cache_k4v3_w512.npz"))
    k, v, q = g["k"], g["v"], g["q"]
    H, L, D = k.shape
    from turboquant_pro_amd.codebooks import random_rotation
    pool = _pool(n_kv_heads=H, max_batch=1, max_seq_len=L, seed=0)
    _fill(pool, k[None], v[None])
    assert pool.n_groups(0) == int(g["n_groups"])
    for i in range(int(g["n_groups"])):
        e = pool.export_group(0, i)
        assert np.array_equal(e["kpacked"], g[f"g{i}_kpacked"])
        assert np.array_equal(e["nf4_scale"], g[f"g{i}_nf4_scale"])
        assert np.array_equal(e["nf4_mean"], g[f"g{i}_nf4_mean"])
        assert np.array_equal(e["outlier_idx"], g[f"g{i}_oidx"])
        assert np.array_equal(e["outlier_val"].view(np.uint16), g[f"g{i}_oval"].view(np.uint16))
        assert np.array_equal(e["vpacked"], g[f"g{i}_vpacked"])
        assert np.array_equal(e["vnorms"], g[f"g{i}_vnorms"])
    got = pool.decode(_dev(q[None])).cpu().numpy()[0]
    assert_attn_close(got, g["attn_out"])
    del random_rotation


@pytest.mark.parametrize("frac", [0.025, 0.03, 0.1, 0.3])
def test_decode_heavy_outliers(frac):
    """Heavy side-lists (turboquant_pro tests/test_kv_fused_pck.py:99-103): at
    10 % and 30 % outliers a 32-token block holds ~400 and ~1200 entries, so
    the decode applies them in several 128-entry passes.  Codes and side-lists
    stay bit-exact; the output stays within the bar of dequantize-then-attend.
    2.5 % and 3 % give k = 6 and 8 outliers per channel of a 256-token group,
    the encode's longer top-k lists (its bitwise search takes k > 8)."""
    B, Hkv, Hq, L = 1, 2, 8, 1100
    print(f"[decode heavy outliers] frac={frac}", flush=True)
    k, v, q = O.synthetic_kv(83, B, Hkv, Hq, L)
    seqs, rot = oracle_state(k, v, 512, 3, seed=4, outlier_frac=frac)
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, rotation=rot,
                 outlier_frac=frac)
    _fill(pool, k, v)
    _check_codes(pool, seqs, B)
    got = pool.decode(_dev(q)).cpu().numpy()
    assert_attn_close(got[0], seqs[0].attend(q[0]), what=f"frac={frac}")


@pytest.mark.parametrize("hq", [8, 16])
def test_decode_token_outliers_span_lanes(hq):
    """A few tokens per group large in every channel: each is an outlier in
    all 128 channels, so its run of side-list entries is longer than two of
    the correction pass's per-lane shares (E = ceil(n / 64) entries each) and
    covers three or more lanes: the pass's cross-lane scan, which the usual
    spread of outliers never needs, joins the run.  GQA 4 (256-token
    segments) and 8 (128-token segments); codes bit-exact, decode within the
    bar."""
    B, Hkv, L = 1, 2, 1100
    print(f"[decode token outliers span lanes] hq={hq}", flush=True)
    k, v, q = O.synthetic_kv(91, B, Hkv, hq, L)
    rng = np.random.default_rng(5)
    spikes = np.sort(rng.choice(768, size=12, replace=False))
    k = k.astype(np.float32)
    k[:, :, spikes, :] *= 6.0
    k = k.astype(np.float16)
    seqs, rot = oracle_state(k, v, 512, 3, seed=4, outlier_frac=0.02)
    # the property the test is about: some segment holds a token with more
    # than 2 E entries
    seg = 256 if hq // Hkv <= 4 else 128
    longest = 0
    for kg in seqs[0].keys:
        idx = np.asarray(kg.outlier_idx, np.int64)
        h_s = idx // 128                      # (head, token) of each entry
        for h in range(Hkv):
            tok = h_s[(h_s // 256) == h] % 256
            for s0 in range(0, 256, seg):
                run = tok[(tok >= s0) & (tok < s0 + seg)]
                if run.size:
                    e = -(-run.size // 64)
                    longest = max(longest, int(np.bincount(run - s0).max()) / e)
    assert longest > 2, f"no token covers three lanes (longest run {longest:.1f} E)"
    pool = _pool(n_kv_heads=Hkv, n_q_heads=hq, max_batch=B, max_seq_len=L, rotation=rot)
    _fill(pool, k, v)
    _check_codes(pool, seqs, B)
    got = pool.decode(_dev(q)).cpu().numpy()
    assert_attn_close(got[0], seqs[0].attend(q[0]), what=f"hq={hq}")


@pytest.mark.parametrize("vbits", [3, 4])
def test_uniform_keys_encode_dequant_decode(vbits):
    """Uniform per-channel keys (turboquant_pro/per_channel_kv.py:303-317,
    529-530) through the same pool and kernels: the encode's codes, scale,
    zero and side-list are bit-exact to the oracle (itself pinned to the
    reference's vectors), the GPU dequant is bit-exact to the reference's
    decompress order, and the fused decode (levels 0..15 in the code table)
    is within the bar of dequantize-then-attend."""
    B, Hkv, Hq, L = 2, 2, 8, 1300
    print(f"[uniform keys] vbits={vbits}", flush=True)
    k, v, q = O.synthetic_kv(87 + vbits, B, Hkv, Hq, L)
    pi, pi_t = O.rotation(2, 128)
    seqs = [O.SequenceCache(hot_window=512, value_bits=vbits, outlier_frac=0.02, key_grid="uniform")
            .build(k[b], v[b], pi, pi_t) for b in range(B)]
    pool = _pool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, rotation=(pi, pi_t),
                 value_bits=vbits, key_grid="uniform")
    _fill(pool, k, v, chunks=[700, 1, 599])
    _check_codes(pool, seqs, B)
    kk, _ = pool.dequant_groups([(0, g) for g in range(pool.n_groups(0))])
    for g in range(pool.n_groups(0)):
        assert np.array_equal(kk[g].cpu().numpy(), O.decode_keys(seqs[0].keys[g]))
    got = pool.decode(_dev(q)).cpu().numpy()
    for b in range(B):
        assert_attn_close(got[b], seqs[b].attend(q[b]), what=f"uniform seq {b}")
