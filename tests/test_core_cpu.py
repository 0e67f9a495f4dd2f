"""Host helpers of the drop-in cache module that need no GPU."""

import numpy as np

from oracle import tq_oracle as O
from turboquant_pro_amd import merge_partials


def _state(rng, H, n, D, q):
    k = rng.standard_normal((H, n, D)).astype(np.float32)
    v = rng.standard_normal((H, n, D)).astype(np.float32)
    sc = np.einsum("hd,hsd->hs", q, k) / np.sqrt(D)
    m = sc.max(1)
    e = np.exp(sc - m[:, None])
    return (m, e.sum(1), np.einsum("hs,hsd->hd", e, v)), k, v


def test_merge_partials_is_attention_over_the_union():
    """Merging the states of disjoint key sets equals one softmax over their
    union (the kv_fused.py:139-153 contract), for NumPy and torch inputs."""
    import torch
    rng = np.random.default_rng(0)
    H, D = 4, 64
    q = rng.standard_normal((H, D)).astype(np.float32)
    parts, ks, vs = zip(*(_state(rng, H, n, D, q) for n in (5, 17, 1)))
    K, V = np.concatenate(ks, 1), np.concatenate(vs, 1)
    want = O.attend(q, K, V)
    got = merge_partials(list(parts))
    assert np.allclose(got, want, atol=1e-5)
    assert np.allclose(got, O.merge_partials(list(parts)), atol=1e-6)
    tparts = [tuple(torch.from_numpy(a) for a in p) for p in parts]
    assert np.allclose(merge_partials(tparts).numpy(), want, atol=1e-5)
