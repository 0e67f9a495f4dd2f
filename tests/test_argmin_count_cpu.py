"""The group encode's counting argmin, restated in NumPy fp32 and checked
against ``np.argmin`` (the reference's nearest-level rule,
turboquant_pro/per_channel_kv.py:377-383): for sorted NF4 levels whose every
gap is at least (|mean| + amax) * 2^-18 -- 16 ulps of the largest distance a
token of the group can have -- the first argmin of |x - c_l| equals the
number of strict decreases d_l < d_(l-1).  Inputs: random channels over many
scales and offsets, tokens at the levels, at fp32 midpoints between them and
at their neighbours, and channels that fail the gap test (for which the
kernel keeps the compare-and-select argmin) are counted to show the test
reaches both sides of the bound."""

import numpy as np

from oracle import tq_oracle as O

NF4 = O.NF4.astype(np.float32)


def levels(mu, amax):
    return (np.float32(mu) + np.float32(amax) * NF4).astype(np.float32)


def spread(mu, amax, c):
    bound = np.float32((np.float32(abs(mu)) + np.float32(amax)) * np.float32(2.0 ** -18))
    return bool(np.all(np.diff(c) >= bound)) and bool(np.all(np.isfinite(c)))


def count_argmin(x, c):
    d = np.abs(x[:, None] - c[None, :])                  # fp32, |fl(x - c_l)|
    return (d[:, 1:] < d[:, :-1]).sum(axis=1)


def test_counting_argmin_equals_first_argmin():
    rng = np.random.default_rng(0)
    n_spread = n_crowded = 0
    for _ in range(4000):
        scale = np.float32(10.0 ** rng.uniform(-6, 4))
        mu = np.float32(rng.choice([0.0, 1.0, -1.0]) * 10.0 ** rng.uniform(-3, 4.8))
        amax = np.float32(max(scale * rng.uniform(0.5, 3.0), 1e-8))
        c = levels(mu, amax)
        if not spread(mu, amax, c):
            n_crowded += 1
            continue
        n_spread += 1
        # tokens of the group: |x - mu| <= amax, as fp16 inputs in the encode
        x = (mu + amax * rng.uniform(-1, 1, 64)).astype(np.float16).astype(np.float32)
        x = x[np.abs(x - mu) <= amax]
        mids = ((c[:-1] + c[1:]) / np.float32(2.0)).astype(np.float32)
        near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
                               c, np.nextafter(c, np.float32(np.inf)), np.nextafter(c, np.float32(-np.inf))])
        near = near[np.abs(near - mu) <= amax]
        xs = np.concatenate([x, mids, near]).astype(np.float32)
        want = np.argmin(np.abs(xs[:, None] - c[None, :]), axis=1)
        assert np.array_equal(count_argmin(xs, c), want), (mu, amax)
    assert n_spread > 1000 and n_crowded > 100, (n_spread, n_crowded)


def test_crowded_levels_need_the_select():
    """With a large mean and a tiny amax the levels collapse in fp32 and the
    count would disagree with the first argmin -- why the gap test exists."""
    mu, amax = np.float32(3.0e4), np.float32(1e-3)
    c = levels(mu, amax)
    assert not spread(mu, amax, c)
    xs = np.array([mu - 2e-3, mu, mu + 2e-3], np.float32)
    want = np.argmin(np.abs(xs[:, None] - c[None, :]), axis=1)
    assert not np.array_equal(count_argmin(xs, c), want)
